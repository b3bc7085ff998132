// Decode attention over the packed KV cache, with the KV pack (append).
//
// One workgroup of 512 threads per query head: it prepares the head's query
// (q-norm factor on its 1/65536 grid, RoPE, q16), scores every position
// 0..pos (exact integer dot products, 1/1024 grid), forms the (max, sum)
// statistics on their q16 grids and the weighted V sum.  In a launch that also
// appends, the first query head of each KV head's group packs this position's
// K (qk-norm, RoPE) and V into the layer's KV row, and every head of the group
// rebuilds the same packed values in LDS for its own position.  Scores and
// exponentials run one position per thread (or per lpp lanes); the K row of a
// position is read as 16-byte vectors.  The weighted V sum runs a wave per
// chunk of positions and a lane per element (or two), with the V values read
// straight into registers.  The two double-precision sums (sum of
// exp, sum over t of p*v) use a fixed order -- chunks of kChunk positions,
// each summed in position order, then the chunk sums in chunk order -- and the
// oracle sums in the same order, so the output is reproducible bit for bit.
//
// HBM layout of a layer's cache: head-major planes, K of KV head 0, 1, ...
// then V of KV head 0, 1, ..., each seq positions x head_dim values, int16
// little-endian (kv_bits 16, grid 1/2048) or int8 (kv_bits 8, grid 1/16).  A
// head's prefix 0..pos is one contiguous run (the reference's interleaved
// [K kv_dim | V kv_dim] texel rows put each head's 96- to 512-byte slice in a
// different part of a row, so a head's reads straddled cache lines).
// vgx_kv_read_rows / write_rows gather the planes into the reference's texel
// rows (big-endian for q16) and back.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "vgx_internal.h"
#include "vgx_qrow.h"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 512;
constexpr int kChunk = 32;  // positions per chunk of the summation order
constexpr int kVStage = 8;  // 16-byte V pieces a thread stages per round (64 KB a workgroup)
// 16-byte K vectors a lane holds for one scored position (int16 / int8 cache)
template <int KVB>
constexpr int kKPre = KVB == 16 ? 8 : 4;

}  // namespace

struct AttnDev {
    int dim, heads, kv_heads, hd, seq, kv_bits, rope_half, qk_norm, group;
    int row_bytes;  // one position of every head, K and V: the texel row MMKV1 persists
    int pstride;    // bytes of one position in a head's plane (head_dim values)
    int lpp;     // lanes per scored position (a power of two): query-block kernel
    int lpp1;    // the same for the per-head kernel
    // the weighted-V lane plan with one element per lane (vG1 waves per chunk,
    // vC1 chunks per round) and with two (vG2, vC2; taken above head_dim 64
    // when the context needs more than one round of the first)
    int vG1, vC1, vG2, vC2;
    int nchmax;  // chunks of a full cache
    // LDS byte offsets
    int o_wmax, o_vpk, o_kpk, o_qhw, o_qlw, o_sc, o_ep, o_csum, o_vpart, o_acc;
};

struct vgx_attn {
    vgx_ctx* ctx = nullptr;
    AttnDev a{};
    int layers = 0;
    std::vector<uint8_t*> kv;  // per layer, nullptr for a non-attention layer
    int32_t* rtab = nullptr;   // [seq][hd/2][2] cos, sin on the 1/4096 grid
    int16_t* qn = nullptr;     // [layers][hd] q16
    int16_t* kn = nullptr;
    size_t lds = 0;
    int nseq = 1;           // sequences whose caches follow one another in each layer
    size_t seq_bytes = 0;   // one sequence's cache of one layer: seq rows
    bool owner = true;      // false for a view of one sequence (shares every buffer)
};

namespace {


__device__ __forceinline__ float rsqrt_d(float x) { return (float)(1.0 / sqrt((double)x)); }
__device__ __forceinline__ float exp_d(float x) { return (float)exp((double)x); }

template <int KVB>
__device__ __forceinline__ int kv_get(const uint8_t* row, int idx) {
    if (KVB == 16) return (int)reinterpret_cast<const int16_t*>(row)[idx];
    return (int)reinterpret_cast<const int8_t*>(row)[idx];
}

template <int KVB>
__device__ __forceinline__ int kv_enc(float v) {
    const float S = KVB == 16 ? 2048.0f : 16.0f;
    float f = floorf(v * S + 0.5f);
    if (KVB == 16) f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    else f = fminf(fmaxf(f, -128.0f), 127.0f);
    return (int)f;
}

template <int KVB>
__device__ __forceinline__ void kv_put(uint8_t* row, int idx, int q) {
    if (KVB == 16) reinterpret_cast<int16_t*>(row)[idx] = (int16_t)q;
    else reinterpret_cast<int8_t*>(row)[idx] = (int8_t)q;
}

__device__ __forceinline__ void rope_pair(int rope_half, int hd, int i, int& j, int& ti, bool& first) {
    const int half = hd / 2;
    if (rope_half) {
        if (i < half) { j = i + half; ti = i; first = true; }
        else { j = i - half; ti = i - half; first = false; }
    } else {
        const bool even = (i & 1) == 0;
        j = even ? i + 1 : i - 1;
        ti = i / 2;
        first = even;
    }
}

// The inputs of one head vector's norm and rotation for lane l's elements
// i = l + 64c (c < 4): the value, its rotation partner, the norm weights of
// both (with qk_norm) and the table's cos and sin.  Indexes past the head
// are clamped to its last element (those lanes' values are not used).
struct RopeIn {
    int a[4], b[4], na[4], nb[4], co[4], sn[4];
};
__device__ __forceinline__ void rope_load(int rope_half, int qk_norm, int hd, const int16_t* x, const int16_t* nw,
                                          const int32_t* rt, int lane, RopeIn& r) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        r.a[c] = r.b[c] = r.na[c] = r.nb[c] = r.co[c] = r.sn[c] = 0;
        if (64 * c >= hd) continue;  // (uniform) no element of this slot in the head
        const int i = min(lane + 64 * c, hd - 1);
        int j, ti;
        bool first;
        rope_pair(rope_half, hd, i, j, ti, first);
        r.a[c] = x[i];
        r.b[c] = x[j];
        r.na[c] = qk_norm ? nw[i] : 0;
        r.nb[c] = qk_norm ? nw[j] : 0;
        r.co[c] = rt[2 * ti];
        r.sn[c] = rt[2 * ti + 1];
    }
}

typedef short short2_t __attribute__((ext_vector_type(2)));

// A buffer resource over the rows 0 .. nrows-1 of one head's K or V slice
// (base: the slice in row 0).  A buffer load past the resource's byte count
// returns zero and makes no memory access, so the lanes of positions at or
// past npos read nothing and need no branch.  Third-word value: the raw
// 32-bit buffer format of the gfx9 family.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const uint8_t* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, bytes, 0x00020000);
}

// Pins a loaded value into registers at this point.  A select between a
// load and a constant is otherwise lowered to a branch around the load, and a
// load under a branch is waited for before the next one issues.
__device__ __forceinline__ void keep(int& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void keep(uint16_t& x) { asm volatile("" : "+v"(x)); }
// A 16-bit field as loaded, and its signed value.
__device__ __forceinline__ uint16_t u16_at(const int16_t* p, int i) { return reinterpret_cast<const uint16_t*>(p)[i]; }
__device__ __forceinline__ int s16(uint16_t raw) { return (int)(int16_t)raw; }
__device__ __forceinline__ void keep(int4& x) { asm volatile("" : "+v"(x.x), "+v"(x.y), "+v"(x.z), "+v"(x.w)); }

// The query split into bytes for the packed integer dot products: q = 256*qh
// + ql with qh in [-128, 127] and ql in [0, 255].  Word w of qhw / qlw holds
// the elements of K word w: two int16 halves (KVB 16) or four int8 bytes
// (KVB 8, low byte stored as ql - 128).
template <int KVB>
__device__ __forceinline__ void q_split(int q, int i, int* qhw, int* qlw) {
    const int qh = q >> 8, ql = q & 255;
    if (KVB == 16) {
        reinterpret_cast<int16_t*>(qhw)[i] = (int16_t)qh;
        reinterpret_cast<int16_t*>(qlw)[i] = (int16_t)ql;
    } else {
        reinterpret_cast<int8_t*>(qhw)[i] = (int8_t)qh;
        reinterpret_cast<int8_t*>(qlw)[i] = (int8_t)(ql - 128);
    }
}

// Exact partial sums of q . k over one 16-byte vector v of a K row (words
// 4v..4v+3).  KVB 16: sh += sum qh*k, sl += sum ql*k over int16 pairs; for
// head_dim <= 256 neither leaves int32 (|sh| <= 2^7*2^15*2^8 = 2^30, |sl| <=
// 255*2^15*2^8 < 2^31).  KVB 8: sh += sum qh*k, sl += sum (ql-128)*k,
// sk += sum k over int8 quads (each below 2^23).  q . k = 256*sh + sl
// (+ 128*sk for KVB 8).
// a, b: the query's qh and ql words of that vector (zero for a vector past the
// row); ones: 0x01010101 (zero past the row).
template <int KVB>
__device__ __forceinline__ void dot_vec(const int4 a, const int4 b, int ones, const uint4 w, int& sh, int& sl,
                                        int& sk) {
    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
    const int as[4] = {a.x, a.y, a.z, a.w}, bs[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (KVB == 16) {
            sh = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, as[u]), __builtin_bit_cast(short2_t, ws[u]), sh,
                                        false);
            sl = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, bs[u]), __builtin_bit_cast(short2_t, ws[u]), sl,
                                        false);
        } else {
            sh = __builtin_amdgcn_sdot4(as[u], (int)ws[u], sh, false);
            sl = __builtin_amdgcn_sdot4(bs[u], (int)ws[u], sl, false);
            sk = __builtin_amdgcn_sdot4(ones, (int)ws[u], sk, false);
        }
    }
}

// The V values of one chunk for one lane's elements vi (and vi+1 when vE is
// 2), as stored (16- or 8-bit fields, the first element low): position
// c*kChunk + u in vch[u].  vrs covers rows 0..npos-1: a row at or past npos
// reads nothing and gives zero (its weight is zero too); the range check is on
// the per-lane offset, so rows past the cache need no clamp.  An idle wave
// passes a chunk past the cache.  c is wave-uniform: one multiply per chunk,
// then an add per row.
template <int KVB>
__device__ __forceinline__ void v_chunk_load(const AttnDev& A, __amdgpu_buffer_rsrc_t vrs, int vE, int c, int vi,
                                             int (&vch)[kChunk]) {
    const int base = c * kChunk * A.pstride + vi * (KVB / 8);
    if (vE == 2) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const int off = base + u * A.pstride;
            if (KVB == 16) vch[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(vrs, off, 0, 0);
            else vch[u] = (int)__builtin_amdgcn_raw_buffer_load_b16(vrs, off, 0, 0);
        }
    } else {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const int off = base + u * A.pstride;
            if (KVB == 16) vch[u] = (int)__builtin_amdgcn_raw_buffer_load_b16(vrs, off, 0, 0);
            else vch[u] = (int)__builtin_amdgcn_raw_buffer_load_b8(vrs, off, 0, 0);
        }
    }
}
// The pair plan's V loads (head_dim up to 32 fields of 32 bits: 64 at a q16
// cache, 128 at q8): the 32-bit field of elements vi .. vi + 32/KVB - 1 (vi a
// multiple of that) at position c*kChunk + u in vch[u]; rows at or past npos
// read zero, as in v_chunk_load.
template <int KVB>
__device__ __forceinline__ void v_pair_load(const AttnDev& A, __amdgpu_buffer_rsrc_t vrs, int c, int vi,
                                            int (&vch)[kChunk]) {
    const int base = c * kChunk * A.pstride + vi * (KVB / 8);
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
        vch[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(vrs, base + u * A.pstride, 0, 0);
}
// The first and second element of a loaded V field.
template <int KVB>
__device__ __forceinline__ int v_lo(int p) { return KVB == 16 ? (int)(int16_t)(p & 0xffff) : (int)(int8_t)(p & 0xff); }
template <int KVB>
__device__ __forceinline__ int v_hi(int p) { return KVB == 16 ? (p >> 16) : (int)(int8_t)((p >> 8) & 0xff); }

// Lane exchanges within rows of 16 lanes (DPP): quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror.  After the four steps of a
// reduction every lane of a row holds the row's result; the four rows are
// joined through readlane.  Called with every lane of the wave active.
template <int CTRL>
__device__ __forceinline__ int dpp(int x) { return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ double dpp(double x) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = (unsigned)dpp<CTRL>((int)(unsigned)b), hi = (unsigned)dpp<CTRL>((int)(unsigned)(b >> 32));
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double readlane_d(double x, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ int wave_max(int x) {
    x = max(x, dpp<0xB1>(x));
    x = max(x, dpp<0x4E>(x));
    x = max(x, dpp<0x141>(x));
    x = max(x, dpp<0x140>(x));
    return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
// The sum over the wave of integers held in doubles, every partial sum below
// 2^53: exact, so the order of the additions does not matter.
__device__ __forceinline__ double wave_sum_exact(double x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return (readlane_d(x, 0) + readlane_d(x, 16)) + (readlane_d(x, 32) + readlane_d(x, 48));
}

// Compile-time loop: f(integral_constant<int, U>) for U = B .. E-1.
template <int B, int E, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// The weight of position U of a chunk in every lane: lane 16r + n of lo holds
// the weight of position n (of hi: 16 + n) in each row r of 16 lanes, and the
// row broadcast (DPP row_newbcast) gives lane n of each row to the whole row.
template <int U>
__device__ __forceinline__ double chunk_w(double lo, double hi) {
    return __builtin_amdgcn_mov_dpp(U < 16 ? lo : hi, 0x150 + (U & 15), 0xf, 0xf, false);
}

// PAIR: the pair plan below is compiled in (the host sets it for heads of at
// most 32 fields of 32 bits; without it the kernel of a wider head keeps the
// registers and schedule of the one- and two-element plans alone).  KS: the
// K vector slots a scoring lane holds, at least the lane plan's slots per row
// (the host takes 3 or 4 when they fit: each slot is a 16-byte K load, two
// query-word reads from LDS and a dot product, whether or not it lies past
// the row).
template <int KVB, bool PAIR, int KS>
__global__ void __launch_bounds__(kThreads) attn_kernel(const AttnDev A, uint8_t* kv, const int32_t* rtab,
                                                        const int16_t* qn, const int16_t* kn,
                                                        const int16_t* qkv, int16_t* out, int pos0,
                                                        int do_write, int do_attend, size_t seq_stride,
                                                        int pos_step, const int* pos_ptr) {
    extern __shared__ __align__(16) uint8_t smem[];
    // Every kernel argument in scalar registers before the first branch: the
    // argument loads then issue as one batch instead of one round trip at
    // each place of first use.
    // (one statement: a wait for its operands covers the whole batch; two
    // statements were waited for one after the other)
    asm volatile("" ::"s"(kv), "s"(rtab), "s"(qn), "s"(kn), "s"(qkv), "s"(out), "s"(pos0), "s"(do_write),
                 "s"(do_attend), "s"(seq_stride), "s"(pos_step), "s"(pos_ptr), "s"(A.dim), "s"(A.kv_heads),
                 "s"(A.hd), "s"(A.seq), "s"(A.rope_half), "s"(A.qk_norm), "s"(A.group), "s"(A.pstride),
                 "s"(A.lpp1), "s"(A.vG1), "s"(A.vC1), "s"(A.vG2), "s"(A.vC2), "s"(A.nchmax), "s"(A.o_wmax),
                 "s"(A.o_vpk), "s"(A.o_kpk), "s"(A.o_qhw), "s"(A.o_qlw), "s"(A.o_sc), "s"(A.o_ep), "s"(A.o_csum),
                 "s"(A.o_vpart), "s"(A.o_acc));
    constexpr int E = KVB == 16 ? 2 : 4;  // values per 32-bit word
    constexpr int KP = KS;
    const int hd = A.hd, G = A.group, kv_dim = A.kv_heads * hd;
    // An attending launch has one workgroup per query head; a write-only
    // launch one per KV head.  The first query head of a KV head's group packs
    // the KV row; the others rebuild the same values in LDS.
    const int h = do_attend ? (int)blockIdx.x : (int)blockIdx.x * G;
    const int kvh = h / G;
    const bool writer = do_write && h == kvh * G;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // blockIdx.y: the position's offset in a batch of consecutive positions,
    // whose qkv and output rows are consecutive rows
    // (blockIdx.y: a batch of consecutive positions of one sequence, pos_step
    // 1; or the same position of consecutive sequences, each with its own
    // cache seq_stride bytes on, pos_step 0)
    kv += (size_t)blockIdx.y * seq_stride;
    qkv += (size_t)blockIdx.y * (A.dim + 2 * kv_dim);
    if (out) out += (size_t)blockIdx.y * A.dim;
    const int16_t* kq = qkv + A.dim + kvh * hd;           // this group's K (q16)
    const int16_t* vq = qkv + A.dim + kv_dim + kvh * hd;  // and V
    const int16_t* qh = qkv + h * hd;                     // this head's q

    // --- every global read of the launch is issued before any store, so
    // that their latencies overlap.  First the ones that do not depend on the
    // position: this thread's element i = tid of q, K, V with its RoPE partner
    // j, the norm weights, the elements of the sums of squares; they go out
    // ahead of the position's own load (a launch replayed from a graph reads
    // it from device memory, and everything below waits for it).  Then the
    // rotation, the K vectors of this thread's first scored position (lpp
    // lanes per position, vectors sj, sj+lpp, ...) and the V values of its
    // element in its wave's chunk of the first round of the weighted-V pass
    // (below).  The element loads are unconditional, from clamped in-range
    // addresses, and unused values are discarded afterwards (a select between
    // a load and a constant would become a branch whose load is waited for
    // before the next one issues).  The K and V row loads are buffer loads
    // bounded to the rows below npos.
    const bool el = tid < hd;
    const int ie = min(tid, hd - 1);
    int j, ti;
    bool first;
    rope_pair(A.rope_half, hd, ie, j, ti, first);
    const int16_t* knp = A.qk_norm ? kn : kq;
    const int16_t* qnp = A.qk_norm ? qn : qh;
    // (a wave with no element of the head below head_dim issues none of the
    // per-element loads: a wave-uniform branch, so the loads of a wave that
    // does need them still go out back to back)
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const bool welm = wave_u * 64 < hd;
    uint16_t kqr = 0, kqjr = 0, vqr = 0, qhr = 0, qhjr = 0, knr = 0, knjr = 0, qnr = 0, qnjr = 0;
    // the whole head's K and q for the sums of squares, which only the
    // threads of an element use: loaded by those waves alone, 64 elements a
    // load (every vector load of the launch takes the CU's address unit, the
    // unit the loads at the start of the launch queue for)
    // (the values are held as loaded, zero-extended 16-bit fields, and
    // sign-extended where they are first used: a value converted where the
    // branch joins is waited for there, before the loads below issue)
    uint16_t ker[4] = {0, 0, 0, 0}, qer[4] = {0, 0, 0, 0};
    if (welm) {
        kqr = u16_at(kq, ie); kqjr = u16_at(kq, j); vqr = u16_at(vq, ie); qhr = u16_at(qh, ie); qhjr = u16_at(qh, j);
        knr = u16_at(knp, ie); knjr = u16_at(knp, j); qnr = u16_at(qnp, ie); qnjr = u16_at(qnp, j);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (64 * c < hd) {
                const int l = min(lane + 64 * c, hd - 1);
                ker[c] = u16_at(kq, l);
                qer[c] = u16_at(qh, l);
            }
        }
    }
    asm volatile("" ::: "memory");

    // pos_ptr: the position read from device memory (a launch captured once
    // and replayed for every token), clamped into the cache
    const int p0 = pos_ptr ? min(max(*pos_ptr, 0), A.seq - 1) : pos0;
    const int pos = p0 + blockIdx.y * pos_step;
    const int npos = pos + 1;
    const int nch = (npos + kChunk - 1) / kChunk;
    const bool own_row = do_write != 0;  // row pos comes from LDS, not from HBM

    int* wmax = reinterpret_cast<int*>(smem + A.o_wmax);        // kThreads/64
    uint8_t* vpk = smem + A.o_vpk;                              // row pos's packed V slice
    uint8_t* kpk = smem + A.o_kpk;                              // row pos's packed K slice
    int* qhw = reinterpret_cast<int*>(smem + A.o_qhw);          // hd/E words
    int* qlw = reinterpret_cast<int*>(smem + A.o_qlw);          // hd/E words
    int16_t* sc = reinterpret_cast<int16_t*>(smem + A.o_sc);    // seq
    // nchmax*kChunk: the exponentials (+0.0 past npos), then the V weights
    double* ep = reinterpret_cast<double*>(smem + A.o_ep);
    double* csum = reinterpret_cast<double*>(smem + A.o_csum);  // nchmax
    double* vpart = reinterpret_cast<double*>(smem + A.o_vpart);  // vC*hd
    double* acc = reinterpret_cast<double*>(smem + A.o_acc);    // hd

    // this KV head's planes: position t of K at khead + t * pstride
    uint8_t* const khead_w = kv + (size_t)kvh * A.seq * A.pstride;
    uint8_t* const vhead_w = kv + (size_t)(A.kv_heads + kvh) * A.seq * A.pstride;
    const uint8_t* khead = khead_w;
    const uint8_t* vhead = vhead_w;
    const int32_t* rt = rtab + (size_t)pos * (hd / 2) * 2;
    int rc = 0, rs = 0;
    if (welm) {
        rc = rt[2 * ti];
        rs = rt[2 * ti + 1];
    }
    const int nv = hd * KVB / 128;  // 16-byte vectors per K row slice
    const int lpp = A.lpp1, sj = tid & (lpp - 1), P = kThreads / lpp;
    // weighted-V lanes: wave w takes chunk slot w / vG of each round and the
    // elements vE*(64*(w % vG) + lane) .. +vE-1 of the head
    // (slot is wave-uniform; readfirstlane lets the compiler see it)
    const bool wide = A.vC2 > A.vC1 && nch > A.vC1;
    const int vE = wide ? 2 : 1, vG = wide ? A.vG2 : A.vG1, vC = wide ? A.vC2 : A.vC1;
    // pair plan (a head of at most 32 fields of 32 bits -- head_dim 64 at a
    // q16 cache, 128 at q8 -- and more chunks than one round of the
    // one-element plan): every wave takes two chunks of a round, lanes 0..31
    // chunk 2*wave and lanes 32..63 chunk 2*wave + 1, the elements of one
    // 32-bit field a lane, so one load per position serves two chunks: 16
    // chunks a round
    constexpr int EPL = 32 / KVB;  // elements a field
    const bool pair = PAIR && hd <= 32 * EPL && nch > A.vC1;
    const int pe = (lane & 31) * EPL, pvi = min(pe, hd - EPL), pch = 2 * wave + (lane >> 5);
    const int slot = __builtin_amdgcn_readfirstlane(wave / vG);
    const int ve = ((wave - slot * vG) * 64 + lane) * vE, vi = min(ve, hd - vE);
    uint4 kreg[KP];
    int vch[kChunk];  // V of elements vi.. at the chunk's positions, as stored
    // rows 0..npos-1 of this head's K and V slices
    const __amdgpu_buffer_rsrc_t krs = rows_rsrc(khead, npos * A.pstride);
    const __amdgpu_buffer_rsrc_t vrs = rows_rsrc(vhead, npos * A.pstride);
    // vector slots k a lane takes: sj + k*lpp < nv for some lane when k < nk;
    // the slots from nk on are past the row in every lane, and their loads
    // are skipped here (wave-uniform branches)
    const int nk = (nv + lpp - 1) / lpp;
    {
        // only the lanes of a scored position read its K row, and a wave
        // whose first position lies past the context issues no K load
        // (kreg is left unset where nothing is loaded: a wave past the
        // context scores no position, and a slot from nk on meets zero query
        // words and a zero ones word in every lane, so its value adds nothing;
        // set to zero, the value would be copied where the branches join,
        // and the copy would wait for the load)
        const int t = min(tid / lpp, npos);
        if (wave_u * (64 / lpp) < npos) {
#pragma unroll
            for (int k = 0; k < KP; ++k)
                if (k < nk)
                    kreg[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                            krs, t * A.pstride + 16 * min(sj + k * lpp, nv - 1), 0, 0));
        }
    }
    // the K loads first: the scores wait for them, not for the V loads after
    asm volatile("" ::: "memory");
    // a wave whose first-round chunk lies past the context issues no V loads
    // (a wave-uniform branch; such a wave does not read vch in that round):
    // every V load takes the CU's address unit whether it reads memory or not
    if (pair ? 2 * wave_u < nch : (slot < vC && slot < nch)) {
        if (pair) v_pair_load<KVB>(A, vrs, pch, pvi, vch);
        else v_chunk_load<KVB>(A, vrs, vE, slot, vi, vch);
    } else {
#pragma unroll
        for (int u = 0; u < kChunk; ++u) vch[u] = 0;
    }
    // the element values are first used here: without this the compiler
    // moves their conversions up beside the loads, into the element waves'
    // branch, which then waits for those loads before any later load issues
    keep(kqr); keep(kqjr); keep(vqr); keep(qhr); keep(qhjr);
    keep(knr); keep(knjr); keep(qnr); keep(qnjr);
    const int kqi = s16(kqr), kqj = s16(kqjr), vqi = s16(vqr), qhi = s16(qhr), qhj = s16(qhjr);
    const int kni = s16(knr), knj = s16(knjr), qni = s16(qnr), qnj = s16(qnjr);
    int ke[4], qe[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        keep(ker[c]);
        keep(qer[c]);
        ke[c] = s16(ker[c]);
        qe[c] = s16(qer[c]);
    }

    // sums of squares of the K head and the query head (exact integers in
    // doubles, below 2^39), whole in every wave: lane l holds elements l,
    // l+64, l+128, l+192
    double ssk = 0.0, ssq = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const bool in = lane + 64 * c < hd;
        const int kc = in ? ke[c] : 0, qc = in ? qe[c] : 0;
        ssk += (double)(kc * kc);
        ssq += (double)(qc * qc);
    }
    ssk = wave_sum_exact(ssk);
    ssq = wave_sum_exact(ssq);
    keep(rc);  // (as the element values: converted here, not in the branch)
    keep(rs);
    const float co = (float)rc / 4096.0f, sn = (float)rs / 4096.0f;

    // --- KV pack of position pos (att_kv_rope)
    if (do_write && el) {
        float rk = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)ssk * (1.0f / 65536.0f);
            rk = rsqrt_d(ss / (float)hd + 1e-6f);
        }
        float vv = (float)kqi / 256.0f, bb = (float)kqj / 256.0f;
        if (A.qk_norm) {
            vv = (vv * rk) * ((float)kni / 256.0f);
            bb = (bb * rk) * ((float)knj / 256.0f);
        }
        const float o = first ? (vv * co) - (bb * sn) : (bb * sn) + (vv * co);
        const int q = kv_enc<KVB>(o);
        const int qv = kv_enc<KVB>((float)vqi / 256.0f);
        if (writer) {
            kv_put<KVB>(khead_w + (size_t)pos * A.pstride, tid, q);
            kv_put<KVB>(vhead_w + (size_t)pos * A.pstride, tid, qv);
        }
        kv_put<KVB>(kpk, tid, q);
        kv_put<KVB>(vpk, tid, qv);
    }
    if (!do_attend) return;

    // --- q prep (att_qnorm_scale + att_qrot)
    if (el) {
        float rq = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)ssq * (1.0f / 65536.0f);
            float r = rsqrt_d(ss / (float)hd + 1e-6f);
            r = fminf(r, 127.0f);
            rq = floorf(r * 65536.0f + 0.5f) / 65536.0f;
        }
        float qv = (float)qhi / 256.0f, b = (float)qhj / 256.0f;
        if (A.qk_norm) {
            qv = (qv * rq) * ((float)qni / 256.0f);
            b = (b * rq) * ((float)qnj / 256.0f);
        }
        const float o = first ? (qv * co) - (b * sn) : (b * sn) + (qv * co);
        q_split<KVB>(q16_round(o * 256.0f), tid, qhw, qlw);
    }
    __syncthreads();

    // --- scores (att_score): exact dot, times 1/sqrt(hd), 1/1024 grid; lpp
    // adjacent lanes per position, joined by exact integer shuffles; the
    // running maximum per wave
    const float invsqrt = 1.0f / sqrtf((float)hd);
    const float unit = KVB == 16 ? 1.0f / 524288.0f : 1.0f / 4096.0f;
    // The lane's query words are the same for every position: held in
    // registers, zeroed for a vector past the row, so the dot products below
    // run on every vector slot without branches.
    int m = -32768;
    if (tid / lpp < npos) {  // the threads of a scored position
    int4 qa[KP], qb[KP];
    int ones[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        const int vc = min(sj + k * lpp, nv - 1);
        qa[k] = reinterpret_cast<const int4*>(qhw)[vc];
        qb[k] = reinterpret_cast<const int4*>(qlw)[vc];
    }
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        const bool in = sj + k * lpp < nv;
        keep(qa[k]);
        keep(qb[k]);
        qa[k] = in ? qa[k] : make_int4(0, 0, 0, 0);
        qb[k] = in ? qb[k] : make_int4(0, 0, 0, 0);
        ones[k] = in ? 0x01010101 : 0;
    }
    // One pass: the dot products of position t with its K row w (the own
    // position's K from the LDS copy: its cache row is being written; one
    // branch, taken by the lanes of one position), joined over the lpp lanes,
    // the score stored on its grid.
    auto score = [&](int t, uint4 (&w)[KP]) {
        int sh = 0, sl = 0, sk = 0;
        if (own_row && t == pos) {
            const uint4* own4 = reinterpret_cast<const uint4*>(kpk);
#pragma unroll
            for (int k = 0; k < KP; ++k) w[k] = own4[min(sj + k * lpp, nv - 1)];
        }
#pragma unroll
        for (int k = 0; k < KP; ++k) dot_vec<KVB>(qa[k], qb[k], ones[k], w[k], sh, sl, sk);
        long long d = 256ll * sh + sl;
        if (KVB == 8) d += 128ll * sk;
        for (int o = 1; o < lpp; o <<= 1) d += __shfl_xor(d, o, 64);
        if (sj == 0) {
            const float s = (float)d * unit;
            float f = floorf((s * invsqrt) * 1024.0f + 0.5f);
            f = fminf(fmaxf(f, -32768.0f), 32767.0f);
            sc[t] = (int16_t)f;
            m = max(m, (int)f);
        }
    };
    // The K rows of the next pass (P positions on) are in flight while this
    // pass's dot products run; a wave whose next positions all lie past the
    // context issues none (wave-uniform), and a row at or past npos reads
    // zero.  The first pass (rows loaded at the start) is straight-line code
    // ahead of the loop: inside it, the wait for those rows would be a wait
    // for every load in flight, the first V round's included.
    uint4 knx[KP];
    const int wt0 = wave_u * (64 / lpp);  // the wave's first position of pass 0
    auto prefetch = [&](int it, int t) {
        if (wt0 + (it + 1) * P < npos) {
            const int tn = min(t + P, npos);
#pragma unroll
            for (int k = 0; k < KP; ++k)
                knx[k] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, tn * A.pstride + 16 * min(sj + k * lpp, nv - 1), 0, 0));
        }
    };
    {
        const int t = tid / lpp;  // below npos (the branch above)
        prefetch(0, t);
        score(t, kreg);
    }
    for (int it = 1;; ++it) {
        const int t = tid / lpp + it * P;
        if (t >= npos) break;
        uint4 w[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) w[k] = knx[k];
        prefetch(it, t);
        score(t, w);
    }
    }
    m = wave_max(m);
    if (lane == 0) wmax[wave] = m;
    __syncthreads();

    // --- stats (att_stats): the max (exact), exponentials, chunk sums in
    // position order, then the chunk sums in chunk order (every thread)
    int mi = -32768;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) mi = max(mi, wmax[w]);
    const float mx = (float)mi / 1024.0f;
    // exponentials to the end of the last chunk, +0.0 past npos: adding +0.0
    // leaves a sum of non-negative terms unchanged, so the sums below run
    // over whole chunks without a branch
    for (int t = tid; t < nch * kChunk; t += kThreads)
        ep[t] = t < npos ? (double)exp_d((float)sc[t] / 1024.0f - mx) : 0.0;
    __syncthreads();
    for (int c = tid; c < nch; c += kThreads) {
        const double2* e2 = reinterpret_cast<const double2*>(ep + c * kChunk);
        double cs = 0.0;
#pragma unroll
        for (int k = 0; k < kChunk / 2; ++k) {
            const double2 f = e2[k];
            cs += f.x;
            cs += f.y;
        }
        csum[c] = cs;
    }
    __syncthreads();
    float iv;
    {
        // every thread adds the chunk sums in chunk order, eight read at a
        // time (a +0.0 past the last chunk leaves the sum as it is)
        double sum = 0.0;
        for (int c0 = 0; c0 < nch; c0 += 8) {
            double t[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) t[k] = c0 + k < nch ? csum[c0 + k] : 0.0;
#pragma unroll
            for (int k = 0; k < 8; ++k) sum += t[k];
        }
        const float fs = (float)sum;
        float qs = floorf(fs * 32.0f + 0.5f);
        qs = fminf(fmaxf(qs, -32768.0f), 32767.0f);
        const float sd = qs / 32.0f;
        iv = sd > 0.0f ? 1.0f / sd : 0.0f;
    }

    // --- weighted V (att_v): rounds of vC chunks, one chunk per vG waves, a
    // lane per element (two above head_dim 64) of the head; each lane sums
    // its elements over the chunk's positions in position order, then the
    // round's chunk sums join the running total in chunk order.
    // The weight of position t, p = e*iv (float) times the V grid unit: a +=
    // p*v with v = q*vunit, and p (24-bit mantissa) times q (at most 16 bits)
    // is exact in double, so fma(p*vunit, q, a) rounds exactly as the add of
    // the product does.  Each row of 16 lanes forms the weights of the
    // chunk's 32 positions in two registers and every position's weight
    // reaches the row by a DPP row broadcast.  Positions past npos have
    // weight zero (a + 0*q is a), so all 32 slots run without a branch.
    const double vunit_d = KVB == 16 ? 1.0 / 2048.0 : 1.0 / 16.0;
    if (pair) {
        // the same arithmetic as the plans below -- a chain per element in
        // position order, the round's chunk partials joined in chunk order --
        // over two chunks a wave (lanes 32..63 the second); the DPP row
        // broadcast stays inside a chunk (16-lane rows)
        constexpr int kPC = 2 * (kThreads / 64);  // chunks a round
        for (int c0 = 0; c0 < nch; c0 += kPC) {
            const int nr = min(kPC, nch - c0);
            const bool more = c0 + kPC < nch;
            int vnx[kChunk];
            if (more && c0 + kPC + 2 * wave_u < nch) {
                v_pair_load<KVB>(A, vrs, c0 + kPC + pch, pvi, vnx);
            } else {
#pragma unroll
                for (int u = 0; u < kChunk; ++u) vnx[u] = 0;
            }
            if (2 * wave < nr) {
                const int c = c0 + pch;  // this lane's chunk (past nch: weights zero)
                const int tlo = c * kChunk + (lane & 15), thi = tlo + 16, tmax = A.nchmax * kChunk - 1;
                double wlo = tlo < npos ? (double)((float)ep[min(tlo, tmax)] * iv) * vunit_d : 0.0;
                double whi = thi < npos ? (double)((float)ep[min(thi, tmax)] * iv) * vunit_d : 0.0;
                // the last position of a launch that appends is pos: its V
                // comes from the LDS copy (its cache row is being written)
                if (own_row) {
                    const int own = (int)*reinterpret_cast<const uint32_t*>(vpk + pvi * (KVB / 8));
                    const int uo = c == nch - 1 ? npos - 1 - c * kChunk : -1;
#pragma unroll
                    for (int u = 0; u < kChunk; ++u) vch[u] = u == uo ? own : vch[u];
                }
                double a[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) a[e] = 0.0;
                static_for<0, kChunk>([&](auto U) {
                    constexpr int u = decltype(U)::value;
                    if constexpr (EPL == 4)
                        asm volatile("" : "+v"(wlo), "+v"(whi), "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]));
                    else
                        asm volatile("" : "+v"(wlo), "+v"(whi), "+v"(a[0]), "+v"(a[1]));
                    const double wu = chunk_w<u>(wlo, whi);
                    const unsigned x = (unsigned)vch[u];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        const int q = KVB == 16 ? (int)(int16_t)(x >> (16 * e)) : (int)(int8_t)(x >> (8 * e));
                        a[e] = fma(wu, (double)q, a[e]);
                    }
                });
                if (pe < hd && c < nch) {
                    double* vp = vpart + (c - c0) * hd + pe;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) vp[e] = a[e];
                }
            }
            __syncthreads();
            const bool last = c0 + nr >= nch;
            for (int i = tid; i < hd; i += kThreads) {
                double sacc = c0 == 0 ? 0.0 : acc[i];
                for (int r0 = 0; r0 < nr; r0 += 8) {
                    double pv[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) pv[k] = vpart[min(r0 + k, kPC - 1) * hd + i];
#pragma unroll
                    for (int k = 0; k < 8; ++k) sacc += r0 + k < nr ? pv[k] : 0.0;
                }
                if (last) out[h * hd + i] = (int16_t)q16_round((float)sacc * 256.0f);
                else acc[i] = sacc;
            }
            if (!last) __syncthreads();
            if (more) {
#pragma unroll
                for (int u = 0; u < kChunk; ++u) vch[u] = vnx[u];
            }
        }
        return;
    }
    for (int c0 = 0; c0 < nch; c0 += vC) {
        const int nr = min(vC, nch - c0);
        // the next round's V values load while this round is summed
        const bool more = c0 + vC < nch;
        int vnx[kChunk];
        if (more && slot < vC && c0 + vC + slot < nch) {
            v_chunk_load<KVB>(A, vrs, vE, c0 + vC + slot, vi, vnx);
        } else {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) vnx[u] = 0;
        }
        if (slot < nr) {
            const int c = c0 + slot;
            // lane 16r + n: the weights of the chunk's positions n (lo) and
            // 16 + n (hi), broadcast along the row to every lane in the chain
            const int tlo = c * kChunk + (lane & 15), thi = tlo + 16;
            double wlo = tlo < npos ? (double)((float)ep[tlo] * iv) * vunit_d : 0.0;
            double whi = thi < npos ? (double)((float)ep[thi] * iv) * vunit_d : 0.0;
            // the last position of a launch that appends is pos: its V comes
            // from the LDS copy (its cache row is being written)
            if (own_row && c == nch - 1) {
                const int own = vE == 2 ? (KVB == 16 ? (int)*reinterpret_cast<const uint32_t*>(vpk + vi * 2)
                                                       : (int)*reinterpret_cast<const uint16_t*>(vpk + vi))
                                          : (KVB == 16 ? (int)*reinterpret_cast<const uint16_t*>(vpk + vi * 2)
                                                       : (int)vpk[vi]);
                const int uo = npos - 1 - c * kChunk;
#pragma unroll
                for (int u = 0; u < kChunk; ++u) vch[u] = u == uo ? own : vch[u];
            }
            // every slot, without a branch: past npos the weight is zero
            // (the weight registers pass through the chain, so each position's
            // broadcast follows the previous fma: hoisted, a chunk's 32
            // broadcasts would not fit in registers)
            double a = 0.0, b = 0.0;
            if (vE == 2) {
                static_for<0, kChunk>([&](auto U) {
                    constexpr int u = decltype(U)::value;
                    asm volatile("" : "+v"(wlo), "+v"(whi), "+v"(a), "+v"(b));
                    const double wu = chunk_w<u>(wlo, whi);
                    a = fma(wu, (double)v_lo<KVB>(vch[u]), a);
                    b = fma(wu, (double)v_hi<KVB>(vch[u]), b);
                });
            } else {
                static_for<0, kChunk>([&](auto U) {
                    constexpr int u = decltype(U)::value;
                    asm volatile("" : "+v"(wlo), "+v"(whi), "+v"(a));
                    a = fma(chunk_w<u>(wlo, whi), (double)v_lo<KVB>(vch[u]), a);
                });
            }
            if (ve < hd) {
                vpart[slot * hd + ve] = a;
                if (vE == 2) vpart[slot * hd + ve + 1] = b;
            }
        }
        __syncthreads();
        const bool last = c0 + nr >= nch;
        for (int i = tid; i < hd; i += kThreads) {
            double s = c0 == 0 ? 0.0 : acc[i];
            for (int r0 = 0; r0 < nr; r0 += 8) {
                double pv[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) pv[k] = vpart[min(r0 + k, vC - 1) * hd + i];
#pragma unroll
                for (int k = 0; k < 8; ++k) s += r0 + k < nr ? pv[k] : 0.0;
            }
            if (last) out[h * hd + i] = (int16_t)q16_round((float)s * 256.0f);
            else acc[i] = s;
        }
        if (!last) __syncthreads();
        if (more) {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) vch[u] = vnx[u];
        }
    }
}

// ---------------------------------------------------------------------------
// KV pack of ntok consecutive positions pos0.. of one sequence (att_kv_rope,
// the batch's rows written before its attention): a wave per (row, KV head),
// lane l taking elements l, l+64, ...; the attention kernels' own-row pack,
// step for step.
constexpr int kPackWaves = 4;

template <int KVB>
__global__ void __launch_bounds__(64 * kPackWaves) kv_pack_kernel(const AttnDev A, uint8_t* kv, const int32_t* rtab,
                                                                  const int16_t* kn, const int16_t* qkv, int pos0,
                                                                  int ntok) {
    const int item = blockIdx.x * kPackWaves + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= ntok * A.kv_heads) return;  // (a whole wave)
    const int row = item / A.kv_heads, kvh = item - row * A.kv_heads;
    const int hd = A.hd, kv_dim = A.kv_heads * hd, pos = pos0 + row;
    const int16_t* kq = qkv + (size_t)row * (A.dim + 2 * kv_dim) + A.dim + kvh * hd;
    RopeIn kin;
    int vin[4];
    rope_load(A.rope_half, A.qk_norm, hd, kq, kn, rtab + (size_t)pos * (hd / 2) * 2, lane, kin);
#pragma unroll
    for (int c = 0; c < 4; ++c) vin[c] = 64 * c < hd ? kq[kv_dim + min(lane + 64 * c, hd - 1)] : 0;
    double ssk = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int k = lane + 64 * c < hd ? kin.a[c] : 0;
        ssk += (double)(k * k);
    }
    ssk = wave_sum_exact(ssk);
    float rk = 1.0f;
    if (A.qk_norm) {
        const float ss = (float)ssk * (1.0f / 65536.0f);
        rk = rsqrt_d(ss / (float)hd + 1e-6f);
    }
    uint8_t* const krow = kv + ((size_t)kvh * A.seq + pos) * A.pstride;
    uint8_t* const vrow = kv + ((size_t)(A.kv_heads + kvh) * A.seq + pos) * A.pstride;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int i = lane + 64 * c;
        if (i >= hd) continue;
        int j, ti;
        bool first;
        rope_pair(A.rope_half, hd, i, j, ti, first);
        const float co = (float)kin.co[c] / 4096.0f, sn = (float)kin.sn[c] / 4096.0f;
        float vv = (float)kin.a[c] / 256.0f, bb = (float)kin.b[c] / 256.0f;
        if (A.qk_norm) {
            vv = (vv * rk) * ((float)kin.na[c] / 256.0f);
            bb = (bb * rk) * ((float)kin.nb[c] / 256.0f);
        }
        const float o = first ? (vv * co) - (bb * sn) : (bb * sn) + (vv * co);
        kv_put<KVB>(krow, i, kv_enc<KVB>(o));
        kv_put<KVB>(vrow, i, kv_enc<KVB>((float)vin[c] / 256.0f));
    }
}

// ---------------------------------------------------------------------------
// Query-block attention: one workgroup per (KV head, slice of its query heads)
// and block of query vectors -- the slice's heads at tq consecutive positions
// of one sequence (batched prefill), or at one position of sequence blockIdx.z
// (sequences in lockstep).  Each position's K row is read once per block and
// dotted with every query vector of the block (the first K rows issue at kernel
// start); the weighted V sum runs a wave per (query vector, chunk) with the V
// values in registers.  The statistics and the weighted V sum of each query
// vector follow the per-head
// kernel step for step (the same score grid, max, exponentials, chunk sums in
// position order, the total in chunk order, weights, per-chunk fma chains
// added in chunk order), so every output equals the per-head kernel's bit for
// bit.
struct GroupArgs {
    uint8_t* kv;
    const int32_t* rtab;
    const int16_t* qn;
    const int16_t* kn;
    const int16_t* qkv;
    int16_t* out;
    size_t seq_stride;  // sequences mode: bytes from one sequence's cache to the next
    int pos0;           // batch: position of row 0; sequences: the position
    int ntok;           // batch: rows of the batch
    int tq;             // batch: rows (positions) per block; sequences: 1
    int hs;             // query heads per workgroup (a divisor of the group)
    int seqs;           // 1: blockIdx.z is the sequence, every row at pos0
    int write;          // sequences: pack row pos0 of this KV head first
    int fstride;        // floats per query vector's score row (nchmax chunks of 33)
    int rc;             // chunks per V round
    int qws;            // int words per query vector's plane (zero-padded to the lane plan)
    int o_qh, o_ql, o_kpk, o_vpk, o_f, o_cs, o_st, o_part, o_vs;  // LDS byte offsets
};

// The own row's V field of elements i (and i+1 when vE is 2) from its LDS copy,
// as v_chunk_load stores it.
template <int KVB>
__device__ __forceinline__ int vpk_word(const uint8_t* vpk, int vE, int i) {
    if (vE == 2)
        return KVB == 16 ? (int)*reinterpret_cast<const uint32_t*>(vpk + i * 2)
                         : (int)*reinterpret_cast<const uint16_t*>(vpk + i);
    return KVB == 16 ? (int)*reinterpret_cast<const uint16_t*>(vpk + i * 2) : (int)vpk[i];
}

// A query vector's score row: position t at t + t/32 (one pad float per chunk,
// so a lane per chunk reads distinct banks).
__device__ __forceinline__ int fidx(int t) { return t + (t >> 5); }

// VE: V elements per lane of the weighted-V pass, 2 above head_dim 64.  QG:
// query vectors per work unit of that pass (2 for blocks of at most two).
template <int KVB, int VE, int QG>
__global__ void __launch_bounds__(kThreads) attn_group_kernel(const AttnDev A, const GroupArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KP = kKPre<KVB>;
    constexpr int VPV = 128 / KVB;  // V values per 16-byte vector
    const int hd = A.hd, G = A.group, kv_dim = A.kv_heads * hd;
    const int nsl = G / g.hs;  // head slices per KV head
    const int kvh = blockIdx.x / nsl, h0 = kvh * G + (blockIdx.x - kvh * nsl) * g.hs;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rbase = g.seqs ? (int)blockIdx.z : (int)blockIdx.y * g.tq;
    const int nrow = g.seqs ? 1 : min(g.tq, g.ntok - rbase);
    const int hs = g.hs, nq = hs * nrow;
    uint8_t* kv = g.kv + (g.seqs ? (size_t)blockIdx.z * g.seq_stride : 0);
    const int qrow = A.dim + 2 * kv_dim;
    const int pfirst = g.seqs ? g.pos0 : g.pos0 + rbase;  // position of the block's row 0
    const int npmax = pfirst + nrow;
    uint8_t* const khead_w = kv + (size_t)kvh * A.seq * A.pstride;
    uint8_t* const vhead_w = kv + (size_t)(A.kv_heads + kvh) * A.seq * A.pstride;
    const uint8_t* khead = khead_w;
    int* qhw = reinterpret_cast<int*>(smem + g.o_qh);  // [nq][qws]
    int* qlw = reinterpret_cast<int*>(smem + g.o_ql);
    uint8_t* kpk = smem + g.o_kpk;  // the own row's packed K / V (sequences mode)
    uint8_t* vpk = smem + g.o_vpk;
    float* F = reinterpret_cast<float*>(smem + g.o_f);         // [nq][fstride]
    double* cs = reinterpret_cast<double*>(smem + g.o_cs);     // [nq][nchmax] chunk sums
    float* st = reinterpret_cast<float*>(smem + g.o_st);       // [nq][2]: max, 1/sum
    double* part = reinterpret_cast<double*>(smem + g.o_part);  // [item][rc][64*vE]
    const bool own = g.write != 0;
    // query vector v = j*hs + i: row j of the block, head h0 + i, position pfirst + j

    // --- every global read that waits for nothing is issued first: the K rows
    // of this thread's first scored position
    const int nv = hd * KVB / 128;
    const int lpp = A.lpp, sj = tid & (lpp - 1), P = kThreads / lpp;
    uint4 kreg[KP];
    {
        const int t = min(tid / lpp, npmax - 1);
        const uint4* src = reinterpret_cast<const uint4*>(khead + (size_t)t * A.pstride);
#pragma unroll
        for (int k = 0; k < KP; ++k) kreg[k] = src[min(sj + k * lpp, nv - 1)];
    }
    const int nchb = (npmax + kChunk - 1) / kChunk;
    constexpr int vE = VE;
    const int nblk = (hd + 64 * vE - 1) / (64 * vE);
    const int nitem = nq * nblk;
    // rows 0 .. npmax-1 of the head's V plane; a row past them reads zero
    const __amdgpu_buffer_rsrc_t vrs = rows_rsrc(vhead_w, npmax * A.pstride);

    // the own row's K and V inputs (last wave, sequences mode) and the first
    // query vector's inputs of each wave: loaded before the first barrier
    const int last = kThreads / 64 - 1;
    const int16_t* const kq = g.qkv + (size_t)rbase * qrow + A.dim + kvh * hd;
    RopeIn kin, qin;
    int vin[4];
    if (own && wave == last) {
        rope_load(A.rope_half, A.qk_norm, hd, kq, g.kn, g.rtab + (size_t)g.pos0 * (hd / 2) * 2, lane, kin);
#pragma unroll
        for (int c = 0; c < 4; ++c) vin[c] = 64 * c < hd ? kq[kv_dim + min(lane + 64 * c, hd - 1)] : 0;
    }
    auto q_load = [&](int v) {
        const int j = v / hs, h = h0 + (v - j * hs);
        rope_load(A.rope_half, A.qk_norm, hd, g.qkv + (size_t)(rbase + j) * qrow + h * hd, g.qn,
                  g.rtab + (size_t)(pfirst + j) * (hd / 2) * 2, lane, qin);
    };
    if (wave < nq) q_load(wave);

    // The V rows of a round, staged in LDS: rows c0*kChunk .. of the head's
    // plane are contiguous, so the round is one byte range read in 16-byte
    // pieces, kVStage a thread at most.  Rows at or past npmax read zero; the
    // own row (sequences mode) comes from its LDS copy, as its cache row is
    // being written.  The first round's pieces are issued after the query
    // and own-row inputs (loads return in order: issued first, they would
    // hold up the query prep) and arrive during the scores and the stats.
    uint8_t* const vs = smem + g.o_vs;  // [rc * kChunk][pstride]
    const int per_row = A.pstride / 16;
    uint4 vst[kVStage];
    int vs_n = 0;  // pieces of the round in flight
    auto stage_load = [&](int c0) {
        const int row0 = c0 * kChunk;
        vs_n = (min(row0 + g.rc * kChunk, npmax) - row0) * per_row;
        const int base = row0 * A.pstride;
#pragma unroll
        for (int k = 0; k < kVStage; ++k)
            if (k * kThreads < vs_n)
                vst[k] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, base + 16 * min(tid + k * kThreads, vs_n - 1), 0, 0));
    };
    auto stage_store = [&](int c0) {
        const int own_piece = own ? (npmax - 1 - c0 * kChunk) * per_row : -1;
#pragma unroll
        for (int k = 0; k < kVStage; ++k) {
            const int i = tid + k * kThreads;
            if (k * kThreads < vs_n && i < vs_n) {
                uint4 x = vst[k];
                if (i >= own_piece && i < own_piece + per_row && own_piece >= 0)
                    x = reinterpret_cast<const uint4*>(vpk)[i - own_piece];
                reinterpret_cast<uint4*>(vs)[i] = x;
            }
        }
    };
    stage_load(0);

    // the query planes' words past the row stay zero, so the scores need no mask
    for (int i = tid; i < nq * g.qws; i += kThreads) qhw[i] = qlw[i] = 0;
    __syncthreads();

    // --- the own row's KV pack (att_kv_rope), by the last wave while the first
    // waves prepare the queries: lane l takes elements l, l+64, ... of the KV
    // head; the first slice's workgroup stores the row
    if (own && wave == last) {
        const bool store = h0 == kvh * G;
        double ssk = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = lane + 64 * c < hd ? kin.a[c] : 0;
            ssk += (double)(k * k);
        }
        ssk = wave_sum_exact(ssk);
        float rk = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)ssk * (1.0f / 65536.0f);
            rk = rsqrt_d(ss / (float)hd + 1e-6f);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int i = lane + 64 * c;
            if (i >= hd) continue;
            int j, ti;
            bool first;
            rope_pair(A.rope_half, hd, i, j, ti, first);
            const float co = (float)kin.co[c] / 4096.0f, sn = (float)kin.sn[c] / 4096.0f;
            float vv = (float)kin.a[c] / 256.0f, bb = (float)kin.b[c] / 256.0f;
            if (A.qk_norm) {
                vv = (vv * rk) * ((float)kin.na[c] / 256.0f);
                bb = (bb * rk) * ((float)kin.nb[c] / 256.0f);
            }
            const float o = first ? (vv * co) - (bb * sn) : (bb * sn) + (vv * co);
            const int q = kv_enc<KVB>(o);
            const int qv = kv_enc<KVB>((float)vin[c] / 256.0f);
            if (store) {
                kv_put<KVB>(khead_w + (size_t)g.pos0 * A.pstride, i, q);
                kv_put<KVB>(vhead_w + (size_t)g.pos0 * A.pstride, i, qv);
            }
            kv_put<KVB>(kpk, i, q);
            kv_put<KVB>(vpk, i, qv);
        }
    }

    // --- q prep (att_qnorm_scale + att_qrot), a wave per query vector
    for (int v = wave; v < nq; v += kThreads / 64) {
        if (v != wave) q_load(v);
        double ssq = 0.0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int q = lane + 64 * c < hd ? qin.a[c] : 0;
            ssq += (double)(q * q);
        }
        ssq = wave_sum_exact(ssq);
        float rq = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)ssq * (1.0f / 65536.0f);
            float r = rsqrt_d(ss / (float)hd + 1e-6f);
            r = fminf(r, 127.0f);
            rq = floorf(r * 65536.0f + 0.5f) / 65536.0f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int i = lane + 64 * c;
            if (i >= hd) continue;
            int jj, ti;
            bool first;
            rope_pair(A.rope_half, hd, i, jj, ti, first);
            const float co = (float)qin.co[c] / 4096.0f, sn = (float)qin.sn[c] / 4096.0f;
            float qv = (float)qin.a[c] / 256.0f, b = (float)qin.b[c] / 256.0f;
            if (A.qk_norm) {
                qv = (qv * rq) * ((float)qin.na[c] / 256.0f);
                b = (b * rq) * ((float)qin.nb[c] / 256.0f);
            }
            const float o = first ? (qv * co) - (b * sn) : (b * sn) + (qv * co);
            q_split<KVB>(q16_round(o * 256.0f), i, qhw + v * g.qws, qlw + v * g.qws);
        }
    }
    __syncthreads();

    // --- scores (att_score): lpp lanes per position, the position's K row in
    // registers, dotted with every query vector of the block whose position
    // reaches it
    {
        const float invsqrt = 1.0f / sqrtf((float)hd);
        const float unit = KVB == 16 ? 1.0f / 524288.0f : 1.0f / 4096.0f;
        for (int t = tid / lpp, it = 0; t < npmax; t += P, ++it) {
            uint4 w[KP];
            if (it == 0) {
#pragma unroll
                for (int k = 0; k < KP; ++k) w[k] = kreg[k];
            } else {
                const uint4* src = reinterpret_cast<const uint4*>(khead + (size_t)t * A.pstride);
#pragma unroll
                for (int k = 0; k < KP; ++k) w[k] = src[min(sj + k * lpp, nv - 1)];
            }
            if (own && t == g.pos0) {
                const uint4* o4 = reinterpret_cast<const uint4*>(kpk);
#pragma unroll
                for (int k = 0; k < KP; ++k) w[k] = o4[min(sj + k * lpp, nv - 1)];
            }
            int sk = 0;
            if (KVB == 8) {
#pragma unroll
                for (int k = 0; k < KP; ++k) {
                    const int ones = sj + k * lpp < nv ? 0x01010101 : 0;
                    const unsigned ws[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) sk = __builtin_amdgcn_sdot4(ones, (int)ws[u], sk, false);
                }
            }
            const int j0 = max(t - pfirst, 0);  // rows j >= j0 reach position t
            for (int v = j0 * hs; v < nq; ++v) {
                const int4* qa4 = reinterpret_cast<const int4*>(qhw + v * g.qws) + sj;
                const int4* qb4 = reinterpret_cast<const int4*>(qlw + v * g.qws) + sj;
                int sh = 0, sl = 0;
#pragma unroll
                for (int k = 0; k < KP; ++k) {
                    const int4 qa = qa4[k * lpp], qb = qb4[k * lpp];
                    const unsigned ws[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
                    const int as[4] = {qa.x, qa.y, qa.z, qa.w}, bs[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        if (KVB == 16) {
                            sh = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, as[u]),
                                                        __builtin_bit_cast(short2_t, ws[u]), sh, false);
                            sl = __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, bs[u]),
                                                        __builtin_bit_cast(short2_t, ws[u]), sl, false);
                        } else {
                            sh = __builtin_amdgcn_sdot4(as[u], (int)ws[u], sh, false);
                            sl = __builtin_amdgcn_sdot4(bs[u], (int)ws[u], sl, false);
                        }
                    }
                }
                long long d = 256ll * sh + sl;
                if (KVB == 8) d += 128ll * sk;
                for (int o = 1; o < lpp; o <<= 1) d += __shfl_xor(d, o, 64);
                if (sj == 0) {
                    const float s = (float)d * unit;
                    float f = floorf((s * invsqrt) * 1024.0f + 0.5f);
                    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
                    F[v * g.fstride + fidx(t)] = f;
                }
            }
        }
    }
    __syncthreads();


    // --- stats (att_stats): the max per query vector (a wave each), the
    // exponentials (+0.0 to the end of the last chunk), chunk sums in position
    // order, their total in chunk order, 1/sum on its grid
    for (int v = wave; v < nq; v += kThreads / 64) {
        const float* Fv = F + v * g.fstride;
        const int npos = pfirst + v / hs + 1;
        int m = -32768;
        for (int t = lane; t < npos; t += 64) m = max(m, (int)Fv[fidx(t)]);
        m = wave_max(m);
        if (lane == 0) st[2 * v] = (float)m / 1024.0f;
    }
    __syncthreads();
    for (int v = 0; v < nq; ++v) {
        float* Fv = F + v * g.fstride;
        const int npos = pfirst + v / hs + 1, nch = (npos + kChunk - 1) / kChunk;
        const float mx = st[2 * v];
        for (int t = tid; t < nch * kChunk; t += kThreads)
            Fv[fidx(t)] = t < npos ? exp_d(Fv[fidx(t)] / 1024.0f - mx) : 0.0f;
    }
    __syncthreads();
    for (int i = tid; i < nq * nchb; i += kThreads) {
        const int v = i / nchb, c = i - v * nchb;
        if (c * kChunk > pfirst + v / hs) continue;
        const float* Fc = F + v * g.fstride + fidx(c * kChunk);
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < kChunk; ++k) s += (double)Fc[k];
        cs[v * A.nchmax + c] = s;
    }
    // the first V round's rows go to LDS beside the chunk sums; the second
    // round's start loading
    stage_store(0);
    if (g.rc < nchb) stage_load(g.rc);
    __syncthreads();
    // 1/sum of query vector v in lane v of every wave
    float ivl = 0.0f;
    if (lane < nq) {
        const int v = lane, nch = (pfirst + v / hs + 1 + kChunk - 1) / kChunk;
        // eight chunk sums read at a time, added in chunk order (a +0.0 past
        // the last chunk leaves the sum as it is)
        double sum = 0.0;
        for (int c0 = 0; c0 < nch; c0 += 8) {
            double t[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) t[k] = c0 + k < nch ? cs[v * A.nchmax + c0 + k] : 0.0;
#pragma unroll
            for (int k = 0; k < 8; ++k) sum += t[k];
        }
        const float fs = (float)sum;
        float qs = floorf(fs * 32.0f + 0.5f);
        qs = fminf(fmaxf(qs, -32768.0f), 32767.0f);
        const float sd = qs / 32.0f;
        ivl = sd > 0.0f ? 1.0f / sd : 0.0f;
    }

    // --- weighted V (att_v) in rounds of rc chunks.  Work unit (group of kQG
    // query vectors, chunk, 64*vE elements), lane = element; the unit's V
    // values come from the round's rows in LDS and are converted once for the
    // group, each query vector's fma chain runs in position order into the
    // round's partials of its item (query vector, elements), then the item's
    // owner wave adds them to its sums in chunk order.  Weight of position t: (double)(e*iv); the sums
    // take the V grid unit at the end (a power of two, so every rounding on
    // the way is the one the weights times the unit would give).
    const double vunit_d = KVB == 16 ? 1.0 / 2048.0 : 1.0 / 16.0;
    constexpr int kItems = 4;  // items per wave (nq * nblk <= 32)
    constexpr int kQG = QG;    // query vectors per work unit (one conversion of V for all)
    double acc_a[kItems], acc_b[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) acc_a[k] = acc_b[k] = 0.0;
    const int wv = __builtin_amdgcn_readfirstlane(wave);  // unit indexing in scalar registers
    for (int r = 0; r * g.rc < nchb; ++r) {
        const int c0 = r * g.rc, ncr = min(g.rc, nchb - c0), nunit = (nq + kQG - 1) / kQG * nblk * ncr;
        if (r > 0) {  // (the first round's rows are in place)
            __syncthreads();  // the previous round's rows and partials are read
            stage_store(c0);
            if (c0 + g.rc < nchb) stage_load(c0 + g.rc);  // the next round's rows load during this one
            __syncthreads();
        }
        for (int unit = wv; unit < nunit; unit += kThreads / 64) {
            const int grp = unit / ncr, c = c0 + unit - grp * ncr;  // grp = query group * nblk + eb
            const int qg = grp / nblk, eb = grp - qg * nblk, v0 = qg * kQG;
            // the group's query vectors that reach chunk c: rows j with c*kChunk <= pfirst + j
            const int vlo = max(v0, (c * kChunk - pfirst) * hs), vhi = min(v0 + kQG, nq);
            if (vlo >= vhi) continue;
            const int vi = min((eb * 64 + lane) * vE, hd - vE);
            const uint8_t* rows = vs + (size_t)(c - c0) * kChunk * A.pstride;
            int vch[kChunk];
#pragma unroll
            for (int u = 0; u < kChunk; ++u) vch[u] = vpk_word<KVB>(rows + u * A.pstride, vE, vi);
            // a query vector of the group that does not reach the chunk runs
            // with zero weights (its sums are not stored): the group's chains
            // interleave without branches
            double wlo[kQG], whi[kQG];
#pragma unroll
            for (int q = 0; q < kQG; ++q) {
                const int v = min(v0 + q, nq - 1);
                const bool on = v0 + q >= vlo && v0 + q < vhi;
                const float* Fc = F + v * g.fstride + fidx(c * kChunk);
                const float iv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ivl), v));
                wlo[q] = on ? (double)(Fc[lane & 15] * iv) : 0.0;
                whi[q] = on ? (double)(Fc[16 + (lane & 15)] * iv) : 0.0;
            }
            double acc[kQG][vE];
#pragma unroll
            for (int q = 0; q < kQG; ++q)
#pragma unroll
                for (int e = 0; e < vE; ++e) acc[q][e] = 0.0;
            // eight positions at a time: each V value converted once for the group
            static_for<0, kChunk / 8>([&](auto UB) {
                constexpr int u0 = decltype(UB)::value * 8;
                double x[8][vE];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    x[j][0] = (double)v_lo<KVB>(vch[u0 + j]);
                    if (vE == 2) x[j][vE - 1] = (double)v_hi<KVB>(vch[u0 + j]);
                }
                static_for<0, 8>([&](auto J) {
                    constexpr int j = decltype(J)::value;
#pragma unroll
                    for (int q = 0; q < kQG; ++q) {
                        // the weight registers pass through the chain here, so
                        // this position's broadcast follows the last fma (hoisted,
                        // a whole chunk's weights would not fit in registers)
                        if constexpr (vE == 2)
                            asm volatile("" : "+v"(wlo[q]), "+v"(whi[q]), "+v"(acc[q][0]), "+v"(acc[q][vE - 1]));
                        else
                            asm volatile("" : "+v"(wlo[q]), "+v"(whi[q]), "+v"(acc[q][0]));
                        const double wu = chunk_w<u0 + j>(wlo[q], whi[q]);
#pragma unroll
                        for (int e = 0; e < vE; ++e) acc[q][e] = fma(wu, x[j][e], acc[q][e]);
                    }
                });
            });
#pragma unroll
            for (int q = 0; q < kQG; ++q) {
                if (v0 + q < vlo || v0 + q >= vhi) continue;
                double* pp = part + ((size_t)((v0 + q) * nblk + eb) * g.rc + (c - c0)) * 64 * vE + lane * vE;
#pragma unroll
                for (int e = 0; e < vE; ++e) pp[e] = acc[q][e];
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            const int it = wv + k * (kThreads / 64);
            const int nch = it < nitem ? (pfirst + (it / nblk) / hs + 1 + kChunk - 1) / kChunk : 0;
            const double* pp = part + (size_t)it * g.rc * 64 * vE + lane * vE;
            const int ncc = min(nch, c0 + ncr) - c0;  // this round's chunks of the item
            // eight partials read at a time, added in chunk order (+0.0 past the last)
            for (int b = 0; b < ncc; b += 8) {
                double ta[8], tb[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    ta[u] = b + u < ncc ? pp[(b + u) * 64 * vE] : 0.0;
                    tb[u] = vE == 2 && b + u < ncc ? pp[(b + u) * 64 * vE + 1] : 0.0;
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc_a[k] += ta[u];
                    if (vE == 2) acc_b[k] += tb[u];
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int item = wave + k * (kThreads / 64);
        const int v = item / nblk, eb = item - v * nblk;
        const int j = v / hs;
        const int ve = (eb * 64 + lane) * vE;
        if (item < nitem && ve < hd) {
            int16_t* o = g.out + (size_t)(rbase + j) * A.dim + (h0 + v - j * hs) * hd;
            o[ve] = (int16_t)q16_round((float)(acc_a[k] * vunit_d) * 256.0f);
            if (vE == 2) o[ve + 1] = (int16_t)q16_round((float)(acc_b[k] * vunit_d) * 256.0f);
        }
    }
}

// LDS carve-up of one workgroup and the lane plan; returns the bytes used.
// The per-head kernel for A's cache width (A laid out by attn_layout), with the
// pair plan for a head of at most 32 fields of 32 bits whose cache holds more
// chunks than one round of the one-element plan.
using AttnKernelFn = void (*)(const AttnDev, uint8_t*, const int32_t*, const int16_t*, const int16_t*,
                              const int16_t*, int16_t*, int, int, int, size_t, int, const int*);
AttnKernelFn attn_kernel_for(const AttnDev& A) {
    const bool pair = A.hd * A.kv_bits <= 32 * 32 && A.nchmax > A.vC1;
    const int nv = A.hd * A.kv_bits / 128;
    if (A.kv_bits == 16) {
        if ((nv + A.lpp1 - 1) / A.lpp1 <= 3) return pair ? attn_kernel<16, true, 3> : attn_kernel<16, false, 3>;
        if ((nv + A.lpp1 - 1) / A.lpp1 <= 4) return pair ? attn_kernel<16, true, 4> : attn_kernel<16, false, 4>;
        return pair ? attn_kernel<16, true, kKPre<16>> : attn_kernel<16, false, kKPre<16>>;
    }
    if ((nv + A.lpp1 - 1) / A.lpp1 <= 3) return pair ? attn_kernel<8, true, 3> : attn_kernel<8, false, 3>;
    return pair ? attn_kernel<8, true, kKPre<8>> : attn_kernel<8, false, kKPre<8>>;
}

size_t attn_layout(AttnDev& A) {
    const int hd = A.hd;
    const int nv = hd * A.kv_bits / 128;
    const int kp = A.kv_bits == 16 ? kKPre<16> : kKPre<8>;
    const int E = A.kv_bits == 16 ? 2 : 4;
    A.lpp = 1;
    while (A.lpp * kp < nv) A.lpp *= 2;
    // The per-head kernel at a q16 cache: the fewest lanes a position (a power
    // of two) that leave at most 4 K vectors a lane, run by the 3- or 4-slot
    // kernel instance.  With more slots a lane, each slot is a 16-byte K load (one
    // lane a position: the wave's 64 lanes a row stride apart), two
    // query-word reads from LDS and a dot product, and the 8-slot instance
    // does all eight whether or not they lie past the row.  Measured against
    // the plan above with the 8-slot kernel: head_dim 64 (two lanes instead
    // of one) the 0.5B t3 decode 1579 -> 1608 tokens/s, the LFM2.5-shaped
    // hybrid's 3126 -> 3151; head_dim 96 (four lanes instead of two, 3 slots)
    // MiniMind3 q8 decode 5882 -> 5972.  The query-block kernel keeps the plan
    // above (two lanes made the 0.5B t3 step over 32 sequences 1.173 -> 1.192
    // ms).
    A.lpp1 = A.lpp;
    if (A.kv_bits == 16) {
        A.lpp1 = 1;
        while ((nv + A.lpp1 - 1) / A.lpp1 > 4) A.lpp1 *= 2;
    }
    A.nchmax = (A.seq + kChunk - 1) / kChunk;
    A.vG1 = (hd + 63) / 64;
    A.vC1 = (kThreads / 64) / A.vG1;
    A.vG2 = hd > 64 ? (hd + 127) / 128 : A.vG1;
    A.vC2 = (kThreads / 64) / A.vG2;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = (off + bytes + 15) & ~(size_t)15;
        return (int)o;
    };
    A.o_wmax = take(4 * (size_t)(kThreads / 64));
    A.o_vpk = take((size_t)hd * A.kv_bits / 8);
    A.o_kpk = take((size_t)hd * A.kv_bits / 8);
    A.o_qhw = take(4 * (size_t)(hd / E));
    A.o_qlw = take(4 * (size_t)(hd / E));
    A.o_sc = take(2 * (size_t)A.seq);
    A.o_ep = take(8 * (size_t)A.nchmax * kChunk);
    A.o_csum = take(8 * (size_t)A.nchmax);
    // (the pair plan, a head of at most 32 fields of 32 bits: 16 chunks a round)
    const int vcm = std::max({A.vC1, A.vC2, hd * A.kv_bits <= 32 * 32 ? 2 * (kThreads / 64) : 0});
    A.o_vpart = take(8 * (size_t)vcm * hd);
    A.o_acc = take(8 * (size_t)hd);
    return off;
}

int launch_group(vgx_attn* at, int layer, int pos, int ntok, const int16_t* qkv, int16_t* out, bool seqs);
// Sequences in lockstep take the query-block kernel from this many query
// heads per KV head (every head of a group then reads the K/V rows once).
constexpr int kGroupSeqsG = 2;

// Positions pos .. pos + ntok - 1 (their qkv and output rows consecutive).
// With ntok > 1 the KV write and the attention must be separate launches: a
// position reads the rows the others write.
int launch(vgx_attn* at, int layer, int pos, int ntok, const int16_t* qkv, int16_t* out, int w, int att,
           bool seqs = false, const int* pos_ptr = nullptr) {
    if (!at) return vgx_fail(VGX_EINVAL, "attention: NULL handle");
    if (layer < 0 || layer >= at->layers || !at->kv[layer])
        return vgx_fail(VGX_ERANGE, "attention: layer " + std::to_string(layer) + " has no KV cache");
    if (ntok <= 0 || ntok > 65535) return vgx_fail(VGX_EINVAL, "attention: ntok outside 1..65535");
    if (seqs) {
        if (ntok > at->nseq)
            return vgx_fail(VGX_ERANGE, "attention: " + std::to_string(ntok) + " sequences, the cache holds " +
                                            std::to_string(at->nseq));
        if (pos < 0 || pos >= at->a.seq)
            return vgx_fail(VGX_ERANGE, "attention: position " + std::to_string(pos) + " outside the KV length");
    } else {
        if (pos < 0 || pos > at->a.seq - ntok)
            return vgx_fail(VGX_ERANGE, "attention: positions " + std::to_string(pos) + ".." +
                                            std::to_string(pos + ntok - 1) + " outside the KV length");
        if (ntok > 1 && w && att) return vgx_fail(VGX_EINVAL, "attention: a batch writes its KV rows first");
    }
    if (!qkv || (att && !out)) return vgx_fail(VGX_EINVAL, "attention: NULL buffer");
    VGX_HIP(hipSetDevice(at->ctx->device));
    const AttnDev& A = at->a;
    const int16_t* qn = at->qn ? at->qn + (size_t)layer * A.hd : nullptr;
    const int16_t* kn = at->kn ? at->kn + (size_t)layer * A.hd : nullptr;
    // a batch of positions, and sequences in lockstep, take the query-block
    // kernel when a block of query vectors fits a workgroup's LDS
    if (att && !pos_ptr && ((!seqs && !w && ntok > 1) || (seqs && w && A.group >= kGroupSeqsG))) {
        const int st = launch_group(at, layer, pos, ntok, qkv, out, seqs);
        if (st != VGX_ESTATE) return st;
    }
    // the rows of a batch of one sequence: the pack kernel
    if (!att && !seqs && !pos_ptr) {
        const dim3 pg((ntok * A.kv_heads + kPackWaves - 1) / kPackWaves);
        if (A.kv_bits == 16)
            hipLaunchKernelGGL(kv_pack_kernel<16>, pg, dim3(64 * kPackWaves), 0, at->ctx->stream, A, at->kv[layer],
                               at->rtab, kn, qkv, pos, ntok);
        else
            hipLaunchKernelGGL(kv_pack_kernel<8>, pg, dim3(64 * kPackWaves), 0, at->ctx->stream, A, at->kv[layer],
                               at->rtab, kn, qkv, pos, ntok);
        VGX_LAUNCH_CHECK("KV pack launch");
        return VGX_OK;
    }
    const dim3 grid(att ? A.heads : A.kv_heads, ntok);
    const size_t stride = seqs ? at->seq_bytes : 0;
    const int step = seqs ? 0 : 1;
    hipLaunchKernelGGL(attn_kernel_for(A), grid, dim3(kThreads), at->lds, at->ctx->stream, A, at->kv[layer],
                       at->rtab, qn, kn, qkv, out, pos, w, att, stride, step, pos_ptr);
    VGX_LAUNCH_CHECK("attention launch");
    return VGX_OK;
}

// LDS of a query-block launch of nq query vectors and rc chunks per V round;
// fills g's offsets.
size_t group_layout(const AttnDev& A, int nq, int rc, GroupArgs& g) {
    const int kp = A.kv_bits == 16 ? kKPre<16> : kKPre<8>;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = (off + bytes + 15) & ~(size_t)15;
        return (int)o;
    };
    g.fstride = A.nchmax * (kChunk + 1);
    g.rc = rc;
    g.qws = 4 * kp * A.lpp;  // every vector slot of the lane plan, zero past the row
    g.o_qh = take(4 * (size_t)nq * g.qws);
    g.o_ql = take(4 * (size_t)nq * g.qws);
    g.o_kpk = take((size_t)A.hd * A.kv_bits / 8);
    g.o_vpk = take((size_t)A.hd * A.kv_bits / 8);
    g.o_f = take(4 * (size_t)nq * g.fstride);
    g.o_cs = take(8 * (size_t)nq * A.nchmax);
    g.o_st = take(8 * (size_t)nq);
    const int vE = A.hd > 64 ? 2 : 1, nblk = (A.hd + 64 * vE - 1) / (64 * vE);
    g.o_part = take((size_t)nq * nblk * rc * 64 * vE * 8);
    g.o_vs = take((size_t)rc * kChunk * A.pstride);
    return off;
}

constexpr size_t kLdsMax = 160 * 1024;

// The block plan of a query-block launch over n rows (batch) or n sequences
// at position pos0: hs query heads per workgroup, tq rows per block -- enough
// workgroups to cover the CUs, at most 16 query vectors a block (32 work items
// of the V pass) -- and rc chunks per V round: the launch's longest context
// when its rows fit the staging registers and LDS.  Returns the LDS bytes, or
// 0 when no plan fits.
size_t group_plan(const AttnDev& A, bool seqs, int pos0, int n, int num_cu, GroupArgs& g) {
    const int G = A.group;
    const int vE = A.hd > 64 ? 2 : 1, nblk = (A.hd + 64 * vE - 1) / (64 * vE);
    const int qmax = std::min(16, 32 / nblk);
    int hs = G;
    while (hs > qmax && hs % 2 == 0) hs /= 2;
    if (hs > qmax) return 0;
    int tq = 1;
    if (seqs) {
        while (hs % 2 == 0 && (long)A.kv_heads * (G / hs) * n < num_cu) hs /= 2;
    } else {
        const int want = (int)(((long)n * A.kv_heads * (G / hs) + num_cu - 1) / num_cu);
        tq = std::max(1, std::min({n, qmax / hs, want}));
    }
    // the score rows do not depend on rc: fit them first
    while (group_layout(A, hs * tq, 1, g) > kLdsMax && tq > 1) --tq;
    const int ctx = seqs ? pos0 + 1 : pos0 + n;
    int rc = std::min({(ctx + kChunk - 1) / kChunk, kVStage * kThreads * 16 / (kChunk * A.pstride), A.nchmax});
    rc = std::max(rc, 1);
    size_t lds = group_layout(A, hs * tq, rc, g);
    while (lds > kLdsMax && rc > 1) lds = group_layout(A, hs * tq, --rc, g);
    if (lds > kLdsMax) return 0;
    g.hs = hs;
    g.tq = tq;
    return lds;
}

using GroupKernel = void (*)(AttnDev, GroupArgs);

// The query-block kernel instance for KV bits, V elements per lane and query
// vectors per V work unit.
GroupKernel group_kernel(int kvb, int ve, int qg) {
    if (kvb == 16) {
        if (ve == 2) return qg == 2 ? attn_group_kernel<16, 2, 2> : attn_group_kernel<16, 2, 4>;
        return qg == 2 ? attn_group_kernel<16, 1, 2> : attn_group_kernel<16, 1, 4>;
    }
    if (ve == 2) return qg == 2 ? attn_group_kernel<8, 2, 2> : attn_group_kernel<8, 2, 4>;
    return qg == 2 ? attn_group_kernel<8, 1, 2> : attn_group_kernel<8, 1, 4>;
}

// The query-block kernel over rows 0..ntok-1 (positions pos .. pos+ntok-1 of
// one sequence), or over position pos of ntok sequences (seqs: packing the
// row first).  Returns VGX_ESTATE when no block plan fits (the caller then
// takes the per-head kernel).
int launch_group(vgx_attn* at, int layer, int pos, int ntok, const int16_t* qkv, int16_t* out, bool seqs) {
    const AttnDev& A = at->a;
    GroupArgs g{};
    const size_t lds = group_plan(A, seqs, pos, ntok, at->ctx->num_cu, g);
    if (!lds) return VGX_ESTATE;
    g.kv = at->kv[layer];
    g.rtab = at->rtab;
    g.qn = at->qn ? at->qn + (size_t)layer * A.hd : nullptr;
    g.kn = at->kn ? at->kn + (size_t)layer * A.hd : nullptr;
    g.qkv = qkv;
    g.out = out;
    g.seq_stride = seqs ? at->seq_bytes : 0;
    g.pos0 = pos;
    g.ntok = ntok;
    g.seqs = seqs ? 1 : 0;
    g.write = seqs ? 1 : 0;
    const int nsl = A.group / g.hs;
    const dim3 grid(A.kv_heads * nsl, seqs ? 1 : (ntok + g.tq - 1) / g.tq, seqs ? ntok : 1);
    hipLaunchKernelGGL(group_kernel(A.kv_bits, A.hd > 64 ? 2 : 1, g.hs * g.tq <= 2 ? 2 : 4), grid, dim3(kThreads), lds,
                       at->ctx->stream, A, g);
    VGX_LAUNCH_CHECK("query-block attention launch");
    return VGX_OK;
}

}  // namespace

extern "C" {

int vgx_attn_create(vgx_ctx* ctx, const vgx_attn_desc* d, vgx_attn** out) {
    return vgx_attn_create_seqs(ctx, d, 1, out);
}

int vgx_attn_create_seqs(vgx_ctx* ctx, const vgx_attn_desc* d, int nseq, vgx_attn** out) {
    if (!ctx || !d || !out) return vgx_fail(VGX_EINVAL, "vgx_attn_create: NULL argument");
    *out = nullptr;
    if (nseq <= 0 || nseq > 65535) return vgx_fail(VGX_EINVAL, "vgx_attn_create_seqs: nseq outside 1..65535");
    if (d->dim <= 0 || d->heads <= 0 || d->kv_heads <= 0 || d->head_dim <= 0 || d->seq <= 0 || d->layers <= 0)
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: empty shape");
    if (d->heads % d->kv_heads) return vgx_fail(VGX_EINVAL, "vgx_attn_create: heads not a multiple of kv_heads");
    if (d->head_dim % 16 || d->head_dim > 256)
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: head_dim must be a multiple of 16, at most 256");
    if (d->heads * d->head_dim != d->dim) return vgx_fail(VGX_EINVAL, "vgx_attn_create: heads*head_dim != dim");
    if (d->kv_bits != 16 && d->kv_bits != 8) return vgx_fail(VGX_EINVAL, "vgx_attn_create: kv_bits must be 16 or 8");
    if (!d->rope_cos || !d->rope_sin) return vgx_fail(VGX_EINVAL, "vgx_attn_create: rope tables are NULL");
    if (d->qk_norm && (!d->q_norm || !d->k_norm)) return vgx_fail(VGX_EINVAL, "vgx_attn_create: qk_norm without weights");
    VGX_HIP(hipSetDevice(ctx->device));
    vgx_attn* at = new vgx_attn();
    at->ctx = ctx;
    at->layers = d->layers;
    AttnDev& A = at->a;
    A.dim = d->dim; A.heads = d->heads; A.kv_heads = d->kv_heads; A.hd = d->head_dim; A.seq = d->seq;
    A.kv_bits = d->kv_bits; A.rope_half = d->rope_half ? 1 : 0; A.qk_norm = d->qk_norm ? 1 : 0;
    A.group = d->heads / d->kv_heads;
    A.row_bytes = 2 * d->kv_heads * d->head_dim * (d->kv_bits / 8);
    A.pstride = d->head_dim * (d->kv_bits / 8);
    at->lds = attn_layout(A);
    if (at->lds > kLdsMax) {
        delete at;
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: seq too long for one workgroup's LDS");
    }
    auto fail = [&](hipError_t e, const char* w) { vgx_attn_free(at); return vgx_hip_fail(e, w); };
    at->nseq = nseq;
    at->seq_bytes = (size_t)A.seq * A.row_bytes;
    const size_t lb = at->seq_bytes * nseq;
    at->kv.assign((size_t)d->layers, nullptr);
    for (int l = 0; l < d->layers; ++l) {
        if (d->layer_is_attn && !d->layer_is_attn[l]) continue;
        hipError_t e = hipMalloc(&at->kv[l], lb);
        if (e == hipSuccess) e = hipMemset(at->kv[l], 0, lb);
        if (e != hipSuccess) return fail(e, "KV cache");
    }
    // RoPE texture (engine/src/gpu_attn.cpp:142-156): lrintf(x*4096)
    const int half = A.hd / 2;
    std::vector<int32_t> tab((size_t)A.seq * half * 2);
    for (size_t k = 0; k < (size_t)A.seq * half; ++k) {
        tab[2 * k] = (int32_t)lrintf(d->rope_cos[k] * 4096.0f);
        tab[2 * k + 1] = (int32_t)lrintf(d->rope_sin[k] * 4096.0f);
    }
    hipError_t e = hipMalloc(&at->rtab, tab.size() * 4);
    if (e == hipSuccess) e = hipMemcpy(at->rtab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(e, "rope table");
    if (A.qk_norm) {
        // make_q16_texture (engine/src/gpu_state.cpp:377-384): quantize_act
        std::vector<int16_t> q((size_t)d->layers * A.hd), k((size_t)d->layers * A.hd);
        vgx_quantize_act(d->q_norm, (int)q.size(), q.data());
        vgx_quantize_act(d->k_norm, (int)k.size(), k.data());
        e = hipMalloc(&at->qn, q.size() * 2);
        if (e == hipSuccess) e = hipMemcpy(at->qn, q.data(), q.size() * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMalloc(&at->kn, k.size() * 2);
        if (e == hipSuccess) e = hipMemcpy(at->kn, k.data(), k.size() * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail(e, "q/k norm weights");
    }
    // the per-head kernel's limit at the most any layout takes (another handle
    // of another shape shares the kernel)
    const hipError_t a1 = hipFuncSetAttribute((const void*)attn_kernel_for(A),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
    if (a1 != hipSuccess) return fail(a1, "hipFuncSetAttribute");
    for (int kvb : {16, 8})
        for (int ve : {1, 2})
            for (int qg : {2, 4}) {
                const hipError_t a = hipFuncSetAttribute((const void*)group_kernel(kvb, ve, qg),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
                if (a != hipSuccess) return fail(a, "hipFuncSetAttribute");
            }
    *out = at;
    return VGX_OK;
}

int vgx_attn_seq_view(vgx_attn* a, int s, vgx_attn** out) {
    if (!a || !out) return vgx_fail(VGX_EINVAL, "vgx_attn_seq_view: NULL argument");
    *out = nullptr;
    if (s < 0 || s >= a->nseq) return vgx_fail(VGX_ERANGE, "vgx_attn_seq_view: no such sequence");
    vgx_attn* v = new vgx_attn(*a);
    v->owner = false;
    v->nseq = 1;
    for (auto& p : v->kv)
        if (p) p += (size_t)s * a->seq_bytes;
    *out = v;
    return VGX_OK;
}

int vgx_attn_free(vgx_attn* at) {
    if (!at) return VGX_OK;
    if (!at->owner) {
        delete at;
        return VGX_OK;
    }
    for (uint8_t* p : at->kv) if (p) (void)hipFree(p);
    if (at->rtab) (void)hipFree(at->rtab);
    if (at->qn) (void)hipFree(at->qn);
    if (at->kn) (void)hipFree(at->kn);
    delete at;
    return VGX_OK;
}

int vgx_kv_append(vgx_attn* a, int layer, int pos, const int16_t* qkv) {
    return launch(a, layer, pos, 1, qkv, nullptr, 1, 0);
}

int vgx_attn_decode(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos, 1, qkv, out, 0, 1);
}

int vgx_attn_block(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos, 1, qkv, out, 1, 1);
}

int vgx_attn_block_at(vgx_attn* a, int layer, const int* pos_dev, const int16_t* qkv, int16_t* out) {
    if (!pos_dev) return vgx_fail(VGX_EINVAL, "vgx_attn_block_at: NULL position");
    return launch(a, layer, 0, 1, qkv, out, 1, 1, false, pos_dev);
}

int vgx_attn_block_seqs(vgx_attn* a, int layer, int pos, int nseq, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos, nseq, qkv, out, 1, 1, true);
}

int vgx_kv_append_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv) {
    return launch(a, layer, pos0, ntok, qkv, nullptr, 1, 0);
}

int vgx_attn_decode_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos0, ntok, qkv, out, 0, 1);
}

int vgx_kv_row_bytes(const vgx_attn* a) { return a ? a->a.row_bytes : 0; }

// The planes' rows row0 .. row0+nrows-1 as texel rows: per position, K of
// every head in head order, then V of every head (q16 big-endian).
int vgx_kv_read_rows(vgx_attn* at, int layer, int row0, int nrows, void* host) {
    if (!at || !host) return vgx_fail(VGX_EINVAL, "vgx_kv_read_rows: NULL argument");
    if (layer < 0 || layer >= at->layers || !at->kv[layer]) return vgx_fail(VGX_ERANGE, "vgx_kv_read_rows: bad layer");
    if (row0 < 0 || nrows < 0 || row0 + nrows > at->a.seq) return vgx_fail(VGX_ERANGE, "vgx_kv_read_rows: rows outside the cache");
    if (nrows == 0) return VGX_OK;
    VGX_HIP(hipSetDevice(at->ctx->device));
    const AttnDev& A = at->a;
    const size_t ps = (size_t)A.pstride, np = 2 * (size_t)A.kv_heads;
    std::vector<uint8_t> planes(np * nrows * ps);  // [plane][row][ps]
    VGX_HIP(hipStreamSynchronize(at->ctx->stream));
    VGX_HIP(hipMemcpy2D(planes.data(), nrows * ps, at->kv[layer] + (size_t)row0 * ps, (size_t)A.seq * ps, nrows * ps, np,
                        hipMemcpyDeviceToHost));
    uint8_t* out = static_cast<uint8_t*>(host);
    for (int r = 0; r < nrows; ++r)
        for (size_t p = 0; p < np; ++p) {
            const uint8_t* src = planes.data() + (p * nrows + r) * ps;
            uint8_t* dst = out + (size_t)r * A.row_bytes + p * ps;
            if (A.kv_bits == 16)
                for (size_t i = 0; i < ps; i += 2) { dst[i] = src[i + 1]; dst[i + 1] = src[i]; }
            else
                memcpy(dst, src, ps);
        }
    return VGX_OK;
}

int vgx_kv_write_rows(vgx_attn* at, int layer, int row0, int nrows, const void* host) {
    if (!at || !host) return vgx_fail(VGX_EINVAL, "vgx_kv_write_rows: NULL argument");
    if (layer < 0 || layer >= at->layers || !at->kv[layer]) return vgx_fail(VGX_ERANGE, "vgx_kv_write_rows: bad layer");
    if (row0 < 0 || nrows < 0 || row0 + nrows > at->a.seq) return vgx_fail(VGX_ERANGE, "vgx_kv_write_rows: rows outside the cache");
    if (nrows == 0) return VGX_OK;
    VGX_HIP(hipSetDevice(at->ctx->device));
    const AttnDev& A = at->a;
    const size_t ps = (size_t)A.pstride, np = 2 * (size_t)A.kv_heads;
    std::vector<uint8_t> planes(np * nrows * ps);
    const uint8_t* in = static_cast<const uint8_t*>(host);
    for (int r = 0; r < nrows; ++r)
        for (size_t p = 0; p < np; ++p) {
            const uint8_t* src = in + (size_t)r * A.row_bytes + p * ps;
            uint8_t* dst = planes.data() + (p * nrows + r) * ps;
            if (A.kv_bits == 16)
                for (size_t i = 0; i < ps; i += 2) { dst[i] = src[i + 1]; dst[i + 1] = src[i]; }
            else
                memcpy(dst, src, ps);
        }
    VGX_HIP(hipStreamSynchronize(at->ctx->stream));
    VGX_HIP(hipMemcpy2D(at->kv[layer] + (size_t)row0 * ps, (size_t)A.seq * ps, planes.data(), nrows * ps, nrows * ps, np,
                        hipMemcpyHostToDevice));
    return VGX_OK;
}

}  // extern "C"
