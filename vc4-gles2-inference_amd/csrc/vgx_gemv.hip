// Dequant-GEMV kernels for gfx950: q8 (q8u8 bytes), q4 (g32 nibbles + int16
// scale/min planes) and t3 (2-bit ternary texel grid), batch 1.
//
// Mapping.  A block is 4 wave64s.  A wave owns RI x (64/LPR) rows: LPR lanes
// cooperate on one row and step through its 16-byte weight chunks (chunk
// c = lane + j*LPR), so one wave instruction reads 64 x 16 B of contiguous row
// segments.  The activation row is staged once per block in LDS, already split
// into the byte planes the dot instructions want:
//   x = 256*xh + xl,  xh = signed high byte, xl = unsigned low byte,
// so an int8 x int16 dot product becomes two 4-wide byte dots:
//   q8 : sum (u-128)*x = 256*sdot4(u^0x80, xh) + udot4(u, xl) - 128*sum(xl)
//   t3 : sum lv*x      = 256*sdot4(lv+1, xh) + udot4(lv+1, xl) - sum(x)
//   q4 : sum n*x       = 256*sdot4(n, xh)    + udot4(n, xl)         (per group)
// (lv+1 in {0,1,2} comes from a 256-entry byte -> 4 levels table in LDS.)
// q4 folds each group's scale and minimum in as integers too,
//   I = sum_g s16_g * D_g + m16_g * X_g   (int64, |I| < 2^47),
// so every row value is an exact integer times one fp32 scale, whatever the
// order the lanes add in.  The epilogue applies the reference's fp32
// scale/round/clamp with no contraction (this file is built with
// -ffp-contract=off).  Rows of a wave are reduced across their LPR lanes by a
// butterfly that halves the row set per step, so RI rows cost RI-1+log2(LPR)
// exchanges instead of RI*log2(LPR).
#include "vgx_internal.h"
#include "vgx_qrow.h"

#pragma clang fp contract(off)

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;


// quantize_act on the device: rint half-even of v*256, int16 rail.
__device__ __forceinline__ int q16_host(float v) {
    float r = __builtin_rintf(v * 256.0f);
    r = fminf(fmaxf(r, -32768.0f), 32767.0f);
    return (int)r;
}


template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int o) {
    return __shfl_xor(v, o, 64);
}

// Sums over the wave (integers, or integers held in doubles with every
// partial sum below 2^53: exact in any order): DPP exchanges within rows of 16 lanes
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
// then the four rows' totals by readlane.  Called with every lane active.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double readlane_d(double x, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ int wave_sum_i(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);
    return (__builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16)) +
           (__builtin_amdgcn_readlane(x, 32) + __builtin_amdgcn_readlane(x, 48));
}
__device__ __forceinline__ double wave_sum_d(double x) {
    x += dpp_d<0xB1>(x);
    x += dpp_d<0x4E>(x);
    x += dpp_d<0x141>(x);
    x += dpp_d<0x140>(x);
    return (readlane_d(x, 0) + readlane_d(x, 16)) + (readlane_d(x, 32) + readlane_d(x, 48));
}

// Global-memory views of the pointers in the launch descriptor.  The
// descriptor arrives by value, so the compiler cannot tell that its pointers
// address global memory and would emit flat accesses; a flat load also counts
// on the LDS wait counter, so every wait for an x-plane read from LDS would
// wait for the weight chunks still in flight as well.  Accesses through these
// views are global loads and stores (measured: q4 HBM-streamed launches +1.4
// points of peak, MiniMind3 decode +1%).
template <typename T>
using gmem_t = __attribute__((address_space(1))) T;
// LDS views, for rows the workgroup stages itself.
template <typename T>
using lmem_t = __attribute__((address_space(3))) T;
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
    return *(const gmem_t<T>*)p;
}
template <typename T>
__device__ __forceinline__ void gst(T* p, T v) {
    *(gmem_t<T>*)p = v;
}

// A 16-byte weight chunk, loaded with the nontemporal hint: every weight byte
// is read once per GEMV, so it should not displace reused lines (measured:
// +15% on HBM-streamed q8/q4 launches, no change on cache-resident decode).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 wload(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load((const gmem_t<u32x4_t>*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// The first matrix descriptor of the launch, read field by field through the
// kernel-argument segment (the launch descriptor is the kernel's only
// argument, at offset 0): scalar loads at fixed offsets.  Reading it through
// the by-value parameter would go through a generic pointer (the parameter's
// address is taken), i.e. vector loads the first weight load must wait for.
__device__ __forceinline__ MatDev kernarg_mat0() {
    typedef __attribute__((address_space(4))) GemvLaunch karg_t;
    const karg_t* K = (const karg_t*)__builtin_amdgcn_kernarg_segment_ptr();
    MatDev m;
    m.body = K->md[0].body;
    m.wsr = K->md[0].wsr;
    m.sm = K->md[0].sm;
    m.ps = K->md[0].ps;
    m.kind = K->md[0].kind;
    m.rows = K->md[0].rows;
    m.cols = K->md[0].cols;
    m.out_off = K->md[0].out_off;
    m.blk_off = K->md[0].blk_off;
    m.pad0 = m.pad1 = 0;
    return m;
}

// Which matrix / row block this block works on.
__device__ __forceinline__ int find_mat(const GemvLaunch& L, int blk) {
    if (L.nmat == 1) return 0;
    int lo = 0, hi = L.nmat - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        const int off = L.nmat <= kInlineMats ? L.md[mid].blk_off : gld(&L.mats[mid].blk_off);
        if (off <= blk) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Select a[r][c] for indices held in registers (unrolled compares, so the
// array stays in registers).
template <int R, int C, typename T>
__device__ __forceinline__ T pick(const T (&a)[R][C], int r, int c) {
    T v = a[0][0];
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
        for (int j = 0; j < C; ++j)
            if (r == k && c == j) v = a[k][j];
    return v;
}


// 4x4 byte transpose of dwords d[0..3] (each = two q16 values, even element
// low): returns the even-column low bytes, even high, odd low, odd high.
__device__ __forceinline__ void planes8eo(const uint32_t d[4], uint32_t& xle, uint32_t& xhe,
                                          uint32_t& xlo, uint32_t& xho) {
    uint32_t A = perm(d[1], d[0], 0x05010400u);
    uint32_t B = perm(d[1], d[0], 0x07030602u);
    uint32_t C = perm(d[3], d[2], 0x05010400u);
    uint32_t D = perm(d[3], d[2], 0x07030602u);
    xle = perm(C, A, 0x05040100u);
    xhe = perm(C, A, 0x07060302u);
    xlo = perm(D, B, 0x05040100u);
    xho = perm(D, B, 0x07060302u);
}


// Sixteen q16 values of x already in registers (two 16-byte loads), as
// load_x16 returns them.
__device__ __forceinline__ void x_regs(const u32x4_t a, const u32x4_t b, uint32_t d[8]) {
    d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
    d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
}

// Load 16 consecutive activations as q16 dwords: from int16, from f32 with
// the host quantisation, or through RMSNorm from the workgroup's LDS copies of
// x (xr) and the q16 norm weight (wr), inv = the row's inverse RMS.  Columns
// >= K read as zero.
template <int XM>
__device__ __forceinline__ void load_x16(const GemvLaunch& L, int col, int K, float inv, uint32_t d[8],
                                         const lmem_t<int16_t>* xr, const lmem_t<int16_t>* wr) {
    const gmem_t<int16_t>* x = (const gmem_t<int16_t>*)L.x;
    if (XM == X_RMS) {
        // from the workgroup's LDS copies of x and the norm weight
        if (col + 16 <= K) {
            const lmem_t<u32x4_t>* p = reinterpret_cast<const lmem_t<u32x4_t>*>(xr + col);
            const lmem_t<u32x4_t>* q = reinterpret_cast<const lmem_t<u32x4_t>*>(wr + col);
            const u32x4_t a = p[0], b = p[1], c = q[0], e = q[1];
            const uint32_t xd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            const uint32_t wd[8] = {c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w};
#pragma unroll
            for (int k = 0; k < 8; ++k)
                d[k] = rms_elem(xd[k] & 0xFFFFu, wd[k] & 0xFFFFu, inv) | (rms_elem(xd[k] >> 16, wd[k] >> 16, inv) << 16);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c0 = col + 2 * k;
                const uint32_t lo = c0 < K ? rms_elem((uint16_t)xr[c0], (uint16_t)wr[c0], inv) : 0u;
                const uint32_t hi = c0 + 1 < K ? rms_elem((uint16_t)xr[c0 + 1], (uint16_t)wr[c0 + 1], inv) : 0u;
                d[k] = lo | (hi << 16);
            }
        }
        return;
    }
    if (XM != X_F32) {
        if (col + 16 <= K) {
            const gmem_t<u32x4_t>* p = reinterpret_cast<const gmem_t<u32x4_t>*>(x + col);
            const u32x4_t a = p[0], b = p[1];
            d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w;
            d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                int c0 = col + 2 * k;
                uint32_t lo = c0 < K ? (uint16_t)x[c0] : 0u;
                uint32_t hi = c0 + 1 < K ? (uint16_t)x[c0 + 1] : 0u;
                d[k] = lo | (hi << 16);
            }
        }
    } else {
        const gmem_t<float>* xf = (const gmem_t<float>*)L.xf;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            int c0 = col + 2 * k;
            uint32_t lo = c0 < K ? (uint16_t)(int16_t)q16_host(xf[c0]) : 0u;
            uint32_t hi = c0 + 1 < K ? (uint16_t)(int16_t)q16_host(xf[c0 + 1]) : 0u;
            d[k] = lo | (hi << 16);
        }
    }
}

// t3 byte -> four (level + 1) bytes: code 1 -> 2, code 3 -> 0, else 1.
__device__ __forceinline__ uint32_t t3_lut_entry(uint32_t b) {
    uint32_t r = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t c = (b >> (2 * k)) & 3u;
        uint32_t lv1 = c == 1u ? 2u : (c == 3u ? 0u : 1u);
        r |= lv1 << (8 * k);
    }
    return r;
}

// ---------------------------------------------------------------------------
// Multi-row butterfly over the LPR lanes of a row segment.  v[r][k], r < R,
// k < NV.  After the call the lane seg_leader picks holds the complete sums
// of row `row` (the returned row slot) in v[0][*]: with several rows a lane,
// the lane whose segment index has zero low bits (cl % (LPR/R) == 0).
//
// One row a lane (R == 1), exact int32 or int64 sums: DPP moves instead of
// shuffles through the LDS crossbar (exchanges inside rows of 16 lanes --
// quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror -- then the row
// broadcasts of lane 15 into rows 1 and 3 and of lane 31 into rows 2 and 3).
// Every lane of a segment's last row of 16 then holds the segment's sums
// (seg_leader).  Integer sums: the pairing does not change the total.
template <int CTRL, int RM>
__device__ __forceinline__ int dpp_row(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, RM, 0xF, false);
}
template <int CTRL, int RM>
__device__ __forceinline__ long long dpp_row(long long x) {
    const unsigned long long b = (unsigned long long)x;
    const unsigned lo = (unsigned)dpp_row<CTRL, RM>((int)(unsigned)b);
    const unsigned hi = (unsigned)dpp_row<CTRL, RM>((int)(unsigned)(b >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}
template <int LPR, int R, typename T>
__device__ constexpr bool seg_dpp() {
    return R == 1 && (std::is_same<T, int>::value || std::is_same<T, long long>::value) && LPR >= 2 && LPR <= 64;
}
// The lane of a segment that holds its complete sums after seg_reduce.
template <int LPR, int R, typename T>
__device__ __forceinline__ bool seg_leader(int cl) {
    if (seg_dpp<LPR, R, T>()) return cl == (LPR <= 16 ? 0 : LPR - 16);
    return (cl % (LPR / R > 0 ? LPR / R : 1)) == 0;
}
template <int LPR, int R, int NV, typename T>
__device__ __forceinline__ int seg_reduce(T (&v)[R][NV], int cl) {
    if constexpr (seg_dpp<LPR, R, T>()) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            T x = v[0][k];
            if (LPR >= 2) x += dpp_row<0xB1, 0xF>(x);
            if (LPR >= 4) x += dpp_row<0x4E, 0xF>(x);
            if (LPR >= 8) x += dpp_row<0x141, 0xF>(x);
            if (LPR >= 16) x += dpp_row<0x140, 0xF>(x);
            if (LPR >= 32) x += dpp_row<0x142, 0xA>(x);
            if (LPR >= 64) x += dpp_row<0x143, 0xC>(x);
            v[0][k] = x;
        }
        return 0;
    }
    int base = 0;
    int m = R;
    int o = LPR / 2;
#pragma unroll
    for (int step = 0; (1 << step) < R; ++step) {
        const bool up = (cl & o) != 0;
        const int h = m / 2;
#pragma unroll
        for (int r = 0; r < R / 2; ++r) {
            if (r < h) {
#pragma unroll
                for (int k = 0; k < NV; ++k) {
                    T mine = up ? v[r + h][k] : v[r][k];
                    T other = up ? v[r][k] : v[r + h][k];
                    v[r][k] = mine + shfl_xor(other, o);
                }
            }
        }
        base += up ? h : 0;
        m = h;
        o >>= 1;
    }
    for (; o >= 1; o >>= 1) {
#pragma unroll
        for (int k = 0; k < NV; ++k) v[0][k] += shfl_xor(v[0][k], o);
    }
    return base;
}

// ---------------------------------------------------------------------------
// Per-format chunk math.


// q4: one chunk = one 32-column group (16 nibble bytes); planes per dword j:
// even-column high/low bytes and odd-column high/low bytes.
__device__ __forceinline__ int q4_chunk(const uint4 w, const uint4 xhe, const uint4 xle,
                                        const uint4 xho, const uint4 xlo) {
    int s1 = 0;
    uint32_t s2 = 0;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const uint32_t he[4] = {xhe.x, xhe.y, xhe.z, xhe.w}, le[4] = {xle.x, xle.y, xle.z, xle.w};
    const uint32_t ho[4] = {xho.x, xho.y, xho.z, xho.w}, lo[4] = {xlo.x, xlo.y, xlo.z, xlo.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t ne = wd[j] & 0x0F0F0F0Fu;
        uint32_t no = (wd[j] >> 4) & 0x0F0F0F0Fu;
        s1 = sdot4(ne, he[j], s1);
        s1 = sdot4(no, ho[j], s1);
        s2 = udot4(ne, le[j], s2);
        s2 = udot4(no, lo[j], s2);
    }
    return s1 * 256 + (int)s2;
}

// ---------------------------------------------------------------------------
// argmax_token (engine/src/sampling.cpp:160-162) fused into the LM-head
// launch.  A stored logit q at output row r is the key
//   (q + 32768) << 32 | (0xFFFFFFFF - r)
// so the largest key is the largest logit and, among equal logits, the first
// row.  Each workgroup reduces the keys of its rows and stores the largest in
// its own slot (argmax_key[blockIdx.x]); a one-workgroup launch on the same
// stream then reduces the slots and decodes the row.  No two workgroups touch
// one address and none waits for another: the launch boundary orders the
// slot stores before their reduction.
__device__ __forceinline__ unsigned long long argmax_key(int q, int row) {
    return ((unsigned long long)(unsigned)(q + 32768) << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)row);
}

// The largest key of the wave (unsigned; zero is the identity) in lane 63:
// DPP exchanges inside rows of 16 lanes, then the lane-15 and lane-31 row
// broadcasts (rows a mask leaves out read zero), as seg_reduce's sums.
__device__ __forceinline__ unsigned long long wave_max_key63(unsigned long long key) {
    auto step = [&](auto ctrl, auto rm) {
        const unsigned long long o = (unsigned long long)dpp_row<decltype(ctrl)::value, decltype(rm)::value>((long long)key);
        key = o > key ? o : key;
    };
    step(std::integral_constant<int, 0xB1>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x4E>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x141>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x140>{}, std::integral_constant<int, 0xF>{});
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xA>{});
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xC>{});
    return key;
}

__device__ __forceinline__ void argmax_tail(const GemvLaunch& L, unsigned long long key) {
    __shared__ unsigned long long s_k[kWaves];
    key = wave_max_key63(key);
    if ((threadIdx.x & 63) == 63) s_k[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        key = s_k[0];  // (lane 0 holds only its row's maximum)
        for (int k = 1; k < kWaves; ++k) key = s_k[k] > key ? s_k[k] : key;
        gst(L.argmax_key + blockIdx.x, key);
    }
}

// The largest of n keys (the first maximum of the rows they cover), one
// workgroup: its row index into *out.
__global__ void __launch_bounds__(256) argmax_keys_kernel(const unsigned long long* keys, int n, int* out,
                                                          const StepTail T) {
    __shared__ unsigned long long s_k[4];
    __shared__ int s_tok;
    // every argument in scalar registers first, one batch of loads (left to
    // the compiler they came in several dependent round trips); the loop
    // stride is the launch's 256 threads, not blockDim.x (an implicit
    // argument in a line of its own)
    asm volatile("" ::"s"(keys), "s"(n), "s"(out), "s"(T.pos), "s"(T.hist), "s"(T.hist_len), "s"(T.emb),
                 "s"(T.emb_scale), "s"(T.vocab), "s"(T.dim), "s"(T.x));
    // Every load that waits for nothing goes out in one batch: the position
    // (read by every lane from its uniform address: read by one lane, the
    // load was waited for before the keys issued; only this launch writes
    // it, at its end) and up to kKeysPer keys a thread from clamped addresses
    // (a repeat of the last key changes no maximum).  Issued one per loop
    // iteration, each 256 keys were a round trip of their own.
    constexpr int kKeysPer = 8;
    // (from a valid address either way: a load under the test was waited
    // for where the branch joined)
    int p = *(T.pos ? T.pos : reinterpret_cast<const int*>(keys));
    const int last = n > 0 ? n - 1 : 0;
    unsigned long long kv[kKeysPer];
#pragma unroll
    for (int j = 0; j < kKeysPer; ++j) kv[j] = keys[min((int)threadIdx.x + 256 * j, last)];
    unsigned long long key = 0ull;
#pragma unroll
    for (int j = 0; j < kKeysPer; ++j) key = kv[j] > key ? kv[j] : key;
    // (held here, past the keys it was issued before: left to the compiler
    // the load moved into the one lane's bookkeeping below)
    asm volatile("" : "+v"(p));
    for (int i = threadIdx.x + 256 * kKeysPer; i < n; i += 256) key = keys[i] > key ? keys[i] : key;
    key = wave_max_key63(key);
    if ((threadIdx.x & 63) == 63) s_k[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        key = s_k[0];  // (lane 0 holds only its row's maximum)
        for (int k = 1; k < 4; ++k) key = s_k[k] > key ? s_k[k] : key;
        const int tok = (int)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
        *out = tok;
        if (T.pos) {
            // the decode step's bookkeeping: the token joins the history at
            // position *pos + 1, and the position advances
            if (p + 1 >= 0 && p + 1 < T.hist_len) T.hist[p + 1] = tok;
            *T.pos = p + 1;
            s_tok = tok;
        }
    }
    if (!T.pos) return;
    __syncthreads();
    // the next step's input: the token's embedding row, as embed_q8_kernel
    // forms it (Session::embedding, engine/src/session.cpp:362-365); the
    // scale and up to kEmbPer bytes a thread load in one batch (clamped
    // addresses, the surplus never stored)
    constexpr int kEmbPer = 8;
    int tok = s_tok;
    if (tok < 0) tok = 0;
    if (tok >= T.vocab) tok = T.vocab - 1;
    const int8_t* er = T.emb + (size_t)tok * T.dim;
    const int dlast = T.dim > 0 ? T.dim - 1 : 0;
    const float sc = T.emb_scale[tok];
    int8_t ev[kEmbPer];
#pragma unroll
    for (int j = 0; j < kEmbPer; ++j) ev[j] = er[min((int)threadIdx.x + 256 * j, dlast)];
    auto put = [&](int i, int8_t e) {
        const float v = (float)e * sc;
        float r = __builtin_rintf(v * 256.0f);
        r = fminf(fmaxf(r, -32768.0f), 32767.0f);
        T.x[i] = (int16_t)r;
    };
#pragma unroll
    for (int j = 0; j < kEmbPer; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < T.dim) put(i, ev[j]);
    }
    for (int i = threadIdx.x + 256 * kEmbPer; i < T.dim; i += 256) put(i, er[i]);
}

// Dynamic LDS of a launch: the x planes (q8: 32 B per 16 columns; t3 and
// q4: 64 B per 32 columns), then t3's level table or q4's per-group x sums,
// then (X_RMS) the copies of x and of the norm weight, 16-byte aligned.
__host__ __device__ inline size_t lds_bytes(int kind, int cols, int xm) {
    size_t b = kind == VGX_Q8 ? (size_t)(cols / 16) * 32
               : kind == VGX_T3 ? (size_t)t3_chunks(cols) * 64 + 256 * 4
                                : (size_t)(cols / 32) * 64 + (size_t)(cols / 32) * 4;
    b = (b + 15) & ~(size_t)15;
    return xm == X_RMS ? b + (size_t)((cols + 7) & ~7) * 4 : b;
}

// ---------------------------------------------------------------------------
// The kernel.  One template per (format, lanes per row, rows per lane,
// epilogue, input type).
//
// LDS layout (dynamic): [planes][scalars]
//   q8 : per 16-col chunk: xh (16 B), xl (16 B)                    -> 32 B/chunk
//   t3 : per 32-col chunk: xh (32 B), xl (32 B)  (natural order)    -> 64 B/chunk
//   q4 : per 32-col group: xhe, xle, xho, xlo (16 B each)           -> 64 B/group
//        plus X_g (int32) per group
//   t3 : + 256 u32 level table
template <int KIND, int LPR, int RI, int EPI, int XM, bool ONE>
__global__ void __launch_bounds__(kThreads) gemv_kernel(const GemvLaunch L) {
    extern __shared__ uint4 lds[];
    // Every kernel argument the launch reads, in scalar registers before
    // anything else: the argument loads then go out as one batch.  Left to
    // the compiler, the arguments past the matrix descriptor came in two more
    // round trips, the x pointer's after the workgroup's first barrier.
    // (one statement: a wait for its operands covers the whole batch; fields
    // a variant does not read are constants here)
    {
        const MatDev m0 = ONE ? kernarg_mat0() : MatDev{};
        const void* xin = XM == X_F32 ? (const void*)L.xf : (const void*)L.x;
        const int16_t* rw0 = XM == X_RMS ? L.rw : nullptr;
        const float eps0 = XM == X_RMS ? L.eps : 0.0f;
        const int hs0 = EPI == EPI_GATE ? L.hs : 0;
        const uint8_t* b3 = EPI == EPI_GATE ? L.md3.body : nullptr;
        const float* w3 = EPI == EPI_GATE ? L.md3.wsr : nullptr;
        const uint32_t* s3 = EPI == EPI_GATE ? L.md3.sm : nullptr;
        const float p3 = EPI == EPI_GATE ? L.md3.ps : 0.0f;
        const int sc0 = EPI == EPI_SPLIT ? L.split_chunk : 0;
        asm volatile("" ::"s"(L.cols), "s"(L.blocks), "s"(L.grid), "s"(L.res), "s"(L.y), "s"(xin), "s"(rw0),
                     "s"(eps0), "s"(hs0), "s"(b3), "s"(w3), "s"(s3), "s"(p3), "s"(sc0), "s"(m0.body), "s"(m0.wsr),
                     "s"(m0.sm), "s"(m0.ps), "s"(m0.rows), "s"(m0.out_off), "s"(m0.blk_off));
    }
    constexpr int RPI = 64 / LPR;
    constexpr int NV = (EPI == EPI_GATE || EPI == EPI_SPLIT) ? 2 : 1;
    // rows a wave owns: t3 counts row *pairs*
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rs = lane / LPR;
    const int cl = lane % LPR;

    // Every matrix of a launch has K = L.cols columns and reads the same x.
    const int K = L.cols;
    constexpr int RPU = KIND == VGX_T3 ? 2 : 1;  // rows per unit
    const MatDev M3 = L.md3;  // W3 of the gate epilogue (single-matrix launches)

    // --- weight chunk geometry
    const int nch = KIND == VGX_Q8 ? (K >> 4) : KIND == VGX_T3 ? t3_chunks(K) : (K >> 5);
    const size_t ustride = KIND == VGX_Q8 ? (size_t)K : KIND == VGX_Q4 ? (size_t)q4_rstride(K)
                                                                     : (size_t)t3_rstride(K);
    const uint8_t* body3 = (EPI == EPI_GATE) ? M3.body : nullptr;
    const int niter = (nch + LPR - 1) / LPR;

    // A workgroup takes row tiles blockIdx.x, blockIdx.x + L.grid, ...;
    // x is staged once for all of them.  Per tile: the matrix descriptor (by
    // value in the launch arguments for up to kInlineMats matrices, else from
    // the device table), the tile's first weight chunk, and -- for one row per
    // lane only -- the epilogue's per-row operands (row scales, residual), so
    // their latency hides under the main loop.  With RI rows per lane those
    // registers would cost occupancy, which the streaming launches need more.
    // With one row per lane (the latency-bound decode shapes) a lane's first
    // NPF chunks all go out in begin_tile, and each chunk consumed is
    // replaced by the one NPF chunks ahead: one memory round trip per tile
    // instead of one per chunk.  Those loads read clamped in-range addresses
    // unconditionally (a chunk or row past the end is computed and dropped):
    // a predicated load would be waited for before the next one is issued.
    constexpr bool PF = RI == 1;
    constexpr int NPF = PF ? 4 : 1;
    // q4 rows lie back to back in HBM (cols/2 bytes each), so consecutive
    // rows share a cache line where a row ends mid line (768 x 2432: 1216-byte
    // rows).  Odd rows walk their chunks last to first: the last chunk of row
    // 2p and the first of row 2p+1 (and the last of 2p+1 and the first of
    // 2p+2) are then loaded by the same instruction, so the shared line is
    // fetched once.  (A row's sum is exact, so its chunk order does not
    // change the result.)  A lane's row slots share one parity when RPI is
    // even, so they keep sharing the x planes of a chunk.
    constexpr bool SNAKE = KIND == VGX_Q4 && (RI == 1 || RPI % 2 == 0);
    bool rev = false;  // SNAKE: this lane's rows are odd
    auto chk = [&](int c) { return (SNAKE && rev) ? nch - 1 - c : c; };
    MatDev M;
    int units = 0, unit0 = 0;
    const uint8_t* body = nullptr;
    float pw[RI][RPU], pw3[RI][RPU];
    int pres[RI][RPU];
    uint4 w[RI], w3[RI];
    uint32_t smv[RI], smv3[RI];
    uint4 pb[NPF], pb3[NPF];     // PF: the lane's chunks cl + s*LPR (+ k*NPF*LPR)
    uint32_t psm[NPF], psm3[NPF];  // PF, q4: their scale/min words
    auto pf_load = [&](int s, int c) {
        const int u = min(unit0 + rs, units - 1);
        const int cc = chk(min(c, nch - 1));
        pb[s] = wload(body + (size_t)u * ustride + (size_t)cc * 16);
        if (EPI == EPI_GATE) pb3[s] = wload(body3 + (size_t)u * ustride + (size_t)cc * 16);
        if (KIND == VGX_Q4) {
            psm[s] = gld(M.sm + (size_t)u * nch + cc);
            if (EPI == EPI_GATE) psm3[s] = gld(M3.sm + (size_t)u * nch + cc);
        }
    };
    auto begin_tile = [&](int tile) {
        // ONE, a single-matrix launch (every decode GEMV but the LM head):
        // the descriptor at fixed kernel-argument offsets, scalar loads in
        // one batch at entry, instead of a matrix search and a descriptor
        // fetch through an index (measured: up to 0.8 us before the first
        // weight load)
        if (ONE) {
            M = kernarg_mat0();
        } else {
            const int mi = L.bpm > 0 ? tile / L.bpm : find_mat(L, tile);
            M = L.nmat <= kInlineMats ? L.md[mi] : L.mats[mi];
        }
        units = KIND == VGX_T3 ? (M.rows + 1) / 2 : M.rows;
        unit0 = (tile - M.blk_off) * (kWaves * RPI * RI) + wave * (RPI * RI);
        rev = SNAKE && ((unit0 + rs) & 1) != 0;
        body = M.body;
#pragma unroll
        for (int it = 0; it < (PF ? RI : 0); ++it) {
#pragma unroll
            for (int hr = 0; hr < RPU; ++hr) {
                // clamped rows: a row past the end is never stored
                const int row = min((unit0 + it * RPI + rs) * RPU + hr, M.rows - 1);
                pw[it][hr] = KIND != VGX_Q4 ? gld(M.wsr + row) : 0.0f;
                pw3[it][hr] = (KIND != VGX_Q4 && EPI == EPI_GATE) ? gld(M3.wsr + row) : 0.0f;
                const bool has_res = (EPI == EPI_STORE || EPI == EPI_STORE_ARGMAX || EPI == EPI_SPLIT) && L.res;
                pres[it][hr] = has_res ? (int)gld(L.res + M.out_off + row) : 0;
            }
        }
        if (PF) {
#pragma unroll
            for (int s = 0; s < NPF; ++s) pf_load(s, cl + s * LPR);
            return;
        }
#pragma unroll
        for (int it = 0; it < RI; ++it) {
            const int u = unit0 + it * RPI + rs;
            const int c = cl;
            const int ca = chk(c);  // the chunk in memory (q4: odd rows reversed)
            const bool ok = u < units && c < nch;
            w[it] = ok ? wload(body + (size_t)u * ustride + (size_t)ca * 16)
                       : make_uint4(0, 0, 0, 0);
            if (EPI == EPI_GATE)
                w3[it] = ok ? wload(body3 + (size_t)u * ustride + (size_t)ca * 16)
                            : make_uint4(0, 0, 0, 0);
            if (KIND == VGX_Q4) {
                smv[it] = ok ? gld(M.sm + (size_t)u * nch + ca) : 0u;
                if (EPI == EPI_GATE) smv3[it] = ok ? gld(M3.sm + (size_t)u * nch + ca) : 0u;
            }
        }
    };

    // --- stage x planes (and the row-independent sums) in LDS
    // the byte split's bias sums, per column half (the split epilogue adds the
    // two halves separately; every other epilogue uses their total)
    __shared__ int s_xpart[kWaves][2];  // each wave's share of the two sums (no clearing, no atomics)
    uint32_t* lut = nullptr;
    int* xg = nullptr;
    const int plane_u4 = KIND == VGX_Q8 ? 2 * nch : 4 * nch;  // uint4 per plane block
    if (KIND == VGX_T3) {
        lut = reinterpret_cast<uint32_t*>(lds + plane_u4);
        for (int b = threadIdx.x; b < 256; b += kThreads) lut[b] = t3_lut_entry((uint32_t)b);
    }
    if (KIND == VGX_Q4) xg = reinterpret_cast<int*>(lds + plane_u4);
    // X_RMS: x and the norm weight are read from global memory once, 16 bytes
    // of each per thread, into LDS (after the planes); the statistics and the
    // normalised planes below read the copies (measured: the second global
    // read of x and the weight cost ~1 us per launch on the decode shapes)
    //
    // RMSNorm statistics (rms_stats_split, engine/src/gpu_upload.cpp:280-365):
    // 32 partial sums of x^2 over contiguous slices of ceil(K/32) values, each
    // stored as floor(P/16 + 1/2).  When K is a multiple of 256 (a slice is
    // whole 8-value pieces of the copy; at most kRmsPieces of them), each
    // thread's sum of squares over the piece it copied goes to LDS with the
    // copy, and after the copy's barrier lane p of every wave adds slice p's
    // pieces and every wave the rounded slices (exact integers): no second
    // pass over the copy and no second barrier.  Otherwise 8 lanes per slice
    // from the copy, then every thread adds the 32 slices.
    constexpr int kRmsPieces = 512;
    __shared__ long long s_rms[32];
    __shared__ long long s_rpiece[kRmsPieces];
    const bool rms_fast = XM == X_RMS && K % 256 == 0 && K / 8 <= kRmsPieces;
    lmem_t<int16_t>* xr = nullptr;
    lmem_t<int16_t>* wr = nullptr;
    // rms_fast: thread t holds pieces t and t + kThreads (columns 8i..8i+7)
    // of x and of the norm weight in registers from the load to the planes
    const int npieces = K / 8;
    u32x4_t rxa[kRmsPieces / kThreads], rwa[kRmsPieces / kThreads];
    // x (and the norm weight) go out first, the first tile's weight chunks
    // right after: loads complete in the order they are issued, so the wait
    // for x is not a wait for the weights (whose latency still overlaps the
    // staging).  Without the fused norm a thread's first chunk of x is loaded
    // here when it is a whole chunk (q8, q4: always; t3: all but a short last
    // chunk), and the staging below takes it from these registers.
    const int xcw = KIND == VGX_Q8 ? 16 : 32;  // x columns a chunk
    const int xc0 = min((int)threadIdx.x, nch - 1);
    const bool xpre = XM == X_I16 && (int)threadIdx.x < nch && (xc0 + 1) * xcw <= K;
    u32x4_t xp[4];
    if (XM == X_I16 && K >= xcw) {
        // (a clamped whole chunk: every thread loads, a thread past the
        // chunks or at a short last chunk discards it)
        const u32x4_t* p = reinterpret_cast<const u32x4_t*>(L.x + (size_t)min(xc0 * xcw, K - xcw));
        xp[0] = gld(p);
        xp[1] = gld(p + 1);
        if (KIND != VGX_Q8) {
            xp[2] = gld(p + 2);
            xp[3] = gld(p + 3);
        }
    }
    if (XM == X_RMS && rms_fast) {
#pragma unroll
        for (int it = 0; it < kRmsPieces / kThreads; ++it) {
            if (it * kThreads >= npieces) break;
            const int i = min((int)threadIdx.x + it * kThreads, npieces - 1);
            rxa[it] = gld(reinterpret_cast<const u32x4_t*>(L.x + 8 * i));
            rwa[it] = gld(reinterpret_cast<const u32x4_t*>(L.rw + 8 * i));
        }
    }
    begin_tile(blockIdx.x);
    if (XM == X_RMS && rms_fast) {
#pragma unroll
        for (int it = 0; it < kRmsPieces / kThreads; ++it) {
            const int i = (int)threadIdx.x + it * kThreads;
            if (i >= npieces) break;
            long long P = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const long long lo = (int16_t)(rxa[it][k] & 0xFFFFu), hi = (int16_t)(rxa[it][k] >> 16);
                P += lo * lo + hi * hi;
            }
            s_rpiece[i] = P;
        }
        __syncthreads();
    } else if (XM == X_RMS) {
        xr = (lmem_t<int16_t>*)(reinterpret_cast<uint8_t*>(lds) + lds_bytes(KIND, K, X_I16));
        wr = xr + ((K + 7) & ~7);
        for (int i = threadIdx.x * 8; i < K; i += kThreads * 8) {
            const u32x4_t a = gld(reinterpret_cast<const u32x4_t*>(L.x + i));
            const u32x4_t b = gld(reinterpret_cast<const u32x4_t*>(L.rw + i));
            *reinterpret_cast<lmem_t<u32x4_t>*>(xr + i) = a;
            *reinterpret_cast<lmem_t<u32x4_t>*>(wr + i) = b;
        }
        __syncthreads();
    }
    if (XM == X_RMS && !rms_fast) {
        const int per = (K + 31) / 32;
        const int p = threadIdx.x >> 3, sub = threadIdx.x & 7;
        long long P = 0;
        for (int k = sub; k < per; k += 8) {
            const int i = p * per + k;
            if (i < K) {
                const long long xi = xr[i];
                P += xi * xi;
            }
        }
        for (int o = 4; o >= 1; o >>= 1) P += shfl_xor(P, o);
        if (sub == 0) s_rms[p] = (P + 8) >> 4;
    }
    if (XM == X_RMS && !rms_fast) __syncthreads();
    float rinv = 0.0f;
    if (XM == X_RMS) {
        long long tot = 0;
        if (rms_fast) {
            const int pps = K / 256;  // pieces per slice
            long long t = 0;
            if (lane < 32) {
                long long P = 0;
                if (pps <= 4) {
                    // every piece read before the first add (exact integers:
                    // the order is free), not one read waited for at a time
                    long long q[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) q[k] = s_rpiece[lane * pps + min(k, pps - 1)];
#pragma unroll
                    for (int k = 0; k < 4; ++k) P += k < pps ? q[k] : 0;
                } else {
                    for (int k = 0; k < pps; ++k) P += s_rpiece[lane * pps + k];
                }
                t = (P + 8) >> 4;
            }
            // the 32 rounded slices (each below 2^32) added as doubles: every
            // partial sum is an integer below 2^53, so the DPP row sums and
            // the four rows' readlanes give the exact total (six dependent
            // 64-bit cross-lane shuffles took longer)
            tot = (long long)wave_sum_d((double)t);
        } else {
            for (int p = 0; p < 32; ++p) tot += s_rms[p];
        }
        const float ss = (float)tot / 4096.0f;
        rinv = (float)(1.0 / sqrt((double)(ss / (float)K + L.eps)));
    }
    int part[2] = {0, 0};
    if (XM == X_RMS && rms_fast) {
        // each thread normalises the pieces it holds (rms_elem, as load_x16
        // does) and writes their bytes into the plane layout: q8 chunk i/2
        // half i%2; t3 chunk i/4, sixteen-column half (i/2)%2, eight-byte
        // half i%2; q4 group i/4, dword i%4 of each of its four planes (the
        // even/odd split of planes8eo), the group's x sum joined over its
        // four pieces' threads
#pragma unroll
        for (int it = 0; it < kRmsPieces / kThreads; ++it) {
            if (it * kThreads >= npieces) break;
            const int i = (int)threadIdx.x + it * kThreads;
            const bool ok = i < npieces;
            uint32_t d[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                d[k] = rms_elem(rxa[it][k] & 0xFFFFu, rwa[it][k] & 0xFFFFu, rinv) |
                       (rms_elem(rxa[it][k] >> 16, rwa[it][k] >> 16, rinv) << 16);
            if (KIND == VGX_Q4) {
                const int c = i >> 2, q = i & 3;
                uint32_t le, he, lo, ho;
                planes8eo(d, le, he, lo, ho);
                int X = 256 * (sdot4(he, 0x01010101u, 0) + sdot4(ho, 0x01010101u, 0)) +
                        (int)(udot4(le, 0x01010101u, 0u) + udot4(lo, 0x01010101u, 0u));
                X = ok ? X : 0;
                X += dpp_row<0xB1, 0xF>(X);  // the quad's four pieces (lanes 4c'..4c'+3)
                X += dpp_row<0x4E, 0xF>(X);
                if (ok) {
                    reinterpret_cast<uint32_t*>(&lds[4 * c + 0])[q] = he;
                    reinterpret_cast<uint32_t*>(&lds[4 * c + 1])[q] = le;
                    reinterpret_cast<uint32_t*>(&lds[4 * c + 2])[q] = ho;
                    reinterpret_cast<uint32_t*>(&lds[4 * c + 3])[q] = lo;
                    if (q == 0) xg[c] = X;
                }
            } else if (ok) {
                const uint2 xh = make_uint2(perm(d[1], d[0], 0x07050301u), perm(d[3], d[2], 0x07050301u));
                const uint2 xl = make_uint2(perm(d[1], d[0], 0x06040200u), perm(d[3], d[2], 0x06040200u));
                if (KIND == VGX_Q8) {
                    const int c = i >> 1, hf = i & 1;
                    const int hh = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
                    reinterpret_cast<uint2*>(&lds[2 * c])[hf] = xh;
                    reinterpret_cast<uint2*>(&lds[2 * c + 1])[hf] = xl;
                    part[hh] = (int)udot4(xl.y, 0x01010101u, udot4(xl.x, 0x01010101u, (uint32_t)part[hh]));
                } else {  // T3
                    const int c = i >> 2, q = i & 3;
                    const int hh = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
                    reinterpret_cast<uint2*>(&lds[4 * c + (q >> 1)])[q & 1] = xh;
                    reinterpret_cast<uint2*>(&lds[4 * c + 2 + (q >> 1)])[q & 1] = xl;
                    part[hh] += 256 * (sdot4(xh.x, 0x01010101u, 0) + sdot4(xh.y, 0x01010101u, 0)) +
                                (int)(udot4(xl.x, 0x01010101u, 0u) + udot4(xl.y, 0x01010101u, 0u));
                }
            }
        }
    } else if (KIND == VGX_Q8) {
        for (int c = threadIdx.x; c < nch; c += kThreads) {
            const int hh = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
            uint32_t d[8], xh[4], xl[4];
            if (XM == X_I16 && xpre && c == (int)threadIdx.x) x_regs(xp[0], xp[1], d);
            else load_x16<XM>(L, c * 16, K, rinv, d, xr, wr);
            planes16(d, xh, xl);
            lds[2 * c] = make_uint4(xh[0], xh[1], xh[2], xh[3]);
            lds[2 * c + 1] = make_uint4(xl[0], xl[1], xl[2], xl[3]);
            for (int k = 0; k < 4; ++k) part[hh] = (int)udot4(xl[k], 0x01010101u, (uint32_t)part[hh]);
        }
    } else if (KIND == VGX_T3) {
        for (int c = threadIdx.x; c < nch; c += kThreads) {
            const int hh = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
            uint32_t d[8], xh[4], xl[4], xh2[4], xl2[4];
            const bool fx = XM == X_I16 && xpre && c == (int)threadIdx.x;
            if (fx) x_regs(xp[0], xp[1], d);
            else load_x16<XM>(L, c * 32, K, rinv, d, xr, wr);
            planes16(d, xh, xl);
            if (fx) x_regs(xp[2], xp[3], d);
            else load_x16<XM>(L, c * 32 + 16, K, rinv, d, xr, wr);
            planes16(d, xh2, xl2);
            lds[4 * c + 0] = make_uint4(xh[0], xh[1], xh[2], xh[3]);
            lds[4 * c + 1] = make_uint4(xh2[0], xh2[1], xh2[2], xh2[3]);
            lds[4 * c + 2] = make_uint4(xl[0], xl[1], xl[2], xl[3]);
            lds[4 * c + 3] = make_uint4(xl2[0], xl2[1], xl2[2], xl2[3]);
            for (int k = 0; k < 4; ++k) {
                part[hh] += 256 * sdot4(xh[k], 0x01010101u, 0) + (int)udot4(xl[k], 0x01010101u, 0u);
                part[hh] += 256 * sdot4(xh2[k], 0x01010101u, 0) + (int)udot4(xl2[k], 0x01010101u, 0u);
            }
        }
    } else {  // Q4
        for (int c = threadIdx.x; c < nch; c += kThreads) {
            uint32_t d[8], d2[8];
            if (XM == X_I16 && xpre && c == (int)threadIdx.x) {
                x_regs(xp[0], xp[1], d);
                x_regs(xp[2], xp[3], d2);
            } else {
                load_x16<XM>(L, c * 32, K, rinv, d, xr, wr);
                load_x16<XM>(L, c * 32 + 16, K, rinv, d2, xr, wr);
            }
            uint32_t he[4], le[4], ho[4], lo[4];
            const uint32_t q0[4] = {d[0], d[1], d[2], d[3]}, q1[4] = {d[4], d[5], d[6], d[7]};
            const uint32_t q2[4] = {d2[0], d2[1], d2[2], d2[3]}, q3[4] = {d2[4], d2[5], d2[6], d2[7]};
            planes8eo(q0, le[0], he[0], lo[0], ho[0]);
            planes8eo(q1, le[1], he[1], lo[1], ho[1]);
            planes8eo(q2, le[2], he[2], lo[2], ho[2]);
            planes8eo(q3, le[3], he[3], lo[3], ho[3]);
            lds[4 * c + 0] = make_uint4(he[0], he[1], he[2], he[3]);
            lds[4 * c + 1] = make_uint4(le[0], le[1], le[2], le[3]);
            lds[4 * c + 2] = make_uint4(ho[0], ho[1], ho[2], ho[3]);
            lds[4 * c + 3] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            int X = 0;
            for (int k = 0; k < 4; ++k) {
                X += 256 * (sdot4(he[k], 0x01010101u, 0) + sdot4(ho[k], 0x01010101u, 0));
                X += (int)(udot4(le[k], 0x01010101u, 0u) + udot4(lo[k], 0x01010101u, 0u));
            }
            xg[c] = X;
        }
    }
    if (KIND != VGX_Q4) {
        const int p0 = wave_sum_i(part[0]), p1 = EPI == EPI_SPLIT ? wave_sum_i(part[1]) : 0;
        if (lane == 0) {
            s_xpart[wave][0] = p0;
            s_xpart[wave][1] = p1;
        }
    }
    __syncthreads();
    int xs0 = 0, xs1 = 0;
    if (KIND != VGX_Q4) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            xs0 += s_xpart[w][0];
            xs1 += s_xpart[w][1];
        }
    }

    unsigned long long akey = 0ull;  // EPI_STORE_ARGMAX: this lane's best key
    for (int tile = blockIdx.x;;) {
    // --- main loop
    if (KIND == VGX_Q4) {
        long long acc[RI][NV];
#pragma unroll
        for (int it = 0; it < RI; ++it)
#pragma unroll
            for (int k = 0; k < NV; ++k) acc[it][k] = 0;
        const float ps = M.ps;
        const float ps3 = (EPI == EPI_GATE) ? M3.ps : 0.0f;
        // one chunk c of row slot it: weights wv, scale/min word sm (and the
        // gate's second matrix); |D| < 2^24, |X| <= 2^20
        auto q4_step = [&](int it, int c, const uint4 wv, uint32_t sm, const uint4 wv3, uint32_t sm3) {
            const uint4 xhe = lds[4 * c], xle = lds[4 * c + 1], xho = lds[4 * c + 2], xlo = lds[4 * c + 3];
            const int Xg = xg[c];
            const int kk = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
            const int D = q4_chunk(wv, xhe, xle, xho, xlo);
            const long long t = (long long)(int16_t)(sm & 0xFFFFu) * D + (long long)(int16_t)(sm >> 16) * Xg;
            if (EPI == EPI_SPLIT) {
                if (kk) acc[it][NV - 1] += t; else acc[it][0] += t;
            } else {
                acc[it][0] += t;
            }
            if (EPI == EPI_GATE) {
                const int D3 = q4_chunk(wv3, xhe, xle, xho, xlo);
                acc[it][NV - 1] += (long long)(int16_t)(sm3 & 0xFFFFu) * D3 + (long long)(int16_t)(sm3 >> 16) * Xg;
            }
        };
        if (PF) {
            for (int j0 = 0; j0 < niter; j0 += NPF) {
#pragma unroll
                for (int s = 0; s < NPF; ++s) {
                    const int c = cl + (j0 + s) * LPR;
                    if (c < nch) q4_step(0, chk(c), pb[s], psm[s], pb3[s], psm3[s]);
                    if (j0 + s + NPF < niter) pf_load(s, c + NPF * LPR);
                }
            }
        }
        for (int j = 0; j < (PF ? 0 : niter); ++j) {
            const int c = cl + j * LPR;
            const bool cok = c < nch;
            uint4 wn[RI], wn3[RI];
            uint32_t sn[RI], sn3[RI];
            const bool more = j + 1 < niter;
            if (more) {
#pragma unroll
                for (int it = 0; it < RI; ++it) {
                    const int u = unit0 + it * RPI + rs;
                    const int cn = c + LPR;
                    const int ca = chk(cn);
                    const bool ok = u < units && cn < nch;
                    wn[it] = ok ? wload(body + (size_t)u * ustride + (size_t)ca * 16)
                                : make_uint4(0, 0, 0, 0);
                    sn[it] = ok ? gld(M.sm + (size_t)u * nch + ca) : 0u;
                    if (EPI == EPI_GATE) {
                        wn3[it] = ok ? wload(body3 + (size_t)u * ustride + (size_t)ca * 16)
                                     : make_uint4(0, 0, 0, 0);
                        sn3[it] = ok ? gld(M3.sm + (size_t)u * nch + ca) : 0u;
                    }
                }
            }
            if (cok) {
#pragma unroll
                for (int it = 0; it < RI; ++it) q4_step(it, chk(c), w[it], smv[it], w3[it], smv3[it]);
            }
            if (more) {
#pragma unroll
                for (int it = 0; it < RI; ++it) {
                    w[it] = wn[it];
                    smv[it] = sn[it];
                    if (EPI == EPI_GATE) { w3[it] = wn3[it]; smv3[it] = sn3[it]; }
                }
            }
        }
        const int row_it = seg_reduce<LPR, RI, NV, long long>(acc, cl);
        if (seg_leader<LPR, RI, long long>(cl)) {
            const int u = unit0 + row_it * RPI + rs;
            if (u < units) {
                const float v = (float)acc[0][0] * ps;
                const float rv = PF ? (float)pick(pres, row_it, 0)
                                    : (L.res ? (float)gld(L.res + M.out_off + u) : 0.0f);
                if (EPI == EPI_STORE || EPI == EPI_STORE_ARGMAX) {
                    const float t = L.res ? v + rv : v;
                    const int q = q16_round(t);
                    gst(static_cast<int16_t*>(L.y) + M.out_off + u, (int16_t)q);
                    if (EPI == EPI_STORE_ARGMAX) {
                        const unsigned long long k = argmax_key(q, M.out_off + u);
                        akey = k > akey ? k : akey;
                    }
                } else if (EPI == EPI_STORE_F32) {
                    gst(static_cast<float*>(L.y) + M.out_off + u, v * (1.0f / 256.0f));
                } else if (EPI == EPI_SPLIT) {
                    const float vb = (float)acc[0][NV - 1] * ps;
                    const float t = v + rv;
                    const float y1 = (float)q16_round(t);
                    gst(static_cast<int16_t*>(L.y) + u, (int16_t)q16_round(vb + y1));
                } else {  // gate
                    const float vb = (float)acc[0][NV - 1] * ps3;
                    const float g = (float)q16_round(v), uu = (float)q16_round(vb);
                    const float a = g / 256.0f;
                    const float e = (float)exp(-(double)a);
                    const float dn = 1.0f + e;
                    const float r = a / dn;
                    float o = r * (uu / 256.0f);
                    o = o * ldexpf(1.0f, -L.hs);
                    gst(static_cast<int16_t*>(L.y) + u, (int16_t)q16_round(o * 256.0f));
                }
            }
        }
    } else {
    // q8 and t3: exact int32 partial sums.  t3 carries two rows (a pair) per unit.
    constexpr int ROWS_PER_UNIT = KIND == VGX_T3 ? 2 : 1;
    constexpr int NI = 2 * NV * ROWS_PER_UNIT;  // ints per unit: (s1, s2) per row per half
    int acc[RI][NI];
#pragma unroll
    for (int it = 0; it < RI; ++it)
#pragma unroll
        for (int k = 0; k < NI; ++k) acc[it][k] = 0;

    // one chunk c of row slot it: weights wa (and wb, the gate's second matrix)
    auto step = [&](int it, int c, const uint4 wa, const uint4 wb) {
        // column half for the split epilogue
        const int hb = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 1 : 0;
        if (KIND == VGX_Q8) {
            const uint4 xh = lds[2 * c], xl = lds[2 * c + 1];
            int s1 = 0;
            uint32_t s2 = 0;
            q8_chunk(wa, xh, xl, s1, s2);
            const int o = 2 * hb;
            acc[it][o] += s1;
            acc[it][o + 1] += (int)s2;
            if (EPI == EPI_GATE) {
                int t1 = 0;
                uint32_t t2 = 0;
                q8_chunk(wb, xh, xl, t1, t2);
                acc[it][2] += t1;
                acc[it][3] += (int)t2;
            }
        } else {  // T3: 4 texels = 32 columns of a row pair
            const uint4 xh0 = lds[4 * c], xh1 = lds[4 * c + 1];
            const uint4 xl0 = lds[4 * c + 2], xl1 = lds[4 * c + 3];
            const uint32_t xh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
            const uint32_t xl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
            // every table entry of the chunk (both matrices) is read before
            // the first product: left to the scheduler the lookups went out a
            // few at a time, each group waited for in turn (one chunk a lane
            // at the decode shapes, so nothing else covered those waits)
            constexpr int NM = EPI == EPI_GATE ? 2 : 1;
            uint32_t lv[NM][16];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint4 wv = m == 0 ? wa : wb;
                const uint32_t td[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int b = 0; b < 4; ++b) lv[m][4 * t + b] = lut[(td[t] >> (8 * b)) & 0xFFu];
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                int a1 = 0, b1 = 0;
                uint32_t a2 = 0, b2 = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t l0 = lv[m][4 * t], l1 = lv[m][4 * t + 1];
                    const uint32_t l2 = lv[m][4 * t + 2], l3 = lv[m][4 * t + 3];
                    a1 = sdot4(l0, xh[2 * t], a1);
                    a1 = sdot4(l1, xh[2 * t + 1], a1);
                    a2 = udot4(l0, xl[2 * t], a2);
                    a2 = udot4(l1, xl[2 * t + 1], a2);
                    b1 = sdot4(l2, xh[2 * t], b1);
                    b1 = sdot4(l3, xh[2 * t + 1], b1);
                    b2 = udot4(l2, xl[2 * t], b2);
                    b2 = udot4(l3, xl[2 * t + 1], b2);
                }
                // layout per unit: [half or matrix][row of pair][s1, s2]
                const int o = 4 * (m + hb);
                acc[it][o + 0] += a1;
                acc[it][o + 1] += (int)a2;
                acc[it][o + 2] += b1;
                acc[it][o + 3] += (int)b2;
            }
        }
    };
    if (PF) {
        for (int j0 = 0; j0 < niter; j0 += NPF) {
            if (KIND == VGX_Q8) {
                // every step's x planes are read before the first product (one
                // LDS round trip for the group, not one per step: under a
                // per-lane test each step was a branch whose reads were waited
                // for before the next step's went out); a chunk past the row
                // reads a clamped chunk and adds nothing
                uint4 xh[NPF], xl[NPF];
#pragma unroll
                for (int s = 0; s < NPF; ++s) {
                    const int cc = min(cl + (j0 + s) * LPR, nch - 1);
                    xh[s] = lds[2 * cc];
                    xl[s] = lds[2 * cc + 1];
                }
#pragma unroll
                for (int s = 0; s < NPF; ++s) {
                    const int c = cl + (j0 + s) * LPR;
                    const bool ok = c < nch;
                    const int o = (EPI == EPI_SPLIT && c >= L.split_chunk) ? 2 : 0;
                    int s1 = 0;
                    uint32_t s2 = 0;
                    q8_chunk(pb[s], xh[s], xl[s], s1, s2);
                    acc[0][o] += ok ? s1 : 0;
                    acc[0][o + 1] += ok ? (int)s2 : 0;
                    if (EPI == EPI_GATE) {
                        int t1 = 0;
                        uint32_t t2 = 0;
                        q8_chunk(pb3[s], xh[s], xl[s], t1, t2);
                        acc[0][2] += ok ? t1 : 0;
                        acc[0][3] += ok ? (int)t2 : 0;
                    }
                    if (j0 + s + NPF < niter) pf_load(s, c + NPF * LPR);
                }
            } else {
#pragma unroll
                for (int s = 0; s < NPF; ++s) {
                    const int c = cl + (j0 + s) * LPR;
                    if (c < nch) step(0, c, pb[s], pb3[s]);
                    if (j0 + s + NPF < niter) pf_load(s, c + NPF * LPR);
                }
            }
        }
    }
    for (int j = 0; j < (PF ? 0 : niter); ++j) {
        const int c = cl + j * LPR;
        const bool cok = c < nch;
        uint4 wn[RI], wn3[RI];
        const bool more = j + 1 < niter;
        if (more) {
#pragma unroll
            for (int it = 0; it < RI; ++it) {
                const int u = unit0 + it * RPI + rs;
                const int cn = c + LPR;
                const bool ok = u < units && cn < nch;
                wn[it] = ok ? wload(body + (size_t)u * ustride + (size_t)cn * 16)
                            : make_uint4(0, 0, 0, 0);
                if (EPI == EPI_GATE)
                    wn3[it] = ok ? wload(body3 + (size_t)u * ustride + (size_t)cn * 16)
                                 : make_uint4(0, 0, 0, 0);
            }
        }
        if (cok) {
#pragma unroll
            for (int it = 0; it < RI; ++it) step(it, c, w[it], w3[it]);
        }
        if (more) {
#pragma unroll
            for (int it = 0; it < RI; ++it) {
                w[it] = wn[it];
                if (EPI == EPI_GATE) w3[it] = wn3[it];
            }
        }
    }

    const int row_it = seg_reduce<LPR, RI, NI, int>(acc, cl);
    const int u = unit0 + row_it * RPI + rs;
    if (seg_leader<LPR, RI, int>(cl) && u < units) {
    // bias of the byte split: q8 -128*sum(xl), t3 -sum(x)
    const long long cmul = KIND == VGX_Q8 ? 128LL : 1LL;
#pragma unroll
    for (int hr = 0; hr < ROWS_PER_UNIT; ++hr) {
        const int row = u * ROWS_PER_UNIT + hr;
        if (row < M.rows) {
        // value of (matrix-or-half h) for this row, times the row scale
        auto val = [&](int h, float scale) -> float {
            const int o = KIND == VGX_T3 ? 4 * h + 2 * hr : 2 * h;
            const long long corr = cmul * (EPI == EPI_SPLIT ? (h ? xs1 : xs0) : (long long)xs0 + xs1);
            const long long s = 256LL * acc[0][o] + (long long)(uint32_t)acc[0][o + 1] - corr;
            return (float)s * scale;
        };
        const float sw = PF ? pick(pw, row_it, hr) : gld(M.wsr + row);
        const float rv = PF ? (float)pick(pres, row_it, hr) : (L.res ? (float)gld(L.res + M.out_off + row) : 0.0f);
        if (EPI == EPI_STORE || EPI == EPI_STORE_ARGMAX) {
            const float v = val(0, sw);
            const float t = L.res ? v + rv : v;
            const int q = q16_round(t);
            gst(static_cast<int16_t*>(L.y) + M.out_off + row, (int16_t)q);
            if (EPI == EPI_STORE_ARGMAX) {
                const unsigned long long k = argmax_key(q, M.out_off + row);
                akey = k > akey ? k : akey;
            }
        } else if (EPI == EPI_STORE_F32) {
            gst(static_cast<float*>(L.y) + M.out_off + row, val(0, sw) * (1.0f / 256.0f));
        } else if (EPI == EPI_SPLIT) {
            const float va = val(0, sw), vb = val(1, sw);
            const float y1 = (float)q16_round(va + rv);
            gst(static_cast<int16_t*>(L.y) + row, (int16_t)q16_round(vb + y1));
        } else {  // gate
            const float v1 = val(0, sw), v3 = val(1, PF ? pick(pw3, row_it, hr) : gld(M3.wsr + row));
            const float g = (float)q16_round(v1), uu = (float)q16_round(v3);
            const float a = g / 256.0f;
            const float e = (float)exp(-(double)a);
            const float dn = 1.0f + e;
            const float r = a / dn;
            float o = r * (uu / 256.0f);
            o = o * ldexpf(1.0f, -L.hs);
            gst(static_cast<int16_t*>(L.y) + row, (int16_t)q16_round(o * 256.0f));
        }
        }
    }
    }
    }
    // the stride from the launch descriptor (L.grid is the launch's grid):
    // gridDim.x is an implicit kernel argument in a cache line nothing else
    // touches, and its load cost a memory round trip before the first tile
    tile += L.grid;
    if (tile >= L.blocks) break;
    begin_tile(tile);
    }
    if (EPI == EPI_STORE_ARGMAX) argmax_tail(L, akey);
}

// argmax with the first-maximum rule over int16 values, one block.
// Row blockIdx.x of a row-major [rows][n] array; out[blockIdx.x].
__global__ void __launch_bounds__(1024) argmax_kernel(const int16_t* v, int n, int* out) {
    __shared__ int sv[16], si[16];
    v += (size_t)blockIdx.x * n;
    out += blockIdx.x;
    int best = -65536, bi = 0x7fffffff;
    // A row on a 16-byte boundary is read as 8-value vectors, eight of them a
    // thread in flight before any comparison; a lane's vectors (and the values
    // inside one) come in increasing index order, so its first maximum is kept.
    int head = 0;
    if (((uintptr_t)v & 15u) == 0) {
        const int nvec = n / 8;
        const uint4* v4 = reinterpret_cast<const uint4*>(v);
        for (int b0 = threadIdx.x; b0 < nvec; b0 += 8 * (int)blockDim.x) {
            uint4 q[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) q[k] = v4[min(b0 + k * (int)blockDim.x, nvec - 1)];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int b = b0 + k * (int)blockDim.x;
                const uint32_t w[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int x = (int)(int16_t)(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFFu);
                    if (b < nvec && x > best) { best = x; bi = 8 * b + e; }
                }
            }
        }
        head = nvec * 8;
    }
    for (int i = head + threadIdx.x; i < n; i += blockDim.x) {
        int x = v[i];
        if (x > best || (x == best && i < bi)) { best = x; bi = i; }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        int ob = __shfl_xor(best, o, 64), oi = __shfl_xor(bi, o, 64);
        if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wv] = best; si[wv] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nw = (blockDim.x + 63) / 64;
        for (int k = 1; k < nw; ++k)
            if (sv[k] > best || (sv[k] == best && si[k] < bi)) { best = sv[k]; bi = si[k]; }
        *out = bi;
    }
}

// Dequantisation to fp32, one thread per weight.
__global__ void dequant_kernel(const MatDev M, float* out) {
    const size_t n = (size_t)M.rows * M.cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / M.cols), c = (int)(i % M.cols);
        float v;
        if (M.kind == VGX_Q8) {
            v = (float)((int)M.body[i] - 128) * M.wsr[r];
        } else if (M.kind == VGX_Q4) {
            const uint8_t b = M.body[(size_t)r * q4_rstride(M.cols) + c / 2];
            const int nb = (c & 1) ? (b >> 4) : (b & 15);
            const uint32_t sm = M.sm[(size_t)r * (M.cols / 32) + c / 32];
            const float sa = (float)(int16_t)(sm & 0xFFFFu) * M.ps;
            const float ma = (float)(int16_t)(sm >> 16) * M.ps;
            v = (float)nb * sa + ma;
        } else {
            const size_t stride = (size_t)t3_rstride(M.cols);
            const uint8_t b = M.body[(size_t)(r / 2) * stride + (size_t)(c >> 3) * 4 + (r & 1) * 2 + ((c >> 2) & 1)];
            const unsigned code = (b >> (2 * (c & 3))) & 3u;
            const int lv = (code & 1u) ? ((code & 2u) ? -1 : 1) : 0;
            v = (float)lv * M.wsr[r];
        }
        out[i] = v;
    }
}

// ---------------------------------------------------------------------------
// Dispatch tables.
using KernFn = void (*)(const GemvLaunch);

template <int KIND, int EPI, int XM, bool ONE>
KernFn pick_kernel(int lpr, int ri) {
#define VGX_K(LP, R) \
    if (lpr == LP && ri == R) return gemv_kernel<KIND, LP, R, EPI, XM, ONE>;
    // the plan pairs 4 rows per lane with 8 or 16 lanes per row only
    VGX_K(8, 1) VGX_K(8, 4) VGX_K(16, 1) VGX_K(16, 4) VGX_K(32, 1) VGX_K(64, 1)
#undef VGX_K
    return nullptr;
}

// The (epilogue, input) pairs the entry points use.
template <int KIND>
KernFn pick_epi(int epi, int xm, int lpr, int ri, bool one) {
    // single-matrix launches: the plain, split, gate and f32 epilogues;
    // groups: store (plain or through RMSNorm), f32 and the fused argmax
    if (one) {
        switch (epi) {
            case EPI_STORE:
                return xm == X_RMS ? pick_kernel<KIND, EPI_STORE, X_RMS, true>(lpr, ri)
                                   : pick_kernel<KIND, EPI_STORE, X_I16, true>(lpr, ri);
            case EPI_STORE_F32: return pick_kernel<KIND, EPI_STORE_F32, X_F32, true>(lpr, ri);
            case EPI_GATE:
                return xm == X_RMS ? pick_kernel<KIND, EPI_GATE, X_RMS, true>(lpr, ri)
                                   : pick_kernel<KIND, EPI_GATE, X_I16, true>(lpr, ri);
            case EPI_SPLIT: return xm == X_I16 ? pick_kernel<KIND, EPI_SPLIT, X_I16, true>(lpr, ri) : nullptr;
        }
        return nullptr;
    }
    switch (epi) {
        case EPI_STORE:
            return xm == X_RMS ? pick_kernel<KIND, EPI_STORE, X_RMS, false>(lpr, ri)
                               : pick_kernel<KIND, EPI_STORE, X_I16, false>(lpr, ri);
        case EPI_STORE_F32: return pick_kernel<KIND, EPI_STORE_F32, X_F32, false>(lpr, ri);
        case EPI_STORE_ARGMAX:
            return xm == X_RMS ? pick_kernel<KIND, EPI_STORE_ARGMAX, X_RMS, false>(lpr, ri) : nullptr;
    }
    return nullptr;
}


}  // namespace

// Rows per lane: 4 when the matrix has enough rows to give every CU several
// waves anyway (the bandwidth-bound launches), else 1 (the latency-bound
// decode shapes).  Lanes per row, latency-bound: q8 and q4 enough that each
// lane has about four chunks, at most one wave per row; t3 one chunk per lane
// where a wave covers the row (its table unpacking is the costly part, and
// shorter lanes spread it over more CUs; measured on the 0.5B ternary decode:
// +10%, while q8 decode lost 7% the same way).  Each lane's chunks all load in
// one round trip.  Bandwidth-bound, from a sweep
// of HBM-streamed launches on MI355X: q8 keeps 16 lanes on a row up to 64
// chunks (K <= 1024) and 8 beyond (more chunks per lane in flight; int32
// accumulators are cheap); q4 (fp64 group sums, more registers per chunk) and
// t3 (two rows per chunk) use 8 lanes up to 48 chunks and 16 beyond.
int vgx_gemv_plan(int kind, int rows, int cols, int num_cu, int* lpr, int* ri, int* rows_per_block) {
    const int nch = kind == VGX_Q8 ? cols / 16 : kind == VGX_T3 ? t3_chunks(cols) : cols / 32;
    int l = 8;
    while (l < 64 && l * 4 < nch) l <<= 1;
    const int units = kind == VGX_T3 ? (rows + 1) / 2 : rows;
    const int waves1 = (units + 64 / l - 1) / (64 / l);
    const int r = waves1 >= 16 * num_cu ? 4 : 1;
    if (r == 4) {
        l = kind == VGX_Q8 ? (nch <= 64 ? 16 : 8) : (nch <= 48 ? 8 : 16);
    } else if (kind == VGX_T3) {
        l = 8;
        while (l < 64 && l < nch) l <<= 1;
    } else if (kind == VGX_Q8 && nch == 64) {
        // 1024-column q8 rows take 32 lanes, two chunks a lane (measured on
        // the hybrid's decode rows: 16 -> 32 lanes +0.9% decode; at 768
        // columns 32 lanes were 0.7% slower, and no other row length was
        // measured, so the rule stays on this one)
        l = 32;
    }
    // a q8 launch of at most 1024 rows (few workgroups) takes at least 32
    // lanes a row: MiniMind3's 768 x 768 wo GEMV (48 workgroups at 16 lanes,
    // 96 at 32) made its q8 decode 5931 -> 5956 tokens/s, where 64 lanes were
    // slower and 32 lanes on every 768-column GEMV had cost 0.7%
    if (r == 1 && kind == VGX_Q8 && rows <= 1024 && l < 32) l = 32;
    const int rpi = 64 / l;
    *lpr = l;
    *ri = r;
    *rows_per_block = kWaves * rpi * r;  // in units (row pairs for t3)
    return 0;
}

int vgx_gemv_launch(const GemvLaunch& L, hipStream_t s) {
    KernFn fn = nullptr;
    const int epi = L.xf ? EPI_STORE_F32
                         : L.gate ? EPI_GATE
                         : L.split_chunk > 0 ? EPI_SPLIT
                         : L.argmax_out ? EPI_STORE_ARGMAX : EPI_STORE;
    const int xm = L.xf ? X_F32 : L.rw ? X_RMS : X_I16;
    if (epi == EPI_STORE_ARGMAX && !L.argmax_key) return vgx_fail(VGX_EINVAL, "gemv: argmax without key slots");
    const bool one = L.nmat == 1 && epi != EPI_STORE_ARGMAX;  // the argmax runs over groups only
    switch (L.kind) {
        case VGX_Q8: fn = pick_epi<VGX_Q8>(epi, xm, L.lpr, L.ri, one); break;
        case VGX_Q4: fn = pick_epi<VGX_Q4>(epi, xm, L.lpr, L.ri, one); break;
        case VGX_T3: fn = pick_epi<VGX_T3>(epi, xm, L.lpr, L.ri, one); break;
    }
    if (!fn) return vgx_fail(VGX_EINVAL, "gemv: no kernel for this shape");
    const size_t shm = lds_bytes(L.kind, L.cols, xm);
    if (shm > 160 * 1024) return vgx_fail(VGX_EINVAL, "gemv: activation row too long for LDS");
    if (L.blocks <= 0) return vgx_fail(VGX_EINVAL, "gemv: empty launch");
    const int grid = L.grid > 0 && L.grid < L.blocks ? L.grid : L.blocks;
    if (epi == EPI_STORE_ARGMAX && grid > L.nkeys) return vgx_fail(VGX_EINVAL, "gemv: more workgroups than key slots");
    GemvLaunch Lk = L;
    Lk.grid = grid;  // the kernel's tile stride
    hipLaunchKernelGGL(fn, dim3(grid), dim3(kThreads), shm, s, Lk);
    VGX_LAUNCH_CHECK("gemv launch");
    if (epi == EPI_STORE_ARGMAX) {
        hipLaunchKernelGGL(argmax_keys_kernel, dim3(1), dim3(256), 0, s, L.argmax_key, grid, L.argmax_out, L.tail);
        VGX_LAUNCH_CHECK("argmax keys launch");
    }
    return VGX_OK;
}

int vgx_argmax_launch(const int16_t* v, int n, int rows, int* out, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, s, v, n, out);
    VGX_LAUNCH_CHECK("argmax launch");
    return VGX_OK;
}

int vgx_dequant_launch(const MatDev& d, float* out, hipStream_t s) {
    const size_t n = (size_t)d.rows * d.cols;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks), dim3(256), 0, s, d, out);
    VGX_LAUNCH_CHECK("dequant launch");
    return VGX_OK;
}
