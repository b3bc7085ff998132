// Batched prefill on the int8 matrix cores: Y[t] = W . X[t] for ntok token
// rows at once, the same exact integer sums as the batch-1 GEMV, so every
// output row is bit-identical to vgx_gemv on that token (the reference's
// acceptance rule for a batched path: the logits of a grouped prefill equal
// the serial ones byte for byte, docs/prefill-batching.md:98-113;
// Session::step_group, engine/src/session.cpp:1741-1795).
//
// v_mfma_i32_32x32x32_i8: one wave multiplies a 32 x 32 int8 tile of A by a
// 32 x 32 tile of B into 32 x 32 int32.  Lane l supplies
//   A[m = l % 32][k = 16*(l/32) .. +15]   (16 int8)
//   B[k = 16*(l/32) .. +15][n = l % 32]   (16 int8)
// and holds C[8*(r/4) + 4*(l/32) + r%4][l % 32] in accumulator r (0..15).
// Here A = activation tokens x columns and B^T = weight rows x columns, so a
// lane's B operand is 16 consecutive weight columns of one row: one 16-byte
// (q8) or 8-byte (q4, t3) load.  The q16 activations are split in registers
// into two int8 planes,
//   x = 256*xh + (xl - 128) + 128,   xh = signed high byte, xl = low byte,
// so  sum w*x = 256*sum w*xh + sum w*(xl - 128) + 128*sum w, every term an
// exact integer (|partial| <= 128*128*K < 2^31 for K <= 32768).
//
// A workgroup owns a 32-token x 32-row output tile; its NW waves (4, or 8
// for a launch of few tiles and long rows: the decode batch) take contiguous
// runs of the k-steps.  A wave works in rounds of 4 k-steps: the round's
// activation block (32 tokens x 128 columns) arrives with coalesced loads and
// passes through the wave's LDS block into the matrix-core layout, while the
// weight operands stream from global memory 4 steps ahead.  Loading the A
// operands straight into the matrix-core layout made every load instruction
// touch 32 token rows 2 bytes x cols apart; on MI355X that cost up to 3.4 us
// per 32-token launch.  The waves leave their partial sums (exact integers)
// in LDS once and every thread adds them for its share of the tile's outputs
// and runs the epilogue for those.  Epilogues restate the batch-1 GEMV's fp32
// expressions: q16 store (+ residual, one rounding), the SwiGLU gate over W1
// and W3, and the two-half residual add of the split w2.  q4 folds each
// 32-column group's scale and minimum in after its k-step (one MFMA k-step =
// one group) as the int64 s16*D + m16*X, and scales the total once.  The RMS
// variants normalise the activation rows on the way into LDS, with the
// statistics formed in the workgroup (GPU::rmsnorm's rounding).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "vgx_internal.h"
#include "vgx_qrow.h"

#pragma clang fp contract(off)

namespace {

typedef signed char i8x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kTile = 32;  // tokens and weight rows per wave tile

enum BatchEpi { BEPI_STORE = 0, BEPI_GATE = 1, BEPI_SPLIT = 2 };

struct GemmLaunch {
    MatDev M, M3;           // W (and W3 for the gate)
    int ntok, cols;
    const int16_t* x;       // ntok rows of cols q16 values, row stride ldx
    int ldx;
    const int16_t* res;     // residual rows (stride ldy) or nullptr
    int16_t* y;             // ntok rows of M.rows q16 values, row stride ldy
    int ldy;
    int hs;                 // gate: hidden store exponent
    int split;              // split: first column of the second half
    const int16_t* rw;      // RMS prologue: the q16 norm weight (cols values)
    float eps;              // RMS prologue: epsilon
    long long* part;        // split K: [split][set][ntok][rows] exact partial sums
    int nz;                 // split K: the launch's splits (its grid's z; from here, not from
                            // gridDim.z, an implicit argument whose load would delay the first weights)
};

union Op {
    i8x16 v;
    uint32_t d[4];
};



__device__ __forceinline__ i32x16 mfma(const Op& a, const Op& b, const i32x16& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a.v, b.v, c, 0, 0, 0);
}


// A operands: 16 q16 activations (two 16-byte loads of one token row) as the
// high-byte plane and the low-byte plane minus 128; xsum = their exact sum.
// ok = false gives zeros.
__device__ __forceinline__ void x_planes(const uint4 a, const uint4 b, bool ok, Op& xh, Op& xl, int& xsum) {
    const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    int sh = 0;
    uint32_t sl = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = ok ? perm(d[2 * k + 1], d[2 * k], 0x06040200u) : 0x80808080u;  // low bytes of 4k..4k+3
        const uint32_t hi = ok ? perm(d[2 * k + 1], d[2 * k], 0x07050301u) : 0u;
        xh.d[k] = hi;
        xl.d[k] = lo ^ 0x80808080u;
        sh = sdot4(hi, 0x01010101u, sh);
        sl = __builtin_amdgcn_udot4(lo, 0x01010101u, sl, false);
    }
    xsum = ok ? 256 * sh + (int)sl : 0;
}

// Four 2-bit t3 codes (one byte, code j at bits 2j..2j+1) as four int8
// levels: bit 0 = |level|, bit 1 = sign (engine/tools/mmcf_hf.py:168-199);
// code 2 (a sign without magnitude) is level 0.  Each code is spread to its
// own byte, then level = |l| ^ ((sign & |l|) * 0xFE): 0x01 or 0xFF.
__device__ __forceinline__ uint32_t t3_levels(uint32_t b) {
    const uint32_t x = (b | (b << 6) | (b << 12) | (b << 18)) & 0x03030303u;
    const uint32_t m = x & 0x01010101u;
    const uint32_t sg = (x >> 1) & m;
    return m ^ (sg * 0xFEu);
}

// The bytes of weight row n, columns k0..k0+15: 16 (q8) or 8 (q4, t3, in .x
// and .y; for t3 the texel pair holding row n).
template <int KIND>
__device__ __forceinline__ uint4 w_raw(const MatDev& M, int n, int k0, int K) {
    if (KIND == VGX_Q8) return *reinterpret_cast<const uint4*>(M.body + (size_t)n * K + k0);
    uint2 v;
    if (KIND == VGX_Q4) {
        v = *reinterpret_cast<const uint2*>(M.body + (size_t)n * q4_rstride(K) + (k0 >> 1));
    } else {
        const size_t ustride = (size_t)t3_rstride(K);
        v = *reinterpret_cast<const uint2*>(M.body + (size_t)(n >> 1) * ustride + (size_t)(k0 >> 3) * 4);
    }
    return make_uint4(v.x, v.y, 0u, 0u);
}

// B operand from those bytes: the 16 weights as int8 levels; wsum = their
// sum.  ok = false gives zeros.
template <int KIND>
__device__ __forceinline__ void w_planes(const uint4 v, int n, bool ok, Op& w, int& wsum) {
    if (KIND == VGX_Q8) {
        w.d[0] = v.x ^ 0x80808080u;
        w.d[1] = v.y ^ 0x80808080u;
        w.d[2] = v.z ^ 0x80808080u;
        w.d[3] = v.w ^ 0x80808080u;
    } else if (KIND == VGX_Q4) {
        const uint32_t lo0 = v.x & 0x0F0F0F0Fu, hi0 = (v.x >> 4) & 0x0F0F0F0Fu;
        const uint32_t lo1 = v.y & 0x0F0F0F0Fu, hi1 = (v.y >> 4) & 0x0F0F0F0Fu;
        // low nibble = even column: interleave (lo.b0, hi.b0, lo.b1, hi.b1), ...
        w.d[0] = perm(hi0, lo0, 0x05010400u);
        w.d[1] = perm(hi0, lo0, 0x07030602u);
        w.d[2] = perm(hi1, lo1, 0x05010400u);
        w.d[3] = perm(hi1, lo1, 0x07030602u);
    } else {
        // texel (c, u): b0 b1 = row 2u columns 8c..8c+7, b2 b3 = row 2u+1
        const int sh = (n & 1) * 16;
        w.d[0] = t3_levels((v.x >> sh) & 0xFFu);
        w.d[1] = t3_levels((v.x >> (sh + 8)) & 0xFFu);
        w.d[2] = t3_levels((v.y >> sh) & 0xFFu);
        w.d[3] = t3_levels((v.y >> (sh + 8)) & 0xFFu);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) w.d[i] = ok ? w.d[i] : 0u;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = sdot4(w.d[i], 0x01010101u, s);
    wsum = s;
}

__device__ __forceinline__ float gate_value(float v1, float v3, int hs) {
    const float g = (float)q16_round(v1), uu = (float)q16_round(v3);
    const float a = g / 256.0f;
    const float e = (float)exp(-(double)a);
    const float dn = 1.0f + e;
    const float r = a / dn;
    float o = r * (uu / 256.0f);
    o = o * ldexpf(1.0f, -hs);
    return o * 256.0f;
}

// The inverse RMS of each of the workgroup's token rows (rms_stats_split,
// engine/src/gpu_upload.cpp:280-365, as the batch-1 GEMV's fused prologue
// forms it): 32 partial sums of x^2 over contiguous slices of ceil(K/32)
// values, each stored as floor(P/16 + 1/2), their exact total tot, then
// inv = 1 / sqrt((tot/4096)/K + eps).  One (token, slice) pair a thread.
template <int NT>
__device__ __forceinline__ void rms_stats(const GemmLaunch& G, int t0, unsigned long long* s_tot, float* s_inv) {
    const int K = G.cols;
    const int per = (K + 31) / 32;
    if (threadIdx.x < kTile) s_tot[threadIdx.x] = 0ull;
    __syncthreads();
    for (int pr = threadIdx.x; pr < kTile * 32; pr += NT) {
        const int tt = pr >> 5, sl = pr & 31;
        const int t = t0 + tt;
        if (t >= G.ntok) continue;
        const int16_t* xr = G.x + (size_t)t * G.ldx;
        const int c0 = sl * per, c1 = min(c0 + per, K);
        long long P = 0;
        if ((per & 7) == 0) {
            for (int c = c0; c < c1; c += 8) {
                const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const long long a = (int16_t)(d[k] & 0xFFFFu), b = (int16_t)(d[k] >> 16);
                    P += a * a + b * b;
                }
            }
        } else {
            for (int c = c0; c < c1; ++c) {
                const long long a = xr[c];
                P += a * a;
            }
        }
        atomicAdd(&s_tot[tt], (unsigned long long)((P + 8) >> 4));
    }
    __syncthreads();
    if (threadIdx.x < kTile) {
        const long long tot = (long long)s_tot[threadIdx.x];
        const float ss = (float)tot / 4096.0f;
        s_inv[threadIdx.x] = (float)(1.0 / sqrt((double)(ss / (float)K + G.eps)));
    }
    __syncthreads();
}

// One workgroup: a 32-token x 32-weight-row output tile.  Its NW waves take
// contiguous runs of the k-steps (32 columns each); every wave keeps the raw
// operand bytes of its next NPF steps in flight, then leaves its exact partial
// sums in LDS, and every thread adds the waves' sums for its outputs of the
// tile and applies the epilogue.  NW = 4 when the launch has many
// tiles; 8 when it has few (the decode batch of up to 32 sequences), so that
// each wave walks fewer steps; 2 above two tiles a CU.  RMS: the input rows go
// through RMSNorm first, the statistics formed in the workgroup.
// Two- and four-wave workgroups are built for two waves a SIMD (at most 256
// VGPRs a lane): left alone the compiler gave the q8 and q4 gate 260-280, one
// workgroup a CU, and the 608-tile 256-token gate ran in 2.4 rounds (q8 gate GEMM
// 10.4 -> 9.1 us, q4 14.5 -> 13.8, no spills).
template <int KIND, int EPI, int NW, bool RMS, bool PART>
__global__ void __launch_bounds__(64 * NW, NW == 8 ? 1 : 2) gemm_kernel(const GemmLaunch G) {
    constexpr int NT = 64 * NW;
    constexpr int NA = EPI == BEPI_STORE ? 1 : 2;  // accumulator sets: W1/W3 or the two halves
    constexpr int NPF = 4;                         // k-steps a round
    // LDS: each wave's activation block for a round (32 tokens x NPF steps of
    // 32 columns, int16: 256 bytes a token), reused for the reduction once
    // every wave is past its last round
    // every kernel argument the launch reads, in scalar registers first: one
    // batch of loads instead of a round trip at each first use (fields a
    // variant does not read are constants here)
    {
        const uint8_t* b3 = EPI == BEPI_GATE ? G.M3.body : nullptr;
        const float* w3 = EPI == BEPI_GATE ? G.M3.wsr : nullptr;
        const uint32_t* s3 = EPI == BEPI_GATE ? G.M3.sm : nullptr;
        const float p3 = EPI == BEPI_GATE ? G.M3.ps : 0.0f;
        const int hs0 = EPI == BEPI_GATE ? G.hs : 0;
        const int sp0 = EPI == BEPI_SPLIT ? G.split : 0;
        const int16_t* rw0 = RMS ? G.rw : nullptr;
        const float eps0 = RMS ? G.eps : 0.0f;
        long long* part0 = PART ? G.part : nullptr;
        const int nz0 = PART ? G.nz : 1;
        asm volatile("" ::"s"(G.M.body), "s"(G.M.wsr), "s"(G.M.sm), "s"(G.M.ps), "s"(G.M.rows), "s"(G.ntok),
                     "s"(G.cols), "s"(G.x), "s"(G.ldx), "s"(G.res), "s"(G.y), "s"(G.ldy), "s"(b3), "s"(w3),
                     "s"(s3), "s"(p3), "s"(hs0), "s"(sp0), "s"(rw0), "s"(eps0), "s"(part0), "s"(nz0));
    }
    extern __shared__ __align__(16) unsigned char s_dyn[];
    __shared__ int s_wsum[NW][NA][64];  // each wave's weight sums per lane
    __shared__ int s_xg[NW][kTile];  // q4: this step's group sum of x per token
    __shared__ unsigned long long s_tot[kTile];
    __shared__ float s_inv[kTile];
    constexpr int XROW = NPF * kTile * 2;  // bytes of a token's row in the block
    constexpr int XB = kTile * XROW;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int half = lane >> 5;
    const int li = lane & 31;
    const int n0 = blockIdx.x * kTile;
    const int t0 = blockIdx.y * kTile;
    const int K = G.cols;
    const MatDev& M = G.M;
    const int n = n0 + li;  // this lane's weight row (B operand) and output column
    const int t = t0 + li;  // this lane's token row (A operand)
    const bool nok = n < M.rows;
    // split K (PART): workgroup z of the launch's G.nz takes k-steps
    // [zs0, zs1) and stores its exact integer sums for the epilogue kernel
    const int nsteps = (K + kTile - 1) / kTile;
    const int zs0 = PART ? (int)(((long)nsteps * blockIdx.z) / G.nz) : 0;
    const int zs1 = PART ? (int)(((long)nsteps * (blockIdx.z + 1)) / G.nz) : nsteps;
    const int s_beg = zs0 + ((zs1 - zs0) * wave) / NW, s_end = zs0 + ((zs1 - zs0) * (wave + 1)) / NW;
    unsigned char* s_xw = s_dyn + (size_t)wave * XB;

    i32x16 ch[NA], cl[NA];
    long long dacc[NA][16];
    long long cw[NA];  // q4: sum over the lane's groups of s16 * (the row's nibble sum)
    int wsum[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
        ch[a] = (i32x16){};
        cl[a] = (i32x16){};
        cw[a] = 0;
        wsum[a] = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) dacc[a][r] = 0;
    }
    const float ps = M.ps, ps3 = G.M3.ps;

    // Weight operands: the raw bytes of the lane's NPF next steps are in
    // flight together (each step's loads go out NPF steps ahead of its
    // multiply), from clamped in-range addresses, unconditionally -- a
    // predicated load would be waited for before the next one is issued --
    // and out-of-range rows and columns become zeros when the bytes are
    // turned into operands.
    struct Raw {
        uint4 w, w3;
        uint32_t sm, sm3;
    };
    const int nn = nok ? n : M.rows - 1;
    // (t3 rows are padded to whole 32-column chunks, so its clamp is the
    // padded length: a last half step past K reads zero codes of its row)
    const int Kw = KIND == VGX_T3 ? t3_chunks(K) * kTile : K;
    auto raw_load = [&](int s, Raw& r) {
        const int k0 = min(s * kTile + half * 16, Kw - 16);
        r.w = w_raw<KIND>(M, nn, k0, K);
        if (EPI == BEPI_GATE) r.w3 = w_raw<KIND>(G.M3, nn, k0, K);
        if (KIND == VGX_Q4) {
            r.sm = M.sm[(size_t)nn * (K >> 5) + s];
            if (EPI == BEPI_GATE) r.sm3 = G.M3.sm[(size_t)nn * (K >> 5) + s];
        }
    };
    // Activation operands: a round's block (the wave's NPF steps for the 32
    // tokens) is read with coalesced loads -- instruction i, lane l: token
    // 4i + l/16, the 16-byte piece l%16 of its 256 bytes -- and stored in the
    // wave's LDS block with piece q of token row r at q ^ (r & 7), so the 8
    // lanes of a matrix-core read group (rows r..r+7) hit 8 bank groups.
    // Tokens past ntok read the last token (only their own outputs, never
    // stored, see them).
    const int pc = lane & 15;
    auto x_load = [&](int s0, uint4 (&v)[8], uint4& wv) {
        const int col = min(s0 * kTile + pc * 8, K - 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int tt = min(t0 + 4 * i + (lane >> 4), G.ntok - 1);
            v[i] = *reinterpret_cast<const uint4*>(G.x + (size_t)tt * G.ldx + col);
        }
        if (RMS) wv = *reinterpret_cast<const uint4*>(G.rw + col);
    };
    auto x_store = [&](const uint4 (&v)[8], const uint4& wv) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 4 * i + (lane >> 4);
            uint4 d = v[i];
            if (RMS) {
                const float inv = s_inv[r];
                const uint32_t xd[4] = {d.x, d.y, d.z, d.w};
                const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
                uint32_t o[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[k] = rms_elem(xd[k] & 0xFFFFu, wd[k] & 0xFFFFu, inv) |
                           (rms_elem(xd[k] >> 16, wd[k] >> 16, inv) << 16);
                d = make_uint4(o[0], o[1], o[2], o[3]);
            }
            *reinterpret_cast<uint4*>(s_xw + r * XROW + ((pc ^ (r & 7)) << 4)) = d;
        }
    };

    // the activation block of round r + 1 and the weights NPF steps ahead
    // are loaded while round r is multiplied (a second round in flight cost
    // more in occupancy than it hid)
    Raw rb[NPF];
    uint4 xn[8], wn = make_uint4(0u, 0u, 0u, 0u);
    if (s_beg < s_end) {
        x_load(s_beg, xn, wn);
#pragma unroll
        for (int j = 0; j < NPF; ++j) raw_load(min(s_beg + j, s_end - 1), rb[j]);
    }
    // this thread's epilogue operands (row scales, residuals) for its
    // outputs of the tile (below), loaded before anything waits: issued at
    // the epilogue they cost a memory round trip there
    constexpr int kOutPer = kTile * kTile / NT;  // outputs a thread takes
    float e_wsr[kOutPer], e_wsr3[kOutPer];
    int e_res[kOutPer];
#pragma unroll
    for (int k = 0; k < kOutPer; ++k) {
        const int p = threadIdx.x + k * NT, l = p & 63, r = p >> 6;
        const int on = min(n0 + (l & 31), M.rows - 1);
        const int ot = min(t0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), G.ntok - 1);
        e_wsr[k] = e_wsr3[k] = 0.0f;
        e_res[k] = 0;
        if (PART) continue;
        if (KIND != VGX_Q4) {
            e_wsr[k] = M.wsr[on];
            if (EPI == BEPI_GATE) e_wsr3[k] = G.M3.wsr[on];
        }
        if (EPI != BEPI_GATE && G.res) e_res[k] = G.res[(size_t)ot * G.ldy + on];
    }
    if (RMS) rms_stats<NT>(G, t0, s_tot, s_inv);
    auto do_round = [&](int s0, uint4 (&xv)[8], uint4& wv, Raw* rr) {
        x_store(xv, wv);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (s0 + NPF < s_end) x_load(s0 + NPF, xv, wv);
#pragma unroll
        for (int j = 0; j < NPF; ++j) {
            const int s = s0 + j;
            if (s >= s_end) break;
            const int k0 = s * kTile + half * 16;
            const int q0 = 4 * j + 2 * half;
            const unsigned char* row = s_xw + li * XROW;
            const uint4 x0 = *reinterpret_cast<const uint4*>(row + ((q0 ^ (li & 7)) << 4));
            const uint4 x1 = *reinterpret_cast<const uint4*>(row + (((q0 + 1) ^ (li & 7)) << 4));
            // Operands are not masked for tokens past ntok or rows past M.rows:
            // they feed only their own outputs, which are never stored.  Only a
            // q8 row's last half step can lie past K (cols % 32 == 16): its
            // weights become zeros (and leave the weight sum), so the clamped
            // activation bytes there multiply nothing.  q4 rows are whole
            // 32-column groups; a t3 row's padding holds zero codes.
            const bool wok = KIND != VGX_Q8 || (K & 31) == 0 || k0 < K;
            Op xh, xl, w, w3;
            int xs, ws, ws3 = 0;
            x_planes(x0, x1, true, xh, xl, xs);
            w_planes<KIND>(rr[j].w, n, wok, w, ws);
            if (EPI == BEPI_GATE) w_planes<KIND>(rr[j].w3, n, wok, w3, ws3);
            const uint32_t sm = KIND == VGX_Q4 ? rr[j].sm : 0u;
            const uint32_t sm3 = (KIND == VGX_Q4 && EPI == BEPI_GATE) ? rr[j].sm3 : 0u;
            raw_load(min(s + NPF, s_end - 1), rr[j]);
            if (KIND != VGX_Q4) {
                if (EPI == BEPI_SPLIT) {
                    // a lane's 16 columns lie on one side of the split (split % 16 == 0)
                    const bool lo_side = k0 < G.split;
                    Op zh, zl;
                    for (int i = 0; i < 4; ++i) { zh.d[i] = 0u; zl.d[i] = 0u; }
                    ch[0] = mfma(lo_side ? xh : zh, w, ch[0]);
                    cl[0] = mfma(lo_side ? xl : zl, w, cl[0]);
                    ch[NA - 1] = mfma(lo_side ? zh : xh, w, ch[NA - 1]);
                    cl[NA - 1] = mfma(lo_side ? zl : xl, w, cl[NA - 1]);
                    if (lo_side) wsum[0] += ws; else wsum[NA - 1] += ws;
                } else {
                    ch[0] = mfma(xh, w, ch[0]);
                    cl[0] = mfma(xl, w, cl[0]);
                    wsum[0] += ws;
                    if (EPI == BEPI_GATE) {
                        ch[NA - 1] = mfma(xh, w3, ch[NA - 1]);
                        cl[NA - 1] = mfma(xl, w3, cl[NA - 1]);
                        wsum[NA - 1] += ws3;
                    }
                }
            } else {
                // one step = one 32-column group g = s: D = sum n*x exactly (|D| <
                // 2^24), then the group's exact s16*D + m16*X in int64.  D's
                // 128*wg term (wg the row's nibble sum over the group) is the
                // same for all of a lane's outputs: s16*wg goes into the lane's
                // cw once, and 128*cw joins every output after the loop.
                const i32x16 zero = {};
                const int xg = xs + __shfl_xor(xs, 32, 64);  // token li's group sum
                if (half == 0) s_xg[wave][li] = xg;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                int X[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) X[r] = s_xg[wave][8 * (r >> 2) + 4 * half + (r & 3)];
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                const int nmat = EPI == BEPI_GATE ? 2 : 1;
                const int side = (EPI == BEPI_SPLIT && s * kTile >= G.split) ? 1 : 0;
#pragma unroll
                for (int mm = 0; mm < nmat; ++mm) {
                    const Op& wo = mm == 0 ? w : w3;
                    const i32x16 dh = mfma(xh, wo, zero);
                    const i32x16 dl = mfma(xl, wo, zero);
                    const int wl = mm == 0 ? ws : ws3;
                    const int wg = wl + __shfl_xor(wl, 32, 64);
                    const uint32_t smm = mm == 0 ? sm : sm3;
                    const int sa = (int16_t)(smm & 0xFFFFu), ma = (int16_t)(smm >> 16);
                    const int slot = EPI == BEPI_GATE ? mm : side;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int Dp = 256 * dh[r] + dl[r];  // |Dp| < 2^24
                        long long acc = dacc[slot][r];
                        acc += (long long)sa * Dp;
                        // (two chained 64-bit multiply-adds: left alone the
                        // compiler forms sa*Dp + ma*X first, then a third add)
                        asm("" : "+v"(acc));
                        acc += (long long)ma * X[r];
                        dacc[slot][r] = acc;
                    }
                    cw[slot] += (long long)sa * wg;
                }
            }
        }

        // this round's reads of the block are done before the next round's stores
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };
    for (int s0 = s_beg; s0 < s_end; s0 += NPF) do_round(s0, xn, wn, rb);
    __syncthreads();  // every wave is past its blocks: the LDS becomes the reduction buffer

    // Every wave leaves its exact partial sums in LDS -- per accumulator set a
    // and register r of lane l: the q4 group sums, or 256*hi + lo as one int64
    // (its row's weight sums apart) -- then every thread takes outputs of the
    // tile: the waves' sums added (integers: any order gives the same total)
    // and the epilogue.  Output (l, r): weight row n0 + l%32, token
    // t0 + 8*(r/4) + 4*(l/32) + r%4.
    long long* s_red = reinterpret_cast<long long*>(s_dyn);  // [NW][NA][16][64]
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            s_red[((wave * NA + a) * 16 + r) * 64 + lane] =
                KIND == VGX_Q4 ? dacc[a][r] + 128LL * cw[a] : 256LL * ch[a][r] + (long long)cl[a][r];
    if (KIND != VGX_Q4) {
#pragma unroll
        for (int a = 0; a < NA; ++a) s_wsum[wave][a][lane] = wsum[a];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kOutPer; ++k) {
        const int p = threadIdx.x + k * NT, l = p & 63, r = p >> 6;
        const int on = n0 + (l & 31), ot = t0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        if (on >= M.rows || ot >= G.ntok) continue;
        long long S[NA];
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            long long t = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w) t += s_red[((w * NA + a) * 16 + r) * 64 + l];
            if (KIND != VGX_Q4) {
                int wt = 0;  // the row's weight sum over both column halves
#pragma unroll
                for (int w = 0; w < NW; ++w) wt += s_wsum[w][a][l] + s_wsum[w][a][l ^ 32];
                t += 128LL * wt;
            }
            S[a] = t;
        }
        if (PART) {
#pragma unroll
            for (int a = 0; a < NA; ++a) G.part[(((size_t)blockIdx.z * NA + a) * G.ntok + ot) * M.rows + on] = S[a];
            continue;
        }
        float v[NA];
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const float sc = KIND == VGX_Q4 ? ((EPI == BEPI_GATE && a == 1) ? ps3 : ps)
                                            : ((EPI == BEPI_GATE && a == 1) ? e_wsr3[k] : e_wsr[k]);
            v[a] = (float)S[a] * sc;
        }
        int16_t* yo = G.y + (size_t)ot * G.ldy + on;
        if (EPI == BEPI_STORE) {
            *yo = (int16_t)q16_round(G.res ? v[0] + (float)e_res[k] : v[0]);
        } else if (EPI == BEPI_SPLIT) {
            const float y1 = (float)q16_round(v[0] + (float)e_res[k]);
            *yo = (int16_t)q16_round(v[NA - 1] + y1);
        } else {
            *yo = (int16_t)q16_round(gate_value(v[0], v[NA - 1], G.hs));
        }
    }
}

// The epilogue of a split-K launch: the splits' exact sums added (in split
// order; integers, so any order gives the same total), then the same fp32
// epilogue as gemm_kernel's.  A thread per output row n of token blockIdx.y.
constexpr int kMaxSplit = 8;

// Output row n of token tt of a split-K launch: the splits' exact sums added
// (integers: any order gives the same total), then gemm_kernel's fp32
// epilogue.
template <int EPI>
__device__ __forceinline__ int16_t epi_value(const GemmLaunch& G, int nz, int tt, int n) {
    constexpr int NA = EPI == BEPI_STORE ? 1 : 2;
    const MatDev& M = G.M;
    float v[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
        // every split's sum loads at once (clamped, unconditional), then adds
        long long p[kMaxSplit];
#pragma unroll
        for (int z = 0; z < kMaxSplit; ++z)
            p[z] = G.part[(((size_t)min(z, nz - 1) * NA + a) * G.ntok + tt) * M.rows + n];
        long long S = 0;
#pragma unroll
        for (int z = 0; z < kMaxSplit; ++z) S += z < nz ? p[z] : 0;
        const MatDev& Ma = (EPI == BEPI_GATE && a == 1) ? G.M3 : M;
        v[a] = M.kind == VGX_Q4 ? (float)S * Ma.ps : (float)S * Ma.wsr[n];
    }
    if (EPI == BEPI_STORE) {
        const float o = G.res ? v[0] + (float)G.res[(size_t)tt * G.ldy + n] : v[0];
        return (int16_t)q16_round(o);
    } else if (EPI == BEPI_SPLIT) {
        const float y1 = (float)q16_round(v[0] + (float)G.res[(size_t)tt * G.ldy + n]);
        return (int16_t)q16_round(v[NA - 1] + y1);
    }
    return (int16_t)q16_round(gate_value(v[0], v[NA - 1], G.hs));
}

// The epilogue of a split-K launch: a thread per output row n of token
// blockIdx.y.
// Every argument an epilogue launch reads, in scalar registers in one batch
// of loads (left to the compiler they came in three or four round trips).
#define VGX_EPI_ARGS(G, nz)                                                                                      \
    asm volatile("" ::"s"(G.M.rows), "s"(G.M.kind), "s"(G.M.ps), "s"(G.M.wsr), "s"(G.M3.ps), "s"(G.M3.wsr),  \
                 "s"(G.part), "s"(G.ntok), "s"(G.res), "s"(G.y), "s"(G.ldy), "s"(G.hs), "s"(nz))

template <int EPI>
__global__ void __launch_bounds__(256) gemm_epi_kernel(const GemmLaunch G, int nz) {
    VGX_EPI_ARGS(G, nz);
    const int n = blockIdx.x * 256 + threadIdx.x, tt = blockIdx.y;
    if (n >= G.M.rows) return;
    G.y[(size_t)tt * G.ldy + n] = epi_value<EPI>(G, nz, tt, n);
}

// The same epilogue for a whole token row per workgroup, followed by the
// RMSNorm of the row it wrote (rmsnorm_kernel's arithmetic: 32 partial sums
// of x^2 over contiguous slices of ceil(rows/32), each floor(P/16 + 1/2),
// then (x * inv) * w on the q16 grid) into yn.  The row is kept in LDS.
constexpr int kNormThreads = 1024;  // a row of up to 1024 values: one value a thread

template <int EPI>
__global__ void __launch_bounds__(kNormThreads) gemm_epi_norm_kernel(const GemmLaunch G, int nz, const int16_t* nw,
                                                                     float neps, int16_t* yn) {
    asm volatile("" ::"s"(G.M.rows), "s"(G.M.kind), "s"(G.M.ps), "s"(G.M.wsr), "s"(G.M3.ps), "s"(G.M3.wsr),
                 "s"(G.part), "s"(G.ntok), "s"(G.res), "s"(G.y), "s"(G.ldy), "s"(G.hs), "s"(nz), "s"(nw), "s"(neps),
                 "s"(yn));
    extern __shared__ __align__(16) unsigned char s_dyn[];
    int16_t* row = reinterpret_cast<int16_t*>(s_dyn);
    __shared__ long long part[32];
    const int tt = blockIdx.x, rows = G.M.rows, tid = threadIdx.x;
    // the norm weight of this thread's first output, loaded before the
    // epilogue's loads (issued after the barriers below it was a round trip
    // of its own at the end)
    uint16_t nw0 = (uint16_t)nw[min(tid, rows - 1)];
    for (int n = tid; n < rows; n += kNormThreads) {
        const int16_t q = epi_value<EPI>(G, nz, tt, n);
        G.y[(size_t)tt * G.ldy + n] = q;
        row[n] = q;
    }
    asm volatile("" : "+v"(nw0));
    __syncthreads();
    const int per = (rows + 31) / 32;
    if (tid < 256) {  // 8 threads a partial slice (whole waves)
        const int p = tid >> 3, sub = tid & 7;
        long long P = 0;
        for (int k = sub; k < per; k += 8) {
            const int i = p * per + k;
            if (i < rows) P += (long long)row[i] * row[i];
        }
        P = sum8_i64(P);  // (DPP; exact integers, any order)
        if (sub == 0) part[p] = (P + 8) >> 4;
    }
    __syncthreads();
    // every wave adds the 32 slices itself (exact integers) and forms inv
    const long long tot = sum32_i64(part[tid & 31]);
    const float ss = (float)tot / 4096.0f;
    const float inv = (float)(1.0 / sqrt((double)(ss / (float)rows + neps)));
    for (int i = tid; i < rows; i += kNormThreads)
        yn[(size_t)tt * rows + i] = (int16_t)rms_elem((uint16_t)row[i], i == tid ? nw0 : (uint16_t)nw[i], inv);
}

using GemmFn = void (*)(const GemmLaunch);

template <int EPI, int NW, bool RMS, bool PART>
GemmFn pick_kind(int kind) {
    switch (kind) {
        case VGX_Q8: return gemm_kernel<VGX_Q8, EPI, NW, RMS, PART>;
        case VGX_Q4: return gemm_kernel<VGX_Q4, EPI, NW, RMS, PART>;
        case VGX_T3: return gemm_kernel<VGX_T3, EPI, NW, RMS, PART>;
    }
    return nullptr;
}

template <int EPI, bool RMS>
GemmFn pick_nw(int kind, int nw, bool part) {
    if (part) return nw == 4 ? pick_kind<EPI, 4, RMS, true>(kind) : nullptr;
    switch (nw) {
        case 2: return pick_kind<EPI, 2, RMS, false>(kind);
        case 4: return pick_kind<EPI, 4, RMS, false>(kind);
        case 8: return pick_kind<EPI, 8, RMS, false>(kind);
    }
    return nullptr;
}

GemmFn pick(int epi, int kind, int nw, bool rms, bool part) {
    if (epi == BEPI_STORE)
        return rms ? pick_nw<BEPI_STORE, true>(kind, nw, part) : pick_nw<BEPI_STORE, false>(kind, nw, part);
    if (epi == BEPI_GATE)
        return rms ? pick_nw<BEPI_GATE, true>(kind, nw, part) : pick_nw<BEPI_GATE, false>(kind, nw, part);
    return rms ? nullptr : pick_nw<BEPI_SPLIT, false>(kind, nw, part);
}

// Splits of K for a launch of one token tile whose row tiles leave most CUs
// idle (the decode batch) and whose rows are longer than 32 k-steps (four a
// wave of an 8-wave workgroup): enough workgroups to cover the CUs, at least
// four k-steps (one per wave) a split; 1 = no split.  Up to 32 k-steps the
// whole row in one 8-wave workgroup beats the split and its epilogue launch
// (the 32-sequence qkv of the 0.5B t3 model, 1280 x 1024: 5.7 against 8.3 us).
int k_splits(int tiles_x, int tiles_y, int nsteps, int num_cu) {
    if (tiles_y != 1 || tiles_x >= num_cu / 2 || nsteps <= 32) return 1;
    return std::max(1, std::min({num_cu / tiles_x, nsteps / 4, kMaxSplit}));
}

// The context's split-K workspace.  k_splits splits only one token tile
// (ntok <= 32) of fewer than num_cu/2 row tiles, at most kMaxSplit ways, with
// at most two accumulator sets, so every split launch fits
//   kMaxSplit * 2 * 32 * (num_cu/2 * 32) int64 sums
// (16 MiB at 256 CUs).  That much is allocated once, at the first launch that
// splits, and never regrown: a graph captured with a split GEMM keeps a valid
// address for the context's life.  No allocation happens under stream capture
// (such a launch runs unsplit until an uncaptured split has allocated the
// buffer).  Returns false when the launch must run unsplit.
size_t ws_bound(int num_cu) {
    return (size_t)kMaxSplit * 2 * kTile * (size_t)(std::max(num_cu, 2) / 2 * kTile) * sizeof(long long);
}

bool workspace(vgx_ctx* ctx, size_t bytes, long long** out) {
    std::lock_guard<std::mutex> lock(ctx->ws_mu);
    if (!ctx->ws) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
        const size_t want = ws_bound(ctx->num_cu);
        if (hipMalloc(&ctx->ws, want) != hipSuccess) {
            (void)hipGetLastError();
            ctx->ws = nullptr;
            return false;
        }
        ctx->ws_bytes = want;
    }
    if (bytes > ctx->ws_bytes) return false;
    *out = static_cast<long long*>(ctx->ws);
    return true;
}

// Waves per workgroup: 4 when the launch has at least one tile per CU (two
// 4-wave workgroups fit a CU's registers where one 8-wave workgroup does, so
// up to two tiles a CU run in one round: the 256-token qkv, 384 tiles, took
// 0.8% less of MiniMind3's 256-token q4 prefill than with 8 waves in two rounds); otherwise (a
// few row tiles: a decode batch, a short prompt) 8 when the row has more than
// 16 k-steps, so the tiles' k-steps are spread over more waves.  (16 waves
// would cap a lane at 128 registers and spill the operands in flight; 8 waves
// with four steps in flight keep as many bytes in flight per CU.)  Above two
// tiles a CU, 2: four 2-wave workgroups fit a CU, so the launch still runs in
// one round (the 256-token q4 gate, 608 tiles: 22.5 -> 21.1 us; with 4 waves
// its last 96 tiles started when the first round ended).
int waves_for(int tiles, int nsteps, int num_cu) {
    if (tiles > 2 * num_cu) return 2;
    return tiles < num_cu && nsteps > 16 ? 8 : 4;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// nrm_w / neps / yn: also the RMSNorm of the rows written (y's rows, W's rows
// wide) into yn, in the split-K epilogue launch or as a launch of its own.
int launch(vgx_ctx* ctx, const vgx_mat* W, const vgx_mat* W3, int ntok, const int16_t* x, const int16_t* res,
           int16_t* y, int epi, int hs, int split, const char* who, const int16_t* rw = nullptr, float eps = 0.0f,
           const int16_t* nrm_w = nullptr, float neps = 0.0f, int16_t* yn = nullptr) {
    if (!ctx || !W || !x || !y) return vgx_fail(VGX_EINVAL, std::string(who) + ": NULL argument");
    if (ntok <= 0 || ntok > 65535 * kTile) return vgx_fail(VGX_EINVAL, std::string(who) + ": ntok outside 1..2097120");
    if (!aligned16(x)) return vgx_fail(VGX_EINVAL, std::string(who) + ": x must be 16-byte aligned");
    if (rw && !aligned16(rw)) return vgx_fail(VGX_EINVAL, std::string(who) + ": the RMSNorm weight must be 16-byte aligned");
    if (rw && !(eps > 0.0f)) return vgx_fail(VGX_EINVAL, std::string(who) + ": the RMSNorm epsilon must be positive");
    const MatDev& M = W->d;
    if (M.cols % (M.kind == VGX_T3 ? 8 : 16))
        return vgx_fail(VGX_EINVAL, std::string(who) + ": cols must be a multiple of " +
                                        std::to_string(M.kind == VGX_T3 ? 8 : 16));
    VGX_HIP(hipSetDevice(ctx->device));
    GemmLaunch L{};
    L.M = M;
    if (W3) L.M3 = W3->d;
    L.ntok = ntok;
    L.cols = M.cols;
    L.x = x;
    L.ldx = M.cols;
    L.res = res;
    L.y = y;
    L.ldy = M.rows;
    L.hs = hs;
    L.split = split;
    L.rw = rw;
    L.eps = eps;
    dim3 grid((M.rows + kTile - 1) / kTile, (ntok + kTile - 1) / kTile);
    const int nsteps = (M.cols + kTile - 1) / kTile;
    // (the RMS variants stay whole: every split would recompute the row statistics)
    int nz = rw ? 1 : k_splits((int)grid.x, (int)grid.y, nsteps, ctx->num_cu);
    if (nz > 1) {
        const int na = epi == BEPI_STORE ? 1 : 2;
        const size_t bytes = (size_t)nz * na * ntok * M.rows * sizeof(long long);
        if (!workspace(ctx, bytes, &L.part)) nz = 1;  // no workspace: one pass
        grid.z = nz;
    }
    L.nz = nz;
    const int nw = nz > 1 ? 4 : waves_for((int)(grid.x * grid.y), nsteps, ctx->num_cu);
    GemmFn fn = pick(epi, M.kind, nw, rw != nullptr, nz > 1);
    if (!fn) return vgx_fail(VGX_EINVAL, std::string(who) + ": unknown weight kind");
    // each wave's activation block (32 tokens x 4 k-steps of 32 int16), then
    // each wave's exact sums (16 int64 a lane per accumulator set)
    const int na = epi == BEPI_STORE ? 1 : 2;
    const int lds = std::max(nw * kTile * 4 * kTile * 2, nw * na * 16 * 64 * 8);
    if (lds > 48 * 1024) {
        static bool lds_set[256];
        const int slot = (((epi * 2 + (rw ? 1 : 0)) * 4 + M.kind) * 3 + (nw == 8 ? 2 : nw == 4 ? 1 : 0)) * 2 + (nz > 1 ? 1 : 0);
        if (!lds_set[slot]) {
            VGX_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
            lds_set[slot] = true;
        }
    }
    hipLaunchKernelGGL(fn, grid, dim3(64 * nw), lds, ctx->stream, L);
    VGX_LAUNCH_CHECK("gemm launch");
    const bool norm_rows = yn && M.rows * 2 <= 64 * 1024;  // the row fits the epilogue's LDS
    if (nz > 1 && yn && norm_rows) {
        const size_t rl = (size_t)M.rows * 2;
        if (epi == BEPI_STORE)
            hipLaunchKernelGGL(gemm_epi_norm_kernel<BEPI_STORE>, dim3(ntok), dim3(kNormThreads), rl, ctx->stream, L,
                               nz, nrm_w, neps, yn);
        else
            hipLaunchKernelGGL(gemm_epi_norm_kernel<BEPI_SPLIT>, dim3(ntok), dim3(kNormThreads), rl, ctx->stream, L,
                               nz, nrm_w, neps, yn);
        VGX_LAUNCH_CHECK("gemm epilogue launch");
        return VGX_OK;
    }
    if (nz > 1) {
        const dim3 eg((M.rows + 255) / 256, ntok);
        if (epi == BEPI_STORE) hipLaunchKernelGGL(gemm_epi_kernel<BEPI_STORE>, eg, dim3(256), 0, ctx->stream, L, nz);
        else if (epi == BEPI_GATE) hipLaunchKernelGGL(gemm_epi_kernel<BEPI_GATE>, eg, dim3(256), 0, ctx->stream, L, nz);
        else hipLaunchKernelGGL(gemm_epi_kernel<BEPI_SPLIT>, eg, dim3(256), 0, ctx->stream, L, nz);
        VGX_LAUNCH_CHECK("gemm epilogue launch");
    }
    if (yn) return vgx_rmsnorm_batch(ctx, ntok, M.rows, y, nrm_w, neps, yn);
    return VGX_OK;
}

}  // namespace

extern "C" {

int vgx_gemm(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* res, int16_t* y) {
    return launch(ctx, W, nullptr, ntok, x, res, y, BEPI_STORE, 0, 0, "vgx_gemm");
}

int vgx_gemm_add_split(vgx_ctx* ctx, const vgx_mat* W, int split, int ntok, const int16_t* x, const int16_t* res,
                       int16_t* y) {
    if (!W || !res) return vgx_fail(VGX_EINVAL, "vgx_gemm_add_split: NULL argument");
    const int unit = W->d.kind == VGX_Q8 ? 16 : 32;
    if (split <= 0 || split >= W->d.cols || split % unit)
        return vgx_fail(VGX_EINVAL, "vgx_gemm_add_split: split must be inside cols and a multiple of " +
                                        std::to_string(unit));
    return launch(ctx, W, nullptr, ntok, x, res, y, BEPI_SPLIT, 0, split, "vgx_gemm_add_split");
}

int vgx_gemm_norm(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* res, int16_t* y,
                  const int16_t* rms_w, float eps, int16_t* yn) {
    if (!rms_w || !yn) return vgx_fail(VGX_EINVAL, "vgx_gemm_norm: NULL RMSNorm weight or output");
    if (!(eps > 0.0f)) return vgx_fail(VGX_EINVAL, "vgx_gemm_norm: the RMSNorm epsilon must be positive");
    return launch(ctx, W, nullptr, ntok, x, res, y, BEPI_STORE, 0, 0, "vgx_gemm_norm", nullptr, 0.0f, rms_w, eps, yn);
}

int vgx_gemm_add_split_norm(vgx_ctx* ctx, const vgx_mat* W, int split, int ntok, const int16_t* x,
                            const int16_t* res, int16_t* y, const int16_t* rms_w, float eps, int16_t* yn) {
    if (!W || !res || !rms_w || !yn) return vgx_fail(VGX_EINVAL, "vgx_gemm_add_split_norm: NULL argument");
    if (!(eps > 0.0f)) return vgx_fail(VGX_EINVAL, "vgx_gemm_add_split_norm: the RMSNorm epsilon must be positive");
    const int unit = W->d.kind == VGX_Q8 ? 16 : 32;
    if (split <= 0 || split >= W->d.cols || split % unit)
        return vgx_fail(VGX_EINVAL, "vgx_gemm_add_split_norm: split must be inside cols and a multiple of " +
                                        std::to_string(unit));
    return launch(ctx, W, nullptr, ntok, x, res, y, BEPI_SPLIT, 0, split, "vgx_gemm_add_split_norm", nullptr, 0.0f,
                  rms_w, eps, yn);
}

int vgx_gemm_rms(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* rms_w, float eps,
                 const int16_t* res, int16_t* y) {
    if (!rms_w) return vgx_fail(VGX_EINVAL, "vgx_gemm_rms: NULL RMSNorm weight");
    return launch(ctx, W, nullptr, ntok, x, res, y, BEPI_STORE, 0, 0, "vgx_gemm_rms", rms_w, eps);
}

int vgx_ffn_gate_batch_rms(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, int ntok, const int16_t* x,
                           const int16_t* rms_w, float eps, int hs, int16_t* h) {
    if (!W1 || !W3 || !rms_w) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch_rms: NULL argument");
    if (W1->d.kind != W3->d.kind || W1->d.rows != W3->d.rows || W1->d.cols != W3->d.cols)
        return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch_rms: W1 and W3 differ in kind or shape");
    if (hs < 0 || hs > 5) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch_rms: hs outside 0..5");
    return launch(ctx, W1, W3, ntok, x, nullptr, h, BEPI_GATE, hs, 0, "vgx_ffn_gate_batch_rms", rms_w, eps);
}

int vgx_ffn_gate_batch(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, int ntok, const int16_t* x, int hs,
                       int16_t* h) {
    if (!W1 || !W3) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: NULL matrix");
    if (W1->d.kind != W3->d.kind || W1->d.rows != W3->d.rows || W1->d.cols != W3->d.cols)
        return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: W1 and W3 differ in kind or shape");
    if (hs < 0 || hs > 5) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: hs outside 0..5");
    return launch(ctx, W1, W3, ntok, x, nullptr, h, BEPI_GATE, hs, 0, "vgx_ffn_gate_batch");
}

}  // extern "C"
