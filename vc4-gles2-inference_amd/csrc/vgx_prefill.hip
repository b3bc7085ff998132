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
// A workgroup owns a 32-token x 32-row output tile; its 4 waves take a
// contiguous quarter of the k-steps each, load each step's operands one step
// ahead, and wave 0 adds the other waves' partial sums (exact integers; for
// q4 doubles, in wave order) before the epilogue.  Epilogues restate the batch-1 GEMV's fp32
// expressions: q16 store (+ residual, one rounding), the SwiGLU gate over W1
// and W3, and the two-half residual add of the split w2.  q4 applies its
// per-group fp32 terms after each 32-column group (one MFMA k-step = one
// group) and sums them in double in group order, as the oracle does.
#include <cmath>
#include <string>

#include "vgx_internal.h"

#pragma clang fp contract(off)

namespace {

typedef signed char i8x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
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
};

union Op {
    i8x16 v;
    uint32_t d[4];
};

__device__ __forceinline__ int q16_round(float v) {
    float f = floorf(v + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

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

// Four 2-bit t3 codes (one byte) as four int8 levels: bit 0 = |level|,
// bit 1 = sign (engine/tools/mmcf_hf.py:168-199).
__device__ __forceinline__ uint32_t t3_levels(uint32_t b) {
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = (b >> (2 * j)) & 3u;
        const uint32_t lv = c == 1u ? 0x01u : (c == 3u ? 0xFFu : 0x00u);
        r |= lv << (8 * j);
    }
    return r;
}

// The bytes of weight row n, columns k0..k0+15: 16 (q8) or 8 (q4, t3, in .x
// and .y; for t3 the texel pair holding row n).
template <int KIND>
__device__ __forceinline__ uint4 w_raw(const MatDev& M, int n, int k0, int K) {
    if (KIND == VGX_Q8) return *reinterpret_cast<const uint4*>(M.body + (size_t)n * K + k0);
    uint2 v;
    if (KIND == VGX_Q4) {
        v = *reinterpret_cast<const uint2*>(M.body + (size_t)n * (K >> 1) + (k0 >> 1));
    } else {
        const size_t ustride = (size_t)(K >> 3) * 4;
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

template <int KIND, int EPI>
__global__ void __launch_bounds__(kThreads) gemm_kernel(const GemmLaunch G) {
    constexpr int NA = EPI == BEPI_STORE ? 1 : 2;  // accumulator sets: W1/W3 or the two halves
    // Waves 1..3 hand their partial sums to wave 0 through LDS, lane-major:
    // q8/t3 [wave-1][set][ch 0..15, cl 0..15][lane] int32 plus the weight
    // sums; q4 [wave-1][set][r][lane] double.
    constexpr int kRedInts = (kWaves - 1) * NA * 32 * 64 + (kWaves - 1) * NA * 64;
    constexpr int kRedBytes = KIND == VGX_Q4 ? (kWaves - 1) * NA * 16 * 64 * 8 : kRedInts * 4;
    __shared__ __align__(16) unsigned char s_red[kRedBytes];
    __shared__ int s_xg[kWaves][kTile];  // q4: this step's group sum of x per token

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
    const bool tok = t < G.ntok;
    const int16_t* xrow = G.x + (size_t)(tok ? t : 0) * G.ldx;
    const int nsteps = (K + kTile - 1) / kTile;
    // the four waves of a workgroup share one 32 x 32 output tile and take a
    // contiguous quarter of the k-steps each
    const int s_beg = (nsteps * wave) / kWaves, s_end = (nsteps * (wave + 1)) / kWaves;

    i32x16 ch[NA], cl[NA];
    double dacc[NA][16];
    int wsum[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
        ch[a] = (i32x16){};
        cl[a] = (i32x16){};
        wsum[a] = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) dacc[a][r] = 0.0;
    }
    const float ps = M.ps, ps3 = G.M3.ps;

    // A step's operands: the raw bytes of the lane's NPF next steps are in
    // flight together (each step's loads go out NPF steps ahead of its
    // multiply), from clamped in-range addresses, unconditionally -- a
    // predicated load would be waited for before the next one is issued --
    // and out-of-range tokens, rows and columns become zeros when the bytes
    // are turned into operands.
    struct Ops {
        Op xh, xl, w, w3;
        int xs, ws, ws3;
        uint32_t sm, sm3;
    };
    struct Raw {
        uint4 xa, xb, w, w3;
        uint32_t sm, sm3;
    };
    const int nn = nok ? n : M.rows - 1;
    auto raw_load = [&](int s, Raw& r) {
        const int k0 = min(s * kTile + half * 16, K - 16);
        const uint4* p = reinterpret_cast<const uint4*>(xrow + k0);
        r.xa = p[0];
        r.xb = p[1];
        r.w = w_raw<KIND>(M, nn, k0, K);
        if (EPI == BEPI_GATE) r.w3 = w_raw<KIND>(G.M3, nn, k0, K);
        if (KIND == VGX_Q4) {
            r.sm = M.sm[(size_t)nn * (K >> 5) + s];
            if (EPI == BEPI_GATE) r.sm3 = G.M3.sm[(size_t)nn * (K >> 5) + s];
        }
    };
    auto process = [&](int s, const Raw& r, Ops& o) {
        const int k0 = s * kTile + half * 16;
        const bool kok = k0 < K;
        x_planes(r.xa, r.xb, tok && kok, o.xh, o.xl, o.xs);
        w_planes<KIND>(r.w, n, nok && kok, o.w, o.ws);
        o.ws3 = 0;
        if (EPI == BEPI_GATE) w_planes<KIND>(r.w3, n, nok && kok, o.w3, o.ws3);
        if (KIND == VGX_Q4) {
            o.sm = nok ? r.sm : 0u;
            o.sm3 = (EPI == BEPI_GATE && nok) ? r.sm3 : 0u;
        }
    };
    constexpr int NPF = 4;
    Raw rb[NPF];
    if (s_beg < s_end) {
#pragma unroll
        for (int j = 0; j < NPF; ++j) raw_load(min(s_beg + j, s_end - 1), rb[j]);
    }
    for (int s0 = s_beg; s0 < s_end; s0 += NPF)
#pragma unroll
    for (int j = 0; j < NPF; ++j) {
        const int s = s0 + j;
        if (s >= s_end) break;
        Ops cur;
        process(s, rb[j], cur);
        raw_load(min(s + NPF, s_end - 1), rb[j]);
        const int k0 = s * kTile + half * 16;
        if (KIND != VGX_Q4) {
            if (EPI == BEPI_SPLIT) {
                // a lane's 16 columns lie on one side of the split (split % 16 == 0)
                const bool lo_side = k0 < G.split;
                Op zh, zl;
                for (int i = 0; i < 4; ++i) { zh.d[i] = 0u; zl.d[i] = 0u; }
                ch[0] = mfma(lo_side ? cur.xh : zh, cur.w, ch[0]);
                cl[0] = mfma(lo_side ? cur.xl : zl, cur.w, cl[0]);
                ch[NA - 1] = mfma(lo_side ? zh : cur.xh, cur.w, ch[NA - 1]);
                cl[NA - 1] = mfma(lo_side ? zl : cur.xl, cur.w, cl[NA - 1]);
                if (lo_side) wsum[0] += cur.ws; else wsum[NA - 1] += cur.ws;
            } else {
                ch[0] = mfma(cur.xh, cur.w, ch[0]);
                cl[0] = mfma(cur.xl, cur.w, cl[0]);
                wsum[0] += cur.ws;
                if (EPI == BEPI_GATE) {
                    ch[NA - 1] = mfma(cur.xh, cur.w3, ch[NA - 1]);
                    cl[NA - 1] = mfma(cur.xl, cur.w3, cl[NA - 1]);
                    wsum[NA - 1] += cur.ws3;
                }
            }
        } else {
            // one step = one 32-column group g = s: D = sum n*x exactly (|D| <
            // 2^24), then the shader's fp32 term (s16*ps)*D + (m16*ps)*X,
            // summed in double
            const i32x16 zero = {};
            const int xg = cur.xs + __shfl_xor(cur.xs, 32, 64);  // token li's group sum
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
                const Op& wv = mm == 0 ? cur.w : cur.w3;
                const float pss = mm == 0 ? ps : ps3;
                const i32x16 dh = mfma(cur.xh, wv, zero);
                const i32x16 dl = mfma(cur.xl, wv, zero);
                const int wl = mm == 0 ? cur.ws : cur.ws3;
                const int wg = wl + __shfl_xor(wl, 32, 64);
                const uint32_t sm = mm == 0 ? cur.sm : cur.sm3;
                const float sa = (float)(int16_t)(sm & 0xFFFFu) * pss;
                const float ma = (float)(int16_t)(sm >> 16) * pss;
                const int slot = EPI == BEPI_GATE ? mm : side;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int D = 256 * dh[r] + dl[r] + 128 * wg;
                    const float t1 = sa * (float)D;
                    const float t2 = ma * (float)X[r];
                    const float tt = t1 + t2;
                    dacc[slot][r] += (double)tt;
                }
            }
        }
    }

    // waves 1..3 hand over; wave 0 adds the partials in wave order and stores
    if (wave > 0) {
        if (KIND == VGX_Q4) {
            double* p = reinterpret_cast<double*>(s_red) + (size_t)(wave - 1) * NA * 16 * 64;
#pragma unroll
            for (int a = 0; a < NA; ++a)
#pragma unroll
                for (int r = 0; r < 16; ++r) p[(a * 16 + r) * 64 + lane] = dacc[a][r];
        } else {
            int* p = reinterpret_cast<int*>(s_red) + (size_t)(wave - 1) * NA * 32 * 64;
            int* pw = reinterpret_cast<int*>(s_red) + (size_t)(kWaves - 1) * NA * 32 * 64 + (wave - 1) * NA * 64;
#pragma unroll
            for (int a = 0; a < NA; ++a) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    p[(a * 32 + r) * 64 + lane] = ch[a][r];
                    p[(a * 32 + 16 + r) * 64 + lane] = cl[a][r];
                }
                pw[a * 64 + lane] = wsum[a];
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;
    for (int wv = 1; wv < kWaves; ++wv) {
        if (KIND == VGX_Q4) {
            const double* p = reinterpret_cast<const double*>(s_red) + (size_t)(wv - 1) * NA * 16 * 64;
#pragma unroll
            for (int a = 0; a < NA; ++a)
#pragma unroll
                for (int r = 0; r < 16; ++r) dacc[a][r] += p[(a * 16 + r) * 64 + lane];
        } else {
            const int* p = reinterpret_cast<const int*>(s_red) + (size_t)(wv - 1) * NA * 32 * 64;
            const int* pw = reinterpret_cast<const int*>(s_red) + (size_t)(kWaves - 1) * NA * 32 * 64 + (wv - 1) * NA * 64;
#pragma unroll
            for (int a = 0; a < NA; ++a) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    ch[a][r] += p[(a * 32 + r) * 64 + lane];
                    cl[a][r] += p[(a * 32 + 16 + r) * 64 + lane];
                }
                wsum[a] += pw[a * 64 + lane];
            }
        }
    }

    // epilogue: this lane holds column n for 16 token rows
    int wtot[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) wtot[a] = wsum[a] + __shfl_xor(wsum[a], 32, 64);
    const float wsr = (KIND != VGX_Q4 && nok) ? M.wsr[n] : 0.0f;
    const float wsr3 = (KIND != VGX_Q4 && EPI == BEPI_GATE && nok) ? G.M3.wsr[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = 8 * (r >> 2) + 4 * half + (r & 3);
        const int tt = t0 + m;
        if (!nok || tt >= G.ntok) continue;
        float v[NA];
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            if (KIND == VGX_Q4) {
                v[a] = (float)dacc[a][r];
            } else {
                const long long S = 256LL * ch[a][r] + (long long)cl[a][r] + 128LL * wtot[a];
                const float sc = (EPI == BEPI_GATE && a == 1) ? wsr3 : wsr;
                v[a] = (float)S * sc;
            }
        }
        int16_t* yo = G.y + (size_t)tt * G.ldy + n;
        if (EPI == BEPI_STORE) {
            const float o = G.res ? v[0] + (float)G.res[(size_t)tt * G.ldy + n] : v[0];
            *yo = (int16_t)q16_round(o);
        } else if (EPI == BEPI_SPLIT) {
            const float y1 = (float)q16_round(v[0] + (float)G.res[(size_t)tt * G.ldy + n]);
            *yo = (int16_t)q16_round(v[NA - 1] + y1);
        } else {
            *yo = (int16_t)q16_round(gate_value(v[0], v[NA - 1], G.hs));
        }
    }
}

using GemmFn = void (*)(const GemmLaunch);

template <int EPI>
GemmFn pick(int kind) {
    switch (kind) {
        case VGX_Q8: return gemm_kernel<VGX_Q8, EPI>;
        case VGX_Q4: return gemm_kernel<VGX_Q4, EPI>;
        case VGX_T3: return gemm_kernel<VGX_T3, EPI>;
    }
    return nullptr;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch(vgx_ctx* ctx, const vgx_mat* W, const vgx_mat* W3, int ntok, const int16_t* x, const int16_t* res,
           int16_t* y, int epi, int hs, int split, const char* who) {
    if (!ctx || !W || !x || !y) return vgx_fail(VGX_EINVAL, std::string(who) + ": NULL argument");
    if (ntok <= 0 || ntok > 65535 * kTile) return vgx_fail(VGX_EINVAL, std::string(who) + ": ntok outside 1..2097120");
    if (!aligned16(x)) return vgx_fail(VGX_EINVAL, std::string(who) + ": x must be 16-byte aligned");
    const MatDev& M = W->d;
    if (M.kind == VGX_Q8 && M.cols % 16)
        return vgx_fail(VGX_EINVAL, std::string(who) + ": q8 cols must be a multiple of 16");
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
    GemmFn fn = epi == BEPI_STORE ? pick<BEPI_STORE>(M.kind)
              : epi == BEPI_GATE ? pick<BEPI_GATE>(M.kind) : pick<BEPI_SPLIT>(M.kind);
    if (!fn) return vgx_fail(VGX_EINVAL, std::string(who) + ": unknown weight kind");
    const dim3 grid((M.rows + kTile - 1) / kTile, (ntok + kTile - 1) / kTile);
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), 0, ctx->stream, L);
    VGX_LAUNCH_CHECK("gemm launch");
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

int vgx_ffn_gate_batch(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, int ntok, const int16_t* x, int hs,
                       int16_t* h) {
    if (!W1 || !W3) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: NULL matrix");
    if (W1->d.kind != W3->d.kind || W1->d.rows != W3->d.rows || W1->d.cols != W3->d.cols)
        return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: W1 and W3 differ in kind or shape");
    if (hs < 0 || hs > 5) return vgx_fail(VGX_EINVAL, "vgx_ffn_gate_batch: hs outside 0..5");
    return launch(ctx, W1, W3, ntok, x, nullptr, h, BEPI_GATE, hs, 0, "vgx_ffn_gate_batch");
}

}  // extern "C"
