// Decode attention over the packed KV cache, with the KV pack (append).
//
// One workgroup of 1024 threads per KV head: it packs this position's K
// (qk-norm, RoPE) and V into the layer's KV row, prepares the GROUP query
// heads that read this KV head (q-norm factor on its 1/65536 grid, RoPE, q16),
// scores every position 0..pos (exact integer dot products, 1/1024 grid), forms
// the per-head (max, sum) statistics on their q16 grids and the weighted V sum.
// Scores and exponentials run one (head, position) per thread; the K row of a
// position is read as 16-byte vectors.  The two double-precision sums (sum of
// exp, sum over t of p*v) use a fixed order -- chunks of kChunk positions,
// each summed in position order, then the chunk sums in chunk order -- and the
// oracle sums in the same order, so the output is reproducible bit for bit.
//
// HBM layout of a layer's cache: seq rows of [K: kv_dim | V: kv_dim], int16
// little-endian (kv_bits 16, grid 1/2048) or int8 (kv_bits 8, grid 1/16).
// The reference's texel rows hold the same values in the same order
// (big-endian for q16); vgx_kv_read_rows / write_rows convert.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "vgx_internal.h"

#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 1024;
constexpr int kChunk = 32;  // positions per chunk of the summation order

}  // namespace

struct AttnDev {
    int dim, heads, kv_heads, hd, seq, kv_bits, rope_half, qk_norm, group;
    int row_bytes;
    int vR;      // chunks per round of the weighted-V pass
    int nchmax;  // chunks of a full cache
    // LDS byte offsets
    int o_ssk, o_mx, o_invs, o_newk, o_newv, o_qrot, o_sc, o_ep, o_csum, o_vpart, o_acc;
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
};

namespace {

__device__ __forceinline__ int q16_round(float v) {
    float f = floorf(v + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

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

__device__ __forceinline__ int lo16(unsigned w) { return (int)(short)(w & 0xffffu); }
__device__ __forceinline__ int hi16(unsigned w) { return (int)w >> 16; }
__device__ __forceinline__ int byte_s(unsigned w, int k) { return ((int)(w << (24 - 8 * k))) >> 24; }

// Exact q . k over one head: q from LDS (int32 per element), k one cache row's
// head slice read as 16-byte vectors (hd*KVB/8 bytes, 16-byte aligned).
template <int KVB>
__device__ __forceinline__ long long dot_row(const int* q, const uint8_t* k, int hd) {
    const uint4* kv4 = reinterpret_cast<const uint4*>(k);
    const int4* q4 = reinterpret_cast<const int4*>(q);
    long long d = 0;
    if (KVB == 16) {
        const int nv = hd / 8;
#pragma unroll 4
        for (int v = 0; v < nv; ++v) {
            const uint4 w = kv4[v];
            const int4 a = q4[2 * v], b = q4[2 * v + 1];
            d += (long long)a.x * lo16(w.x);
            d += (long long)a.y * hi16(w.x);
            d += (long long)a.z * lo16(w.y);
            d += (long long)a.w * hi16(w.y);
            d += (long long)b.x * lo16(w.z);
            d += (long long)b.y * hi16(w.z);
            d += (long long)b.z * lo16(w.w);
            d += (long long)b.w * hi16(w.w);
        }
    } else {
        const int nv = hd / 16;
#pragma unroll 2
        for (int v = 0; v < nv; ++v) {
            const uint4 w = kv4[v];
            const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int4 a = q4[4 * v + u];
                d += (long long)a.x * byte_s(ws[u], 0);
                d += (long long)a.y * byte_s(ws[u], 1);
                d += (long long)a.z * byte_s(ws[u], 2);
                d += (long long)a.w * byte_s(ws[u], 3);
            }
        }
    }
    return d;
}

template <int KVB>
__global__ void __launch_bounds__(kThreads) attn_kernel(const AttnDev A, uint8_t* kv, const int32_t* rtab,
                                                        const int16_t* qn, const int16_t* kn,
                                                        const int16_t* qkv, int16_t* out, int pos0,
                                                        int do_write, int do_attend) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int kvh = blockIdx.x;
    const int hd = A.hd, G = A.group, kv_dim = A.kv_heads * hd, GH = G * hd, seq = A.seq;
    const int tid = threadIdx.x;
    // blockIdx.y: the position's offset in a batch of consecutive positions,
    // whose qkv and output rows are consecutive rows
    const int pos = pos0 + blockIdx.y;
    qkv += (size_t)blockIdx.y * (A.dim + 2 * kv_dim);
    if (out) out += (size_t)blockIdx.y * A.dim;
    const int npos = pos + 1;
    const int nch = (npos + kChunk - 1) / kChunk;

    unsigned long long* ssk = reinterpret_cast<unsigned long long*>(smem + A.o_ssk);  // 1 + G
    float* mxs = reinterpret_cast<float*>(smem + A.o_mx);                             // G
    float* invs = reinterpret_cast<float*>(smem + A.o_invs);                          // G
    int* newk = reinterpret_cast<int*>(smem + A.o_newk);                              // hd
    int* newv = reinterpret_cast<int*>(smem + A.o_newv);                              // hd
    int* qrot = reinterpret_cast<int*>(smem + A.o_qrot);                              // G*hd
    int16_t* sc = reinterpret_cast<int16_t*>(smem + A.o_sc);                          // G*seq
    float* ep = reinterpret_cast<float*>(smem + A.o_ep);                              // G*seq
    double* csum = reinterpret_cast<double*>(smem + A.o_csum);                        // G*nchmax
    double* vpart = reinterpret_cast<double*>(smem + A.o_vpart);                      // vR*G*hd
    double* acc = reinterpret_cast<double*>(smem + A.o_acc);                          // G*hd

    if (tid <= G) ssk[tid] = 0ull;
    __syncthreads();

    const int16_t* kq = qkv + A.dim + kvh * hd;           // this head's K (q16)
    const int16_t* vq = qkv + A.dim + kv_dim + kvh * hd;  // and V
    uint8_t* row = kv + (size_t)pos * A.row_bytes;
    const int32_t* rt = rtab + (size_t)pos * (hd / 2) * 2;

    // sums of squares: K head (slot 0) and the G query heads (slots 1..G)
    if (A.qk_norm) {
        if (do_write && tid < hd) atomicAdd(&ssk[0], (unsigned long long)(long long)(kq[tid] * kq[tid]));
        if (do_attend) {
            for (int idx = tid; idx < GH; idx += kThreads) {
                const int g = idx / hd, i = idx - g * hd;
                const int v = qkv[(kvh * G + g) * hd + i];
                atomicAdd(&ssk[1 + g], (unsigned long long)(long long)(v * v));
            }
        }
    }
    __syncthreads();

    // --- KV pack of position pos (att_kv_rope)
    if (do_write && tid < hd) {
        float rk = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)(long long)ssk[0] * (1.0f / 65536.0f);
            rk = rsqrt_d(ss / (float)hd + 1e-6f);
        }
        const int i = tid;
        int j, ti;
        bool first;
        rope_pair(A.rope_half, hd, i, j, ti, first);
        float vv = (float)kq[i] / 256.0f, bb = (float)kq[j] / 256.0f;
        if (A.qk_norm) {
            vv = (vv * rk) * ((float)kn[i] / 256.0f);
            bb = (bb * rk) * ((float)kn[j] / 256.0f);
        }
        const float co = (float)rt[2 * ti] / 4096.0f, sn = (float)rt[2 * ti + 1] / 4096.0f;
        const float o = first ? (vv * co) - (bb * sn) : (bb * sn) + (vv * co);
        const int q = kv_enc<KVB>(o);
        kv_put<KVB>(row, kvh * hd + i, q);
        newk[i] = q;
        const int qv = kv_enc<KVB>((float)vq[i] / 256.0f);
        kv_put<KVB>(row, kv_dim + kvh * hd + i, qv);
        newv[i] = qv;
    }
    if (!do_attend) return;

    // --- q prep (att_qnorm_scale + att_qrot)
    for (int idx = tid; idx < GH; idx += kThreads) {
        const int g = idx / hd, i = idx - g * hd;
        const int h = kvh * G + g;
        const int16_t* qh = qkv + h * hd;
        float rq = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)(long long)ssk[1 + g] * (1.0f / 65536.0f);
            float r = rsqrt_d(ss / (float)hd + 1e-6f);
            r = fminf(r, 127.0f);
            rq = floorf(r * 65536.0f + 0.5f) / 65536.0f;
        }
        int j, ti;
        bool first;
        rope_pair(A.rope_half, hd, i, j, ti, first);
        float qv = (float)qh[i] / 256.0f, b = (float)qh[j] / 256.0f;
        if (A.qk_norm) {
            qv = (qv * rq) * ((float)qn[i] / 256.0f);
            b = (b * rq) * ((float)qn[j] / 256.0f);
        }
        const float co = (float)rt[2 * ti] / 4096.0f, sn = (float)rt[2 * ti + 1] / 4096.0f;
        const float o = first ? (qv * co) - (b * sn) : (b * sn) + (qv * co);
        qrot[idx] = q16_round(o * 256.0f);
    }
    __syncthreads();

    // --- scores (att_score): exact dot, times 1/sqrt(hd), 1/1024 grid; one
    // (position, head) per thread, the heads of a position in adjacent lanes
    const float invsqrt = 1.0f / sqrtf((float)hd);
    const float unit = KVB == 16 ? 1.0f / 524288.0f : 1.0f / 4096.0f;
    const uint8_t* khead = kv + (size_t)kvh * hd * (KVB / 8);
    for (int idx = tid; idx < G * npos; idx += kThreads) {
        const int t = idx / G, g = idx - t * G;
        const int* qg = qrot + g * hd;
        long long d = 0;
        if (t == pos && do_write) {
            for (int i = 0; i < hd; ++i) d += (long long)qg[i] * newk[i];
        } else {
            d = dot_row<KVB>(qg, khead + (size_t)t * A.row_bytes, hd);
        }
        const float s = (float)d * unit;
        float f = floorf((s * invsqrt) * 1024.0f + 0.5f);
        f = fminf(fmaxf(f, -32768.0f), 32767.0f);
        sc[(size_t)g * seq + t] = (int16_t)f;
    }
    __syncthreads();

    // --- stats (att_stats): max per head (exact), one wave per head
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += kThreads / 64) {
        int m = -32768;
        for (int t = lane; t < npos; t += 64) m = max(m, (int)sc[(size_t)g * seq + t]);
        for (int o = 32; o >= 1; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
        if (lane == 0) mxs[g] = (float)m / 1024.0f;
    }
    __syncthreads();
    for (int idx = tid; idx < G * npos; idx += kThreads) {
        const int g = idx / npos, t = idx - g * npos;
        ep[(size_t)g * seq + t] = exp_d((float)sc[(size_t)g * seq + t] / 1024.0f - mxs[g]);
    }
    __syncthreads();
    // chunk sums of exp, in position order within a chunk
    for (int idx = tid; idx < G * nch; idx += kThreads) {
        const int g = idx / nch, c = idx - g * nch;
        const int t0 = c * kChunk, t1 = min(t0 + kChunk, npos);
        const float* e = ep + (size_t)g * seq;
        double cs = 0.0;
        for (int t = t0; t < t1; ++t) cs += (double)e[t];
        csum[g * A.nchmax + c] = cs;
    }
    __syncthreads();
    if (tid < G) {
        const int g = tid;
        double sum = 0.0;
        for (int c = 0; c < nch; ++c) sum += csum[g * A.nchmax + c];
        const float fs = (float)sum;
        float qs = floorf(fs * 32.0f + 0.5f);
        qs = fminf(fmaxf(qs, -32768.0f), 32767.0f);
        const float sd = qs / 32.0f;
        invs[g] = sd > 0.0f ? 1.0f / sd : 0.0f;
    }
    __syncthreads();

    // --- weighted V (att_v): rounds of vR chunks; a thread sums one chunk of
    // one (head, element), then the round's chunk sums join the running total
    // in chunk order
    const float vunit = KVB == 16 ? 1.0f / 2048.0f : 1.0f / 16.0f;
    const uint8_t* vhead = kv + (size_t)(kv_dim + kvh * hd) * (KVB / 8);
    const bool own_last = do_write != 0;  // position pos comes from LDS
    for (int c0 = 0; c0 < nch; c0 += A.vR) {
        const int nr = min(A.vR, nch - c0);
        for (int idx = tid; idx < nr * GH; idx += kThreads) {
            const int r = idx / GH, gi = idx - r * GH;
            const int g = gi / hd, i = gi - g * hd;
            const int t0 = (c0 + r) * kChunk, t1 = min(t0 + kChunk, npos);
            const int tend = (own_last && t1 == npos) ? t1 - 1 : t1;
            const float* pg = ep + (size_t)g * seq;
            const float iv = invs[g];
            const uint8_t* vp = vhead + (size_t)i * (KVB / 8);
            double a = 0.0;
            int t = t0;
            for (; t + 8 <= tend; t += 8) {
                int q[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) q[u] = kv_get<KVB>(vp + (size_t)(t + u) * A.row_bytes, 0);
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float p = pg[t + u] * iv;
                    const float v = (float)q[u] * vunit;
                    a += (double)p * (double)v;
                }
            }
            for (; t < tend; ++t) {
                const float p = pg[t] * iv;
                const float v = (float)kv_get<KVB>(vp + (size_t)t * A.row_bytes, 0) * vunit;
                a += (double)p * (double)v;
            }
            if (tend != t1) {
                const float p = pg[pos] * iv;
                const float v = (float)newv[i] * vunit;
                a += (double)p * (double)v;
            }
            vpart[idx] = a;
        }
        __syncthreads();
        const bool last = c0 + nr >= nch;
        for (int gi = tid; gi < GH; gi += kThreads) {
            double s = c0 == 0 ? 0.0 : acc[gi];
            for (int r = 0; r < nr; ++r) s += vpart[r * GH + gi];
            if (last) {
                const int g = gi / hd, i = gi - g * hd;
                out[(kvh * G + g) * hd + i] = (int16_t)q16_round((float)s * 256.0f);
            } else {
                acc[gi] = s;
            }
        }
        __syncthreads();
    }
}

// LDS carve-up of one workgroup; returns the bytes used.
size_t attn_layout(AttnDev& A) {
    const int G = A.group, hd = A.hd, GH = G * hd;
    A.nchmax = (A.seq + kChunk - 1) / kChunk;
    A.vR = GH >= kThreads ? 1 : kThreads / GH;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = (off + bytes + 15) & ~(size_t)15;
        return (int)o;
    };
    A.o_ssk = take(8 * (size_t)(1 + G));
    A.o_mx = take(4 * (size_t)G);
    A.o_invs = take(4 * (size_t)G);
    A.o_newk = take(4 * (size_t)hd);
    A.o_newv = take(4 * (size_t)hd);
    A.o_qrot = take(4 * (size_t)GH);
    A.o_sc = take(2 * (size_t)G * A.seq);
    A.o_ep = take(4 * (size_t)G * A.seq);
    A.o_csum = take(8 * (size_t)G * A.nchmax);
    A.o_vpart = take(8 * (size_t)A.vR * GH);
    A.o_acc = take(8 * (size_t)GH);
    return off;
}

// Positions pos .. pos + ntok - 1 (their qkv and output rows consecutive).
// With ntok > 1 the KV write and the attention must be separate launches: a
// position reads the rows the others write.
int launch(vgx_attn* at, int layer, int pos, int ntok, const int16_t* qkv, int16_t* out, int w, int att) {
    if (!at) return vgx_fail(VGX_EINVAL, "attention: NULL handle");
    if (layer < 0 || layer >= at->layers || !at->kv[layer])
        return vgx_fail(VGX_ERANGE, "attention: layer " + std::to_string(layer) + " has no KV cache");
    if (ntok <= 0 || ntok > 65535) return vgx_fail(VGX_EINVAL, "attention: ntok outside 1..65535");
    if (pos < 0 || pos > at->a.seq - ntok)
        return vgx_fail(VGX_ERANGE, "attention: positions " + std::to_string(pos) + ".." +
                                        std::to_string(pos + ntok - 1) + " outside the KV length");
    if (!qkv || (att && !out)) return vgx_fail(VGX_EINVAL, "attention: NULL buffer");
    if (ntok > 1 && w && att) return vgx_fail(VGX_EINVAL, "attention: a batch writes its KV rows first");
    VGX_HIP(hipSetDevice(at->ctx->device));
    const AttnDev& A = at->a;
    const int16_t* qn = at->qn ? at->qn + (size_t)layer * A.hd : nullptr;
    const int16_t* kn = at->kn ? at->kn + (size_t)layer * A.hd : nullptr;
    const dim3 grid(A.kv_heads, ntok);
    if (A.kv_bits == 16)
        hipLaunchKernelGGL(attn_kernel<16>, grid, dim3(kThreads), at->lds, at->ctx->stream, A,
                           at->kv[layer], at->rtab, qn, kn, qkv, out, pos, w, att);
    else
        hipLaunchKernelGGL(attn_kernel<8>, grid, dim3(kThreads), at->lds, at->ctx->stream, A,
                           at->kv[layer], at->rtab, qn, kn, qkv, out, pos, w, att);
    VGX_LAUNCH_CHECK("attention launch");
    return VGX_OK;
}

}  // namespace

extern "C" {

int vgx_attn_create(vgx_ctx* ctx, const vgx_attn_desc* d, vgx_attn** out) {
    if (!ctx || !d || !out) return vgx_fail(VGX_EINVAL, "vgx_attn_create: NULL argument");
    *out = nullptr;
    if (d->dim <= 0 || d->heads <= 0 || d->kv_heads <= 0 || d->head_dim <= 0 || d->seq <= 0 || d->layers <= 0)
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: empty shape");
    if (d->heads % d->kv_heads) return vgx_fail(VGX_EINVAL, "vgx_attn_create: heads not a multiple of kv_heads");
    if (d->head_dim % 16 || d->head_dim > 256)
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: head_dim must be a multiple of 16, at most 256");
    if (d->heads / d->kv_heads > 16) return vgx_fail(VGX_EINVAL, "vgx_attn_create: more than 16 query heads per KV head");
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
    at->lds = attn_layout(A);
    if (at->lds > 160 * 1024) {
        delete at;
        return vgx_fail(VGX_EINVAL, "vgx_attn_create: seq too long for one workgroup's LDS");
    }
    auto fail = [&](hipError_t e, const char* w) { vgx_attn_free(at); return vgx_hip_fail(e, w); };
    const size_t lb = (size_t)A.seq * A.row_bytes;
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
    if (at->lds > 64 * 1024) {
        hipError_t a1 = hipFuncSetAttribute((const void*)attn_kernel<16>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)at->lds);
        hipError_t a2 = hipFuncSetAttribute((const void*)attn_kernel<8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)at->lds);
        if (a1 != hipSuccess) return fail(a1, "hipFuncSetAttribute");
        if (a2 != hipSuccess) return fail(a2, "hipFuncSetAttribute");
    }
    *out = at;
    return VGX_OK;
}

int vgx_attn_free(vgx_attn* at) {
    if (!at) return VGX_OK;
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

int vgx_kv_append_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv) {
    return launch(a, layer, pos0, ntok, qkv, nullptr, 1, 0);
}

int vgx_attn_decode_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos0, ntok, qkv, out, 0, 1);
}

int vgx_kv_row_bytes(const vgx_attn* a) { return a ? a->a.row_bytes : 0; }

int vgx_kv_read_rows(vgx_attn* at, int layer, int row0, int nrows, void* host) {
    if (!at || !host) return vgx_fail(VGX_EINVAL, "vgx_kv_read_rows: NULL argument");
    if (layer < 0 || layer >= at->layers || !at->kv[layer]) return vgx_fail(VGX_ERANGE, "vgx_kv_read_rows: bad layer");
    if (row0 < 0 || nrows < 0 || row0 + nrows > at->a.seq) return vgx_fail(VGX_ERANGE, "vgx_kv_read_rows: rows outside the cache");
    VGX_HIP(hipSetDevice(at->ctx->device));
    const size_t n = (size_t)nrows * at->a.row_bytes;
    VGX_HIP(hipStreamSynchronize(at->ctx->stream));
    VGX_HIP(hipMemcpy(host, at->kv[layer] + (size_t)row0 * at->a.row_bytes, n, hipMemcpyDeviceToHost));
    if (at->a.kv_bits == 16) {
        uint8_t* b = static_cast<uint8_t*>(host);
        for (size_t i = 0; i + 1 < n; i += 2) { uint8_t t = b[i]; b[i] = b[i + 1]; b[i + 1] = t; }
    }
    return VGX_OK;
}

int vgx_kv_write_rows(vgx_attn* at, int layer, int row0, int nrows, const void* host) {
    if (!at || !host) return vgx_fail(VGX_EINVAL, "vgx_kv_write_rows: NULL argument");
    if (layer < 0 || layer >= at->layers || !at->kv[layer]) return vgx_fail(VGX_ERANGE, "vgx_kv_write_rows: bad layer");
    if (row0 < 0 || nrows < 0 || row0 + nrows > at->a.seq) return vgx_fail(VGX_ERANGE, "vgx_kv_write_rows: rows outside the cache");
    VGX_HIP(hipSetDevice(at->ctx->device));
    const size_t n = (size_t)nrows * at->a.row_bytes;
    std::vector<uint8_t> tmp(static_cast<const uint8_t*>(host), static_cast<const uint8_t*>(host) + n);
    if (at->a.kv_bits == 16)
        for (size_t i = 0; i + 1 < n; i += 2) { uint8_t t = tmp[i]; tmp[i] = tmp[i + 1]; tmp[i + 1] = t; }
    VGX_HIP(hipStreamSynchronize(at->ctx->stream));
    VGX_HIP(hipMemcpy(at->kv[layer] + (size_t)row0 * at->a.row_bytes, tmp.data(), n, hipMemcpyHostToDevice));
    return VGX_OK;
}

}  // extern "C"
