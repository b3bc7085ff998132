// Decode attention over the packed KV cache, with the KV pack (append).
//
// One workgroup per KV head: it packs this position's K (qk-norm, RoPE) and V
// into the layer's KV row, prepares the GROUP query heads that read this KV
// head (q-norm factor on its 1/65536 grid, RoPE, q16), scores every position
// 0..pos (exact integer dot products, 1/1024 grid), forms the per-head
// (max, sum) statistics on their q16 grids and the weighted V sum.  The
// sequential reductions (sum of exp, sum over t of p*v) run in the same order
// as the oracle in double, so the output is reproducible bit for bit.
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

struct AttnDev {
    int dim, heads, kv_heads, hd, seq, kv_bits, rope_half, qk_norm, group;
    int row_bytes;
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

constexpr int kThreads = 256;

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

// Sum over a head (hd <= 256 values, one per thread i < hd) of v^2 as int64,
// through LDS atomics.
__device__ __forceinline__ void head_ss_add(unsigned long long* acc, long long v) {
    atomicAdd(acc, (unsigned long long)v);
}

template <int KVB>
__global__ void __launch_bounds__(kThreads) attn_kernel(const AttnDev A, uint8_t* kv, const int32_t* rtab,
                                                        const int16_t* qn, const int16_t* kn,
                                                        const int16_t* qkv, int16_t* out, int pos,
                                                        int do_write, int do_attend) {
    extern __shared__ uint8_t smem[];
    const int kvh = blockIdx.x;
    const int hd = A.hd, G = A.group, kv_dim = A.kv_heads * hd;
    const int half = hd / 2;
    const int tid = threadIdx.x;
    const int npos = pos + 1;

    // LDS carve-up
    unsigned long long* ssk = reinterpret_cast<unsigned long long*>(smem);  // 1 + G
    int* newk = reinterpret_cast<int*>(smem + 8 * 32);                     // hd
    int* newv = newk + 256;                                                // hd
    int* qrot = newv + 256;                                                // G*hd
    float* mxs = reinterpret_cast<float*>(qrot + 16 * 256);               // G
    float* invs = mxs + 16;                                                // G
    int16_t* sc = reinterpret_cast<int16_t*>(invs + 16);                   // G*seq
    float* ep = reinterpret_cast<float*>(sc + (size_t)G * A.seq + (A.seq & 1 ? G : 0));  // G*seq

    if (tid < 32) ssk[tid] = 0ull;
    __syncthreads();

    const int16_t* kq = qkv + A.dim + kvh * hd;          // this head's K (q16)
    const int16_t* vq = qkv + A.dim + kv_dim + kvh * hd; // and V
    uint8_t* row = kv + (size_t)pos * A.row_bytes;
    const int32_t* rt = rtab + (size_t)pos * half * 2;

    // sums of squares: K head (slot 0) and the G query heads (slots 1..G)
    if (A.qk_norm) {
        if (do_write && tid < hd) head_ss_add(&ssk[0], (long long)kq[tid] * kq[tid]);
        if (do_attend) {
            for (int idx = tid; idx < G * hd; idx += kThreads) {
                const int g = idx / hd, i = idx - g * hd;
                const int16_t v = qkv[(kvh * G + g) * hd + i];
                head_ss_add(&ssk[1 + g], (long long)v * v);
            }
        }
    }
    __syncthreads();

    // --- KV pack of position pos (att_kv_rope)
    if (do_write) {
        float rk = 1.0f;
        if (A.qk_norm) {
            const float ss = (float)(long long)ssk[0] * (1.0f / 65536.0f);
            rk = rsqrt_d(ss / (float)hd + 1e-6f);
        }
        if (tid < hd) {
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
    }
    if (!do_attend) return;

    // --- q prep (att_qnorm_scale + att_qrot)
    for (int idx = tid; idx < G * hd; idx += kThreads) {
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
        qrot[g * hd + i] = q16_round(o * 256.0f);
    }
    __syncthreads();

    // --- scores (att_score): exact dot, times 1/sqrt(hd), 1/1024 grid
    const float invsqrt = 1.0f / sqrtf((float)hd);
    const float unit = KVB == 16 ? 1.0f / 524288.0f : 1.0f / 4096.0f;
    for (int idx = tid; idx < G * npos; idx += kThreads) {
        const int g = idx / npos, t = idx - g * npos;
        const int* qg = qrot + g * hd;
        long long d = 0;
        if (t == pos && do_write) {
            for (int i = 0; i < hd; ++i) d += (long long)qg[i] * newk[i];
        } else {
            const uint8_t* r = kv + (size_t)t * A.row_bytes;
            for (int i = 0; i < hd; ++i) d += (long long)qg[i] * kv_get<KVB>(r, kvh * hd + i);
        }
        const float s = (float)d * unit;
        float f = floorf((s * invsqrt) * 1024.0f + 0.5f);
        f = fminf(fmaxf(f, -32768.0f), 32767.0f);
        sc[(size_t)g * A.seq + t] = (int16_t)f;
    }
    __syncthreads();

    // --- stats (att_stats): max per head (exact), exp per position, sequential sum
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += kThreads / 64) {
        int m = -32768;
        for (int t = lane; t < npos; t += 64) m = max(m, (int)sc[(size_t)g * A.seq + t]);
        for (int o = 32; o >= 1; o >>= 1) m = max(m, __shfl_xor(m, o, 64));
        if (lane == 0) mxs[g] = (float)m / 1024.0f;
    }
    __syncthreads();
    for (int idx = tid; idx < G * npos; idx += kThreads) {
        const int g = idx / npos, t = idx - g * npos;
        ep[(size_t)g * A.seq + t] = exp_d((float)sc[(size_t)g * A.seq + t] / 1024.0f - mxs[g]);
    }
    __syncthreads();
    if (tid < G) {
        const int g = tid;
        double sum = 0.0;
        for (int t = 0; t < npos; ++t) sum += (double)ep[(size_t)g * A.seq + t];
        const float fs = (float)sum;
        float qs = floorf(fs * 32.0f + 0.5f);
        qs = fminf(fmaxf(qs, -32768.0f), 32767.0f);
        const float sd = qs / 32.0f;
        invs[g] = sd > 0.0f ? 1.0f / sd : 0.0f;
        // the stored max is the grid value itself: mxs[g] already is q/1024
    }
    __syncthreads();
    for (int idx = tid; idx < G * npos; idx += kThreads) {
        const int g = idx / npos, t = idx - g * npos;
        ep[(size_t)g * A.seq + t] = ep[(size_t)g * A.seq + t] * invs[g];
    }
    __syncthreads();

    // --- weighted V (att_v)
    const float vunit = KVB == 16 ? 1.0f / 2048.0f : 1.0f / 16.0f;
    for (int idx = tid; idx < G * hd; idx += kThreads) {
        const int g = idx / hd, i = idx - g * hd;
        const float* pg = ep + (size_t)g * A.seq;
        double a = 0.0;
        for (int t = 0; t < npos; ++t) {
            const int q = (t == pos && do_write) ? newv[i]
                                                 : kv_get<KVB>(kv + (size_t)t * A.row_bytes, kv_dim + kvh * hd + i);
            const float v = (float)q * vunit;
            a += (double)pg[t] * (double)v;
        }
        out[(kvh * G + g) * hd + i] = (int16_t)q16_round((float)a * 256.0f);
    }
}

size_t attn_lds(const AttnDev& A) {
    // ssk(256 B) + newk/newv (2*256 ints) + qrot (16*256 ints) + mxs/invs (32 floats)
    size_t b = 256 + 2 * 256 * 4 + 16 * 256 * 4 + 32 * 4;
    b += (size_t)A.group * A.seq * 2 + (A.seq & 1 ? (size_t)A.group * 2 : 0);
    b += (size_t)A.group * A.seq * 4;
    return b;
}

int launch(vgx_attn* at, int layer, int pos, const int16_t* qkv, int16_t* out, int w, int att) {
    if (!at) return vgx_fail(VGX_EINVAL, "attention: NULL handle");
    if (layer < 0 || layer >= at->layers || !at->kv[layer])
        return vgx_fail(VGX_ERANGE, "attention: layer " + std::to_string(layer) + " has no KV cache");
    if (pos < 0 || pos >= at->a.seq)
        return vgx_fail(VGX_ERANGE, "attention: pos " + std::to_string(pos) + " outside the KV length");
    if (!qkv || (att && !out)) return vgx_fail(VGX_EINVAL, "attention: NULL buffer");
    VGX_HIP(hipSetDevice(at->ctx->device));
    const AttnDev& A = at->a;
    const int16_t* qn = at->qn ? at->qn + (size_t)layer * A.hd : nullptr;
    const int16_t* kn = at->kn ? at->kn + (size_t)layer * A.hd : nullptr;
    if (A.kv_bits == 16)
        hipLaunchKernelGGL(attn_kernel<16>, dim3(A.kv_heads), dim3(kThreads), at->lds, at->ctx->stream, A,
                           at->kv[layer], at->rtab, qn, kn, qkv, out, pos, w, att);
    else
        hipLaunchKernelGGL(attn_kernel<8>, dim3(A.kv_heads), dim3(kThreads), at->lds, at->ctx->stream, A,
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
    at->lds = attn_lds(A);
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
    return launch(a, layer, pos, qkv, nullptr, 1, 0);
}

int vgx_attn_decode(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos, qkv, out, 0, 1);
}

int vgx_attn_block(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out) {
    return launch(a, layer, pos, qkv, out, 1, 1);
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
