// RMSNorm, the q8 embedding row, the decode step's device bookkeeping and the
// logits candidate pass.
#include <cmath>
#include <string>

#include "vgx_internal.h"
#include "vgx_qrow.h"

#pragma clang fp contract(off)

namespace {


// GPU::rmsnorm (engine/src/gpu_upload.cpp:280-365) as one workgroup:
// rms_stats_split's 32 partial sums of v^2 over contiguous slices of
// ceil(dim/32) values, each on the 1/4096 grid (P = sum x^2 in Q units, stored
// value floor(P/16 + 1/2)), their total ss, inv = inversesqrt(ss/dim + eps),
// y = q16(x * inv * w).  One workgroup per row of x (rows `dim` apart): slice
// p is 8 threads, thread `sub` taking elements p*per + sub + 8k.  REG (dim up
// to 2048, at most kNormRegs elements a thread): every x and w value is
// loaded at the start and kept in registers for the output, so the row is
// read once.  The slices' partials meet in LDS once and every wave adds the
// 32 itself (exact integers, so any order gives the same total).
constexpr int kNormRegs = 8;

template <bool REG>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const int16_t* x, const int16_t* w, int dim,
                                                       float eps, int16_t* y) {
    __shared__ long long part[32];
    x += (size_t)blockIdx.x * dim;
    y += (size_t)blockIdx.x * dim;
    const int per = (dim + 31) / 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int p = tid >> 3, sub = tid & 7, i0 = p * per + sub;
    auto in = [&](int k) { return sub + 8 * k < per && i0 + 8 * k < dim; };
    int xr[kNormRegs], wr[kNormRegs];
    long long P = 0;
    if (REG) {
#pragma unroll
        for (int k = 0; k < kNormRegs; ++k) {
            const int i = min(i0 + 8 * k, dim - 1);
            xr[k] = x[i];
            wr[k] = w[i];
        }
#pragma unroll
        for (int k = 0; k < kNormRegs; ++k)
            if (in(k)) P += (long long)xr[k] * xr[k];
    } else {
        for (int k = 0; sub + 8 * k < per; ++k)
            if (in(k)) P += (long long)x[i0 + 8 * k] * x[i0 + 8 * k];
    }
    // (the slice's 8 lanes and then the 32 slices joined by DPP: exact
    // integers, so the order does not matter)
    P = sum8_i64(P);
    if (sub == 0) part[p] = (P + 8) >> 4;
    __syncthreads();
    const long long tot = sum32_i64(part[lane & 31]);
    const float ss = (float)tot / 4096.0f;
    const float inv = (float)(1.0 / sqrt((double)(ss / (float)dim + eps)));
    auto put = [&](int i, int xi, int wi) {
        const float xv = (float)xi / 256.0f;
        const float wv = (float)wi / 256.0f;
        const float v = (xv * inv) * wv;
        y[i] = (int16_t)q16_round(v * 256.0f);
    };
    if (REG) {
#pragma unroll
        for (int k = 0; k < kNormRegs; ++k)
            if (in(k)) put(i0 + 8 * k, xr[k], wr[k]);
    } else {
        for (int k = 0; sub + 8 * k < per; ++k)
            if (in(k)) put(i0 + 8 * k, x[i0 + 8 * k], w[i0 + 8 * k]);
    }
}

// The instance for a row of dim values.
void (*rmsnorm_for(int dim))(const int16_t*, const int16_t*, int, float, int16_t*) {
    return (dim + 31) / 32 <= 8 * kNormRegs ? rmsnorm_kernel<true> : rmsnorm_kernel<false>;
}

// The q8 embedding row of token[blockIdx.x] (embed_q8_kernel's arithmetic)
// into x and its RMSNorm (rmsnorm_kernel's) into y, in one workgroup per row:
// rmsnorm_kernel<true>'s element mapping with the row formed in registers
// (rows of up to 2048 values), the norm weight loaded with the token.
__global__ void __launch_bounds__(256) embed_rms_kernel(const int8_t* emb, const float* scale, int vocab, int dim,
                                                         const int* token, const int16_t* w, float eps, int16_t* x,
                                                         int16_t* y) {
    __shared__ long long part[32];
    x += (size_t)blockIdx.x * dim;
    y += (size_t)blockIdx.x * dim;
    const int per = (dim + 31) / 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int p = tid >> 3, sub = tid & 7, i0 = p * per + sub;
    auto in = [&](int k) { return sub + 8 * k < per && i0 + 8 * k < dim; };
    int wr[kNormRegs];
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k) wr[k] = w[min(i0 + 8 * k, dim - 1)];
    int tok = token[blockIdx.x];
    tok = min(max(tok, 0), vocab - 1);
    const float sc = scale[tok];
    const int8_t* er = emb + (size_t)tok * dim;
    int xr[kNormRegs];
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k) {
        const float v = (float)er[min(i0 + 8 * k, dim - 1)] * sc;
        float r = __builtin_rintf(v * 256.0f);
        r = fminf(fmaxf(r, -32768.0f), 32767.0f);
        xr[k] = (int)r;
    }
    long long P = 0;
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k)
        if (in(k)) {
            P += (long long)xr[k] * xr[k];
            x[i0 + 8 * k] = (int16_t)xr[k];
        }
    // (the slice's 8 lanes and then the 32 slices joined by DPP: exact
    // integers, so the order does not matter)
    P = sum8_i64(P);
    if (sub == 0) part[p] = (P + 8) >> 4;
    __syncthreads();
    const long long tot = sum32_i64(part[lane & 31]);
    const float ss = (float)tot / 4096.0f;
    const float inv = (float)(1.0 / sqrt((double)(ss / (float)dim + eps)));
#pragma unroll
    for (int k = 0; k < kNormRegs; ++k)
        if (in(k)) {
            const float xv = (float)xr[k] / 256.0f;
            const float wv = (float)wr[k] / 256.0f;
            const float v = (xv * inv) * wv;
            y[i0 + 8 * k] = (int16_t)q16_round(v * 256.0f);
        }
}

// Session::embedding, q8 rows (engine/src/session.cpp:362-365).  Row
// blockIdx.y of x takes token[blockIdx.y].
__global__ void embed_q8_kernel(const int8_t* emb, const float* scale, int vocab, int dim,
                                const int* token, int16_t* x) {
    x += (size_t)blockIdx.y * dim;
    int tok = token[blockIdx.y];
    if (tok < 0) tok = 0;
    if (tok >= vocab) tok = vocab - 1;
    const float s = scale[tok];
    for (int i = threadIdx.x + blockIdx.x * blockDim.x; i < dim; i += blockDim.x * gridDim.x) {
        const float v = (float)emb[(size_t)tok * dim + i] * s;
        float r = __builtin_rintf(v * 256.0f);
        r = fminf(fmaxf(r, -32768.0f), 32767.0f);
        x[i] = (int16_t)r;
    }
}

// The candidate pass of GPU::logits_candidates_from (engine/src/gpu_matvec.cpp:
// 152-230; kernels top2 / top2_packed, engine/src/shaders_attn.cpp:477-494 and
// 574-594): chunk c covers logits [16c, min(16c + 16, n)), scanned in index
// order.  With strict comparisons v1/i1 is the chunk's first maximum and
// v2/i2 the first maximum of the rest (i2 = -1 for a one-logit chunk);
// (lm, ls) is the scan's running maximum and sum of exp((v - lm) * invt), the
// sum rescaled whenever the maximum grows and stored as
// floor(ls * 2048 + 1/2).  Values are q16 integers (the logit times 256).
// One thread per chunk; out holds 6 ints a chunk: v1, i1, v2, i2, lm, the
// stored sum.
__global__ void __launch_bounds__(256) chunks_kernel(const int16_t* logits, int n, float invt, int* out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= (n + 15) / 16) return;
    const int s = c * 16, e = min(s + 16, n);
    int v1 = logits[s], i1 = s, v2 = 0, i2 = -1;
    float lm = (float)v1 / 256.0f, ls = 1.0f;
    for (int i = s + 1; i < e; ++i) {
        const int q = logits[i];
        if (q > v1) {
            v2 = v1; i2 = i1; v1 = q; i1 = i;
        } else if (i2 < 0 || q > v2) {
            v2 = q; i2 = i;
        }
        const float v = (float)q / 256.0f;
        if (v > lm) {
            ls = ls * (float)exp((double)((lm - v) * invt)) + 1.0f;
            lm = v;
        } else {
            ls += (float)exp((double)((v - lm) * invt));
        }
    }
    int* o = out + (size_t)c * 6;
    o[0] = v1; o[1] = i1; o[2] = v2; o[3] = i2;
    o[4] = (int)lrintf(lm * 256.0f);
    o[5] = (int)floorf(ls * 2048.0f + 0.5f);
}

// One decode step's bookkeeping on the device: the token just chosen for
// position *pos + 1 goes to the history, and *pos advances.  One thread.
__global__ void advance_kernel(int* pos, const int* token, int* hist, int hist_len) {
    const int p = *pos;
    if (p + 1 >= 0 && p + 1 < hist_len) hist[p + 1] = *token;
    *pos = p + 1;
}

}  // namespace

extern "C" {

int vgx_decode_advance(vgx_ctx* ctx, int* pos, const int* token, int* hist, int hist_len) {
    if (!ctx || !pos || !token || !hist) return vgx_fail(VGX_EINVAL, "vgx_decode_advance: NULL argument");
    if (hist_len <= 0) return vgx_fail(VGX_EINVAL, "vgx_decode_advance: empty history");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, ctx->stream, pos, token, hist, hist_len);
    VGX_LAUNCH_CHECK("advance launch");
    return VGX_OK;
}

int vgx_logits_chunks(vgx_ctx* ctx, const int16_t* logits, int n, float temp, int* out) {
    if (!ctx || !logits || !out) return vgx_fail(VGX_EINVAL, "vgx_logits_chunks: NULL argument");
    if (n <= 0) return vgx_fail(VGX_EINVAL, "vgx_logits_chunks: empty logits row");
    if (!(temp == temp)) return vgx_fail(VGX_EINVAL, "vgx_logits_chunks: temperature is NaN");
    // the pass's uniform: invt = 1 / max(0.0001, temp) (engine/src/gpu_matvec.cpp:164)
    const float invt = 1.0f / (temp > 0.0001f ? temp : 0.0001f);
    const int nch = (n + 15) / 16;
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(chunks_kernel, dim3((nch + 255) / 256), dim3(256), 0, ctx->stream, logits, n, invt, out);
    VGX_LAUNCH_CHECK("logits chunks launch");
    return VGX_OK;
}

int vgx_rmsnorm(vgx_ctx* ctx, int dim, const int16_t* x, const int16_t* w, float eps, int16_t* y) {
    if (!ctx || !x || !w || !y) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm: NULL argument");
    if (dim <= 0 || dim > 65536) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm: dim outside 1..65536");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(rmsnorm_for(dim), dim3(1), dim3(256), 0, ctx->stream, x, w, dim, eps, y);
    VGX_LAUNCH_CHECK("rmsnorm launch");
    return VGX_OK;
}

int vgx_embed_q8(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim,
                 const int* token, int16_t* x) {
    if (!ctx || !emb || !emb_scale || !token || !x) return vgx_fail(VGX_EINVAL, "vgx_embed_q8: NULL argument");
    if (vocab <= 0 || dim <= 0) return vgx_fail(VGX_EINVAL, "vgx_embed_q8: empty shape");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(embed_q8_kernel, dim3(1), dim3(256), 0, ctx->stream, emb, emb_scale, vocab, dim, token, x);
    VGX_LAUNCH_CHECK("embed launch");
    return VGX_OK;
}

int vgx_rmsnorm_batch(vgx_ctx* ctx, int ntok, int dim, const int16_t* x, const int16_t* w, float eps,
                      int16_t* y) {
    if (!ctx || !x || !w || !y) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm_batch: NULL argument");
    if (dim <= 0 || dim > 65536) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm_batch: dim outside 1..65536");
    if (ntok <= 0 || ntok > 65535) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm_batch: ntok outside 1..65535");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(rmsnorm_for(dim), dim3(ntok), dim3(256), 0, ctx->stream, x, w, dim, eps, y);
    VGX_LAUNCH_CHECK("rmsnorm launch");
    return VGX_OK;
}

int vgx_embed_q8_batch(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim, int ntok,
                       const int* tokens, int16_t* x) {
    if (!ctx || !emb || !emb_scale || !tokens || !x) return vgx_fail(VGX_EINVAL, "vgx_embed_q8_batch: NULL argument");
    if (vocab <= 0 || dim <= 0) return vgx_fail(VGX_EINVAL, "vgx_embed_q8_batch: empty shape");
    if (ntok <= 0 || ntok > 65535) return vgx_fail(VGX_EINVAL, "vgx_embed_q8_batch: ntok outside 1..65535");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(embed_q8_kernel, dim3(1, ntok), dim3(256), 0, ctx->stream, emb, emb_scale, vocab, dim, tokens,
                       x);
    VGX_LAUNCH_CHECK("embed launch");
    return VGX_OK;
}

int vgx_embed_q8_rms_batch(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim, int ntok,
                           const int* tokens, int16_t* x, const int16_t* rms_w, float eps, int16_t* y) {
    if (!ctx || !emb || !emb_scale || !tokens || !x || !rms_w || !y)
        return vgx_fail(VGX_EINVAL, "vgx_embed_q8_rms_batch: NULL argument");
    if (vocab <= 0 || dim <= 0 || dim > 65536) return vgx_fail(VGX_EINVAL, "vgx_embed_q8_rms_batch: empty or oversized shape");
    if (ntok <= 0 || ntok > 65535) return vgx_fail(VGX_EINVAL, "vgx_embed_q8_rms_batch: ntok outside 1..65535");
    if ((dim + 31) / 32 > 8 * kNormRegs) {  // a row too long for the registers: the two launches
        const int st = vgx_embed_q8_batch(ctx, emb, emb_scale, vocab, dim, ntok, tokens, x);
        return st ? st : vgx_rmsnorm_batch(ctx, ntok, dim, x, rms_w, eps, y);
    }
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(embed_rms_kernel, dim3(ntok), dim3(256), 0, ctx->stream, emb, emb_scale, vocab, dim, tokens,
                       rms_w, eps, x, y);
    VGX_LAUNCH_CHECK("embed + rmsnorm launch");
    return VGX_OK;
}

}  // extern "C"
