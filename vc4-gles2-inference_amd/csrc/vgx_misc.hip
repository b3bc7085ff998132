// RMSNorm and the q8 embedding row.
#include <cmath>
#include <string>

#include "vgx_internal.h"

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ int q16_round(float v) {
    float f = floorf(v + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

// GPU::rmsnorm (engine/src/gpu_upload.cpp:280-365) as one workgroup:
// rms_stats_split's 32 partial sums of v^2 over contiguous slices of
// ceil(dim/32) values, each on the 1/4096 grid (P = sum x^2 in Q units, stored
// value floor(P/16 + 1/2)), their total ss, inv = inversesqrt(ss/dim + eps),
// y = q16(x * inv * w).  One workgroup per row of x (rows `dim` apart).
__global__ void __launch_bounds__(256) rmsnorm_kernel(const int16_t* x, const int16_t* w, int dim,
                                                       float eps, int16_t* y) {
    __shared__ long long part[32];
    __shared__ float s_inv;
    x += (size_t)blockIdx.x * dim;
    y += (size_t)blockIdx.x * dim;
    const int per = (dim + 31) / 32;
    const int tid = threadIdx.x;
    // 8 threads per partial slice
    {
        const int p = tid >> 3, sub = tid & 7;
        long long P = 0;
        for (int k = sub; k < per; k += 8) {
            const int i = p * per + k;
            if (i < dim) P += (long long)x[i] * x[i];
        }
        for (int o = 4; o >= 1; o >>= 1) P += __shfl_xor(P, o, 64);
        if (sub == 0) part[p] = (P + 8) >> 4;
    }
    __syncthreads();
    if (tid == 0) {
        long long tot = 0;
        for (int p = 0; p < 32; ++p) tot += part[p];
        const float ss = (float)tot / 4096.0f;
        s_inv = (float)(1.0 / sqrt((double)(ss / (float)dim + eps)));
    }
    __syncthreads();
    const float inv = s_inv;
    for (int i = tid; i < dim; i += blockDim.x) {
        const float xv = (float)x[i] / 256.0f;
        const float wv = (float)w[i] / 256.0f;
        const float v = (xv * inv) * wv;
        y[i] = (int16_t)q16_round(v * 256.0f);
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

int vgx_rmsnorm(vgx_ctx* ctx, int dim, const int16_t* x, const int16_t* w, float eps, int16_t* y) {
    if (!ctx || !x || !w || !y) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm: NULL argument");
    if (dim <= 0 || dim > 65536) return vgx_fail(VGX_EINVAL, "vgx_rmsnorm: dim outside 1..65536");
    VGX_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, ctx->stream, x, w, dim, eps, y);
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
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(ntok), dim3(256), 0, ctx->stream, x, w, dim, eps, y);
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

}  // extern "C"
