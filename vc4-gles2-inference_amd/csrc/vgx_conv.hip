// LFM2's gated short-convolution block between in_proj and out_proj
// (GPU::conv_block, engine/src/gpu_conv.cpp:165-225), for one position or a
// batch of consecutive positions.
//
// Per channel i and position t, from the q16 in_proj rows B, C, x
// (engine/src/model.cpp:1314-1316):
//   gated_t = q16(B/256 * x/256)                                mul_act
//   cv_t    = q16r(((k0*gated_{t-2} + k1*gated_{t-1}) + k2*gated_t) * 2^-8)
//                                                               conv3_act
//   y_t     = q16(C/256 * cv_t/256)                             mul_act
// (engine/src/shaders.cpp:1991-2051), fp32 in the shaders' order, operands of
// conv3 in q16 units, taps = q16 of the f32 kernel (set_conv_kernel,
// engine/src/gpu_conv.cpp:84-101).  The state is the last two gated values
// per layer.  One thread per channel walks the batch in position order, so a
// batch of n positions equals n single steps.
//
// HBM layout: taps [layers][3][dim] int16, state [layers][2][dim] int16
// (gated of pos-2, then pos-1).
#include <cmath>
#include <string>
#include <vector>

#include "vgx_internal.h"

#pragma clang fp contract(off)

struct vgx_conv {
    vgx_ctx* ctx = nullptr;
    int dim = 0, layers = 0;
    int16_t* taps = nullptr;
    int16_t* state = nullptr;
    std::vector<uint8_t> is_conv;
};

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int q16_store(float v) {
    float f = floorf(v * 256.0f + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

__device__ __forceinline__ int q16_round(float q) {
    float f = floorf(q + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

__global__ void __launch_bounds__(kThreads) conv_kernel(int dim, int ntok, const int16_t* bcx, const int16_t* taps,
                                                        int16_t* state, int16_t* y) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= dim) return;
    const float k0 = (float)taps[i], k1 = (float)taps[dim + i], k2 = (float)taps[2 * dim + i];
    int s2 = state[i], s1 = state[dim + i];
    for (int t = 0; t < ntok; ++t) {
        const int16_t* row = bcx + (size_t)t * 3 * dim;
        const float bv = (float)row[i] / 256.0f, cvv = (float)row[dim + i] / 256.0f;
        const float xv = (float)row[2 * dim + i] / 256.0f;
        const int g = q16_store(bv * xv);
        const float acc = ((k0 * (float)s2 + k1 * (float)s1) + k2 * (float)g) * 0.00390625f;
        const int cq = q16_round(acc);
        y[(size_t)t * dim + i] = (int16_t)q16_store(cvv * ((float)cq / 256.0f));
        s2 = s1;
        s1 = g;
    }
    state[i] = (int16_t)s2;
    state[dim + i] = (int16_t)s1;
}

// zero fill by a kernel (safe inside a captured graph)
__global__ void zero_kernel(int16_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace

extern "C" {

int vgx_conv_create(vgx_ctx* ctx, int dim, int layers, int kernel, const float* w, const uint8_t* layer_is_conv,
                    vgx_conv** out) {
    if (!ctx || !w || !out) return vgx_fail(VGX_EINVAL, "vgx_conv_create: NULL argument");
    *out = nullptr;
    if (dim <= 0 || layers <= 0) return vgx_fail(VGX_EINVAL, "vgx_conv_create: empty shape");
    if (kernel != 3) return vgx_fail(VGX_EINVAL, "vgx_conv_create: only the 3-tap kernel (LFM2's) is supported");
    VGX_HIP(hipSetDevice(ctx->device));
    vgx_conv* c = new vgx_conv();
    c->ctx = ctx;
    c->dim = dim;
    c->layers = layers;
    c->is_conv.assign((size_t)layers, 1);
    if (layer_is_conv)
        for (int l = 0; l < layers; ++l) c->is_conv[l] = layer_is_conv[l] ? 1 : 0;
    // set_conv_kernel: q16 = lrintf(w * 256), clamped; [layer][tap][channel]
    std::vector<int16_t> taps((size_t)layers * 3 * dim, 0);
    for (int l = 0; l < layers; ++l) {
        if (!c->is_conv[l]) continue;
        const float* wl = w + (size_t)l * dim * 3;
        for (int t = 0; t < 3; ++t)
            for (int i = 0; i < dim; ++i) {
                long q = lrintf(wl[(size_t)i * 3 + t] * 256.0f);
                taps[((size_t)l * 3 + t) * dim + i] = (int16_t)(q < -32768 ? -32768 : q > 32767 ? 32767 : q);
            }
    }
    const size_t sb = (size_t)layers * 2 * dim * sizeof(int16_t);
    hipError_t e = hipMalloc(&c->taps, taps.size() * sizeof(int16_t));
    if (e == hipSuccess) e = hipMemcpy(c->taps, taps.data(), taps.size() * sizeof(int16_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&c->state, sb);
    if (e == hipSuccess) e = hipMemset(c->state, 0, sb);
    if (e != hipSuccess) {
        vgx_conv_free(c);
        return vgx_hip_fail(e, "vgx_conv_create");
    }
    *out = c;
    return VGX_OK;
}

int vgx_conv_free(vgx_conv* c) {
    if (!c) return VGX_OK;
    if (c->taps) (void)hipFree(c->taps);
    if (c->state) (void)hipFree(c->state);
    delete c;
    return VGX_OK;
}

int vgx_conv_reset(vgx_conv* c) {
    if (!c) return vgx_fail(VGX_EINVAL, "vgx_conv_reset: NULL handle");
    VGX_HIP(hipSetDevice(c->ctx->device));
    const size_t n = (size_t)c->layers * 2 * c->dim;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024)), dim3(256), 0,
                       c->ctx->stream, c->state, n);
    VGX_LAUNCH_CHECK("conv reset");
    return VGX_OK;
}

int vgx_conv_step(vgx_conv* c, int layer, int ntok, const int16_t* bcx, int16_t* y) {
    if (!c || !bcx || !y) return vgx_fail(VGX_EINVAL, "vgx_conv_step: NULL argument");
    if (layer < 0 || layer >= c->layers || !c->is_conv[layer])
        return vgx_fail(VGX_ERANGE, "vgx_conv_step: layer " + std::to_string(layer) + " has no conv block");
    if (ntok <= 0) return vgx_fail(VGX_EINVAL, "vgx_conv_step: ntok must be positive");
    VGX_HIP(hipSetDevice(c->ctx->device));
    const int16_t* taps = c->taps + (size_t)layer * 3 * c->dim;
    int16_t* st = c->state + (size_t)layer * 2 * c->dim;
    hipLaunchKernelGGL(conv_kernel, dim3((c->dim + kThreads - 1) / kThreads), dim3(kThreads), 0, c->ctx->stream,
                       c->dim, ntok, bcx, taps, st, y);
    VGX_LAUNCH_CHECK("conv launch");
    return VGX_OK;
}

int vgx_conv_state_read(vgx_conv* c, int layer, int16_t* host) {
    if (!c || !host) return vgx_fail(VGX_EINVAL, "vgx_conv_state_read: NULL argument");
    if (layer < 0 || layer >= c->layers) return vgx_fail(VGX_ERANGE, "vgx_conv_state_read: bad layer");
    VGX_HIP(hipSetDevice(c->ctx->device));
    VGX_HIP(hipStreamSynchronize(c->ctx->stream));
    VGX_HIP(hipMemcpy(host, c->state + (size_t)layer * 2 * c->dim, (size_t)2 * c->dim * sizeof(int16_t),
                      hipMemcpyDeviceToHost));
    return VGX_OK;
}

int vgx_conv_state_write(vgx_conv* c, int layer, const int16_t* host) {
    if (!c || !host) return vgx_fail(VGX_EINVAL, "vgx_conv_state_write: NULL argument");
    if (layer < 0 || layer >= c->layers) return vgx_fail(VGX_ERANGE, "vgx_conv_state_write: bad layer");
    VGX_HIP(hipSetDevice(c->ctx->device));
    VGX_HIP(hipStreamSynchronize(c->ctx->stream));
    VGX_HIP(hipMemcpy(c->state + (size_t)layer * 2 * c->dim, host, (size_t)2 * c->dim * sizeof(int16_t),
                      hipMemcpyHostToDevice));
    return VGX_OK;
}

}  // extern "C"
