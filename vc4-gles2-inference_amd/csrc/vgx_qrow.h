// Device helpers shared by the GEMV, GEMM, norm and attention kernels: the
// byte dot products, the q16 store rounding, the RMSNorm output element and
// the byte planes of a q16 activation chunk.  Every kernel that reproduces a
// GEMV row or a normalised activation uses these same expressions, so the
// paths stay bit-identical.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#pragma clang fp contract(off)

namespace {

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
__device__ __forceinline__ uint32_t udot4(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_udot4(a, b, c, false);
}
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

// A 64-bit integer moved between lanes by one DPP control (both halves).
template <int CTRL>
__device__ __forceinline__ long long dpp_i64(long long x) {
    const unsigned long long b = (unsigned long long)x;
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
    return (long long)(((unsigned long long)hi << 32) | lo);
}
// The exact sum over each aligned group of 8 lanes, in every lane of the
// group: lane ^ 1, lane ^ 2 (quad permutes), then the half-row mirror.  Every
// lane of the wave active.
__device__ __forceinline__ long long sum8_i64(long long x) {
    x += dpp_i64<0xB1>(x);
    x += dpp_i64<0x4E>(x);
    x += dpp_i64<0x141>(x);
    return x;
}
// The exact sum over lanes 0..31 (the other lanes' values are ignored), in
// every lane: each row of 16 lanes summed by DPP, rows 0 and 1 read out.
// Every lane of the wave active.
__device__ __forceinline__ long long sum32_i64(long long x) {
    x = sum8_i64(x);
    x += dpp_i64<0x140>(x);
    const unsigned long long b = (unsigned long long)x;
    const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
    const unsigned long long r0 = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)hi, 0) << 32) |
                                  (unsigned)__builtin_amdgcn_readlane((int)lo, 0);
    const unsigned long long r1 = ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)hi, 16) << 32) |
                                  (unsigned)__builtin_amdgcn_readlane((int)lo, 16);
    return (long long)r0 + (long long)r1;
}

// clamp(floor(v + 0.5)) -- the shader's q16 store of a value in Q units.
__device__ __forceinline__ int q16_round(float v) {
    float f = floorf(v + 0.5f);
    f = fminf(fmaxf(f, -32768.0f), 32767.0f);
    return (int)f;
}

// GPU::rmsnorm's output element (engine/src/gpu_upload.cpp:280-365):
// q16(x * inv * w) with the shader's floor(v + 0.5) store.
__device__ __forceinline__ uint32_t rms_elem(uint32_t xv16, uint32_t wv16, float inv) {
    const float xv = (float)(int16_t)xv16 / 256.0f;
    const float wv = (float)(int16_t)wv16 / 256.0f;
    const float v = (xv * inv) * wv;
    return (uint32_t)(uint16_t)(int16_t)q16_round(v * 256.0f);
}

// Pack 16 q16 values (8 dwords, two per dword, element 2k in the low half)
// into the natural-order planes: xl[k] / xh[k] = low / high bytes of elements
// 4k..4k+3.
__device__ __forceinline__ void planes16(const uint32_t d[8], uint32_t xh[4], uint32_t xl[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        xl[k] = perm(d[2 * k + 1], d[2 * k], 0x06040200u);
        xh[k] = perm(d[2 * k + 1], d[2 * k], 0x07050301u);
    }
}

// q8: one chunk = 16 bytes of one row (q8u8: each weight + 128) = 16 columns,
// against the planes xh, xl of the same 16 activations:
//   sum (u-128)*x = 256*sdot4(u^0x80, xh) + udot4(u, xl) - 128*sum(xl)
// (the last term is the caller's, once per row).
__device__ __forceinline__ void q8_chunk(const uint4 w, const uint4 xh, const uint4 xl, int& s1,
                                         uint32_t& s2) {
    s1 = sdot4(w.x ^ 0x80808080u, xh.x, s1);
    s1 = sdot4(w.y ^ 0x80808080u, xh.y, s1);
    s1 = sdot4(w.z ^ 0x80808080u, xh.z, s1);
    s1 = sdot4(w.w ^ 0x80808080u, xh.w, s1);
    s2 = udot4(w.x, xl.x, s2);
    s2 = udot4(w.y, xl.y, s2);
    s2 = udot4(w.z, xl.z, s2);
    s2 = udot4(w.w, xl.w, s2);
}

}  // namespace
