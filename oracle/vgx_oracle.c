/*
 * vgx_oracle.c -- CPU restatement of the reference's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker and the timed CPU baseline.  The
 * product never links or calls it.  Build: oracle/Makefile (gcc, -O3,
 * -ffp-contract=off, OpenMP over output rows).
 *
 * Paths in citations are relative to the reference repository root.
 */
#include "vgx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* (float)f((double)x): the build's definition of the shader's exp and
 * inversesqrt (the reference uses the GL driver's, which no test pins). */
static inline float exp_d(float x) { return (float)exp((double)x); }
static inline float rsqrt_d(float x) { return (float)(1.0 / sqrt((double)x)); }

static inline int clampi(long v, long lo, long hi) { return (int)(v < lo ? lo : v > hi ? hi : v); }

/* ======================================================================
 * Activation grid
 * ====================================================================== */

/* quantize_act, engine/src/common.h:188-195: lrintf (half-even), int16 rail. */
int16_t vgxo_quantize_act(float x) {
    long v = lrintf(x * 256.0f);
    return (int16_t)clampi(v, -32768, 32767);
}

void vgxo_quantize_act_n(const float* v, long n, int16_t* out) {
    for (long i = 0; i < n; ++i) out[i] = vgxo_quantize_act(v[i]);
}

/* x_per_texel / x_texels, engine/src/xformat.cpp:22-36. */
int vgxo_x_texels(int count, int fmt) {
    int n = (fmt == VGXO_I16_2 || fmt == VGXO_BF16) ? 2 : fmt == VGXO_I8_4 ? 4 : 1;
    return (count + n - 1) / n;
}

/* x_pack, engine/src/xformat.cpp:45-104: the bytes a value becomes in a texel. */
void vgxo_x_pack(const float* v, int count, int fmt, uint8_t* out) {
    const int texels = vgxo_x_texels(count, fmt);
    memset(out, 0, (size_t)texels * 4);
    for (int t = 0; t < texels; ++t) {
        uint8_t* p = out + (size_t)t * 4;
        if (fmt == VGXO_I16_1) {
            uint16_t q = (uint16_t)vgxo_quantize_act(v[t]);
            p[0] = (uint8_t)(q >> 8); p[1] = (uint8_t)q; p[2] = 0; p[3] = 255;
        } else if (fmt == VGXO_I24_1) {
            long q = lrintf(v[t] * 256.0f);
            q = (q < -8388608L ? -8388608L : q > 8388607L ? 8388607L : q) + 8388608L;
            p[0] = 0; p[1] = (uint8_t)(q >> 16); p[2] = (uint8_t)(q >> 8); p[3] = (uint8_t)q;
        } else if (fmt == VGXO_F32) {
            uint32_t u; memcpy(&u, &v[t], 4);
            p[0] = (uint8_t)(u >> 24); p[1] = (uint8_t)(u >> 16); p[2] = (uint8_t)(u >> 8); p[3] = (uint8_t)u;
        } else if (fmt == VGXO_BF16) {
            for (int k = 0; k < 2; ++k) {
                int i = 2 * t + k;
                uint32_t u = 0;
                if (i < count) memcpy(&u, &v[i], 4);
                uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
                p[2 * k] = (uint8_t)(r >> 8); p[2 * k + 1] = (uint8_t)r;
            }
        } else if (fmt == VGXO_I16_2) {
            uint16_t q0 = (uint16_t)vgxo_quantize_act(v[2 * t]);
            uint16_t q1 = 2 * t + 1 < count ? (uint16_t)vgxo_quantize_act(v[2 * t + 1]) : 0;
            p[0] = (uint8_t)(q0 >> 8); p[1] = (uint8_t)q0; p[2] = (uint8_t)(q1 >> 8); p[3] = (uint8_t)q1;
        } else { /* I8_4 */
            for (int k = 0; k < 4; ++k) {
                int i = 4 * t + k;
                int q = i < count ? (int)lrintf(v[i] * 16.0f) : 0;
                q = q < -127 ? -127 : q > 127 ? 127 : q;
                p[k] = (uint8_t)(q + 128);
            }
        }
    }
}

/* The shader-side q16 store: x_i16enc / x_q16enc, engine/src/xformat.cpp:205-209:
 * clamp(floor(v*256 + 0.5)). */
int16_t vgxo_q16_store(float v) {
    float q = v * 256.0f;
    float f = floorf(q + 0.5f);
    return (int16_t)(f < -32768.0f ? -32768 : f > 32767.0f ? 32767 : (int)f);
}

/* qz / x_q16enc on a value already in q16 units (engine/src/shaders.cpp:116-120). */
int16_t vgxo_q16_round(float q) {
    float f = floorf(q + 0.5f);
    return (int16_t)(f < -32768.0f ? -32768 : f > 32767.0f ? 32767 : (int)f);
}

/* ======================================================================
 * Packers: engine/tools/mmcf_hf.py, numpy float32 semantics (NEP 50: a
 * Python float against a float32 array is cast to float32 first).
 * ====================================================================== */

/* qmat, mmcf_hf.py:51-57.  s is the Python float mx/32767.0. */
void vgxo_qmat(const float* w, long n, int16_t* q, double* s) {
    float mx = 0.0f;
    for (long i = 0; i < n; ++i) { float a = fabsf(w[i]); if (a > mx) mx = a; }
    double m = mx == 0.0f ? 1.0 : (double)mx;
    double sd = m / 32767.0;
    float sf = (float)sd;
    for (long i = 0; i < n; ++i) {
        float r = rintf(w[i] / sf);
        r = r < -32767.0f ? -32767.0f : r > 32767.0f ? 32767.0f : r;
        q[i] = (int16_t)r;
    }
    *s = sd;
}

/* q8mat, mmcf_hf.py:60-66. */
void vgxo_q8mat(const float* w, long n, int8_t* q, double* s) {
    float mx = 0.0f;
    for (long i = 0; i < n; ++i) { float a = fabsf(w[i]); if (a > mx) mx = a; }
    double m = mx == 0.0f ? 1.0 : (double)mx;
    double sd = m / 127.0;
    float sf = (float)sd;
    for (long i = 0; i < n; ++i) {
        float r = rintf(w[i] / sf);
        r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
        q[i] = (int8_t)r;
    }
    *s = sd;
}

/* q8_from_i16, mmcf_hf.py:1821-1823: i16 first, dequantised, then q8. */
void vgxo_q8_from_i16(const float* w, long n, int8_t* q, double* s) {
    int16_t* q16 = (int16_t*)malloc((size_t)n * sizeof(int16_t));
    float* w2 = (float*)malloc((size_t)n * sizeof(float));
    double s16;
    vgxo_qmat(w, n, q16, &s16);
    float sf = (float)s16;
    for (long i = 0; i < n; ++i) w2[i] = (float)q16[i] * sf;
    vgxo_q8mat(w2, n, q, s);
    free(q16); free(w2);
}

/* q8_per_row, mmcf_hf.py:1825-1838: one scale per output row. */
void vgxo_q8_per_row(const float* w, int rows, int cols, int8_t* q, float* unit, float* plane) {
    float* s = (float*)malloc((size_t)rows * sizeof(float));
    float u = 0.0f;
    for (int r = 0; r < rows; ++r) {
        float mx = 0.0f;
        for (int c = 0; c < cols; ++c) { float a = fabsf(w[(size_t)r * cols + c]); if (a > mx) mx = a; }
        float sr = mx / 127.0f;
        if (sr == 0.0f) sr = 1.0f;
        s[r] = sr;
        if (sr > u) u = sr;
        for (int c = 0; c < cols; ++c) {
            float v = rintf(w[(size_t)r * cols + c] / sr);
            v = v < -127.0f ? -127.0f : v > 127.0f ? 127.0f : v;
            q[(size_t)r * cols + c] = (int8_t)v;
        }
    }
    for (int r = 0; r < rows; ++r) plane[r] = s[r] / u;
    *unit = u;
    free(s);
}

/* q4mat, mmcf_hf.py:69-91: groups of 32, asymmetric min/scale, nibbles with the
 * even column in the low nibble, int16 scale/min planes at one shared step ps. */
int vgxo_q4mat(const float* w, int rows, int cols, uint8_t* packed, int16_t* s16, int16_t* m16,
               double* ps) {
    if (cols % 32) return -1;
    const int groups = cols / 32;
    float* sc = (float*)malloc((size_t)rows * groups * sizeof(float));
    float* lo = (float*)malloc((size_t)rows * groups * sizeof(float));
    float asc = 0.0f, alo = 0.0f;
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < groups; ++g) {
            const float* z = w + (size_t)r * cols + (size_t)g * 32;
            float l = z[0], h = z[0];
            for (int k = 1; k < 32; ++k) { if (z[k] < l) l = z[k]; if (z[k] > h) h = z[k]; }
            float d = h - l;
            float s = d / 15.0f;
            if (s == 0.0f) s = 1.0f;
            sc[(size_t)r * groups + g] = s;
            lo[(size_t)r * groups + g] = l;
            if (fabsf(s) > asc) asc = fabsf(s);
            if (fabsf(l) > alo) alo = fabsf(l);
            for (int k = 0; k < 32; k += 2) {
                float n0 = rintf((z[k] - l) / s), n1 = rintf((z[k + 1] - l) / s);
                n0 = n0 < 0.0f ? 0.0f : n0 > 15.0f ? 15.0f : n0;
                n1 = n1 < 0.0f ? 0.0f : n1 > 15.0f ? 15.0f : n1;
                packed[(size_t)r * (cols / 2) + (size_t)g * 16 + k / 2] =
                    (uint8_t)((int)n0 | ((int)n1 << 4));
            }
        }
    }
    /* max(np.float32, np.float32, 1e-12) / 32767.0: a float32 division unless
     * the Python float wins, which then divides in double. */
    float m = asc > alo ? asc : alo;
    double psd = (double)m > 1e-12 ? (double)(m / 32767.0f) : 1e-12 / 32767.0;
    float psf = (float)psd;
    for (long i = 0; i < (long)rows * groups; ++i) {
        float a = rintf(sc[i] / psf), b = rintf(lo[i] / psf);
        a = a < -32767.0f ? -32767.0f : a > 32767.0f ? 32767.0f : a;
        b = b < -32767.0f ? -32767.0f : b > 32767.0f ? 32767.0f : b;
        s16[i] = (int16_t)a;
        m16[i] = (int16_t)b;
    }
    *ps = psd;
    free(sc); free(lo);
    return 0;
}

long vgxo_t3_bytes(int rows, int cols) {
    return (long)((rows + 1) / 2) * (long)(((cols + 7) / 8) * 4);
}

/* _t3_unpack, mmcf_hf.py:182-190 (and the host decode, engine/src/model.cpp:944-967):
 * texel (c, t) holds row 2t cols 8c..8c+3 (b0), 8c+4..8c+7 (b1), row 2t+1 in b2/b3;
 * weight k of a byte sits at bits 2k..2k+1. */
void vgxo_t3_codes(const uint8_t* packed, int rows, int cols, uint8_t* codes) {
    const long stride = ((cols + 7) / 8) * 4;
    for (int r = 0; r < rows; ++r) {
        const uint8_t* band = packed + (long)(r / 2) * stride;
        for (int x = 0; x < cols; ++x) {
            uint8_t byte = band[(long)(x >> 3) * 4 + (r & 1) * 2 + ((x >> 2) & 1)];
            codes[(long)r * cols + x] = (uint8_t)((byte >> (2 * (x & 3))) & 3u);
        }
    }
}

/* t3mat, mmcf_hf.py:112-165: certify per-row ternary, 2-bit codes (bit 0
 * magnitude, bit 1 sign), unit = largest row step, plane = step/unit.
 * Returns 0, or -1 when a row is not {0, +-s} (row_ternary, rtol 1e-3), or -2
 * when the decode round trip is not exact. */
int vgxo_t3mat(const float* w, int rows, int cols, uint8_t* packed, float* unit, float* plane) {
    float* s = (float*)malloc((size_t)rows * sizeof(float));
    const long stride = ((cols + 7) / 8) * 4;
    memset(packed, 0, (size_t)vgxo_t3_bytes(rows, cols));
    float u = 0.0f, wmax = 0.0f;
    int bad = 0;
    for (int r = 0; r < rows && !bad; ++r) {
        const float* wr = w + (size_t)r * cols;
        float mx = 0.0f;
        for (int c = 0; c < cols; ++c) { float a = fabsf(wr[c]); if (a > mx) mx = a; }
        if (mx > wmax) wmax = mx;
        for (int c = 0; c < cols; ++c) {
            float a = fabsf(wr[c]);
            if (a != 0.0f) {
                float rel = fabsf(a - mx) / (mx > 1e-30f ? mx : 1e-30f);
                if (rel > 1e-3f) { bad = 1; break; }
            }
        }
        float sr = mx / 127.0f;
        if (sr == 0.0f) sr = 1.0f;
        s[r] = sr;
        if (sr > u) u = sr;
        const float st = sr * 127.0f;
        uint8_t* band = packed + (long)(r / 2) * stride;
        for (int c = 0; c < cols; ++c) {
            float lev = rintf(wr[c] / st);
            unsigned code = (fabsf(lev) > 0.5f ? 1u : 0u) | (lev < -0.5f ? 2u : 0u);
            band[(long)(c >> 3) * 4 + (r & 1) * 2 + ((c >> 2) & 1)] |= (uint8_t)(code << (2 * (c & 3)));
        }
    }
    if (bad) { free(s); return -1; }
    /* the self-check: unpack * (s*127) must reproduce w to 1e-6 of max|w| */
    float err = 0.0f;
    for (int r = 0; r < rows; ++r) {
        const uint8_t* band = packed + (long)(r / 2) * stride;
        float st = s[r] * 127.0f;
        for (int c = 0; c < cols; ++c) {
            unsigned code = (band[(long)(c >> 3) * 4 + (r & 1) * 2 + ((c >> 2) & 1)] >> (2 * (c & 3))) & 3u;
            float mag = (float)(code & 1u), sgn = (float)((code >> 1) & 1u);
            float back = mag * (1.0f - 2.0f * sgn) * st;
            float d = fabsf(back - w[(size_t)r * cols + c]);
            if (d > err) err = d;
        }
    }
    if (err > 1e-6f * (wmax > 1.0f ? wmax : 1.0f)) { free(s); return -2; }
    for (int r = 0; r < rows; ++r) plane[r] = s[r] / u;
    *unit = u;
    free(s);
    return 0;
}

/* ======================================================================
 * Unpack / dequantise
 * ====================================================================== */

/* The per-row weight scale the kernels multiply by.  The part-3 plane is
 * re-quantised to 16 bits at upload (engine/src/gpu_upload.cpp:46-50, lrint
 * in double, clamped to [0, 65535]) and the shader rebuilds
 * (p16 * ws) * (1/65536) in fp32 (wrow_scale, engine/src/shaders.cpp:364-371).
 * Without a plane every row uses ws.  `scale` is the Mat's scale: the record
 * scale for q8, record scale * 127 for t3 (engine/src/model.cpp:927). */
void vgxo_row_scales(int rows, float scale, const float* plane, float* wsr) {
    for (int r = 0; r < rows; ++r) {
        if (!plane) { wsr[r] = scale; continue; }
        long q = lrint((double)plane[r] * 65536.0);
        if (q < 0) q = 0;
        if (q > 65535) q = 65535;
        float p16 = (float)q;
        wsr[r] = (p16 * scale) * (1.0f / 65536.0f);
    }
}

/* q8 level = byte - 128 for the biased q8u8 body (dtype 2, mmcf_pack.py:405-410,
 * shaders.cpp:392 `c*255-128`), the signed byte for q8i8. */
static inline int q8_level(uint8_t b, int prebiased) { return prebiased ? (int)b - 128 : (int)(int8_t)b; }

void vgxo_dequant_q8(const uint8_t* body, int prebiased, int rows, int cols, const float* wsr,
                     float* out) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c)
            out[(size_t)r * cols + c] = (float)q8_level(body[(size_t)r * cols + c], prebiased) * wsr[r];
}

/* q4 weight = n * (s16*ps) + m16*ps (engine/src/shaders.cpp:1259-1272). */
void vgxo_dequant_q4(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                     int rows, int cols, float* out) {
    const int groups = cols / 32;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            uint8_t b = nib[(size_t)r * (cols / 2) + c / 2];
            int n = (c & 1) ? (b >> 4) : (b & 15);
            float sa = (float)s16[(size_t)r * groups + c / 32] * ps;
            float ma = (float)m16[(size_t)r * groups + c / 32] * ps;
            out[(size_t)r * cols + c] = (float)n * sa + ma;
        }
}

static inline int t3_level(unsigned code) { return (code & 1u) ? ((code & 2u) ? -1 : 1) : 0; }

void vgxo_dequant_t3(const uint8_t* body, int rows, int cols, const float* wsr, float* out) {
    uint8_t* codes = (uint8_t*)malloc((size_t)rows * cols);
    vgxo_t3_codes(body, rows, cols, codes);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c)
            out[(size_t)r * cols + c] = (float)t3_level(codes[(size_t)r * cols + c]) * wsr[r];
    free(codes);
}

/* ======================================================================
 * Dequant-GEMV.  x is the q16 integer row (Q units).  The row value v_r is
 * what the shader rounds: s*ws_r for q8/t3 (matvec_q8_pair_logits,
 * shaders.cpp:704-747; matvec_q8_add_pair :1161-1214; matvec_t3_pair
 * :554-600) and the group-scaled sum for q4 (matvec_i4_add_pair :1322-1354).
 * ====================================================================== */

void vgxo_rowsum_q8(const uint8_t* body, int prebiased, int rows, int cols, const int16_t* x,
                    int64_t* s) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* wr = body + (size_t)r * cols;
        int64_t acc = 0;
        for (int c0 = 0; c0 < cols; c0 += 256) {
            int32_t part = 0; /* <= 256 * 128 * 32768 = 2^30 */
            const int c1 = c0 + 256 < cols ? c0 + 256 : cols;
            if (prebiased)
                for (int c = c0; c < c1; ++c) part += ((int32_t)wr[c] - 128) * (int32_t)x[c];
            else
                for (int c = c0; c < c1; ++c) part += (int32_t)(int8_t)wr[c] * (int32_t)x[c];
            acc += part;
        }
        s[r] = acc;
    }
}

void vgxo_rowval_q8(const uint8_t* body, int prebiased, int rows, int cols, const float* wsr,
                    const int16_t* x, float* v) {
    int64_t* s = (int64_t*)malloc((size_t)rows * sizeof(int64_t));
    vgxo_rowsum_q8(body, prebiased, rows, cols, x, s);
    for (int r = 0; r < rows; ++r) v[r] = (float)s[r] * wsr[r];
    free(s);
}

/* The literal fp32 order of the GLSL loop: four products a step, summed
 * left to right, then added to the running sum. */
void vgxo_rowval_q8_ref32(const uint8_t* body, int prebiased, int rows, int cols,
                          const float* wsr, const int16_t* x, float* v) {
    for (int r = 0; r < rows; ++r) {
        const uint8_t* wr = body + (size_t)r * cols;
        float s = 0.0f;
        for (int q = 0; q < cols / 4; ++q) {
            float w0 = (float)q8_level(wr[4 * q], prebiased), w1 = (float)q8_level(wr[4 * q + 1], prebiased);
            float w2 = (float)q8_level(wr[4 * q + 2], prebiased), w3 = (float)q8_level(wr[4 * q + 3], prebiased);
            float a = w0 * (float)x[4 * q];
            a = a + w1 * (float)x[4 * q + 1];
            a = a + w2 * (float)x[4 * q + 2];
            a = a + w3 * (float)x[4 * q + 3];
            s = s + a;
        }
        v[r] = s * wsr[r];
    }
}

/* q4: the weight is n*(s16*ps) + m16*ps per 32-group (the packed view,
 * engine/src/shaders.cpp:1784-1811), so a row value is
 *   sum_g ps*(s16_g*D_g + m16_g*X_g),  D = sum n*x, X = sum x.
 * The build takes the integer I = sum_g s16_g*D_g + m16_g*X_g exactly
 * (|D| < 2^24, |X| <= 2^20, |I| < 2^47) and rounds once, (float)I * ps: the
 * rule of q8's (float)S * wsr, and independent of the order groups are added
 * in.  The shader's own fp32 order is vgxo_rowval_q4_ref32. */
void vgxo_rowval_q4(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                    int rows, int cols, const int16_t* x, float* v) {
    const int groups = cols / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        int64_t I = 0;
        for (int g = 0; g < groups; ++g) {
            int32_t D = 0, X = 0;
            const uint8_t* b = nib + (size_t)r * (cols / 2) + (size_t)g * 16;
            const int16_t* xg = x + (size_t)g * 32;
            for (int k = 0; k < 16; ++k) {
                D += (int32_t)(b[k] & 15) * xg[2 * k] + (int32_t)(b[k] >> 4) * xg[2 * k + 1];
                X += xg[2 * k] + xg[2 * k + 1];
            }
            I += (int64_t)s16[(size_t)r * groups + g] * D + (int64_t)m16[(size_t)r * groups + g] * X;
        }
        v[r] = (float)I * ps;
    }
}

void vgxo_rowval_q4_ref32(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                          int rows, int cols, const int16_t* x, float* v) {
    const int groups = cols / 32;
    for (int r = 0; r < rows; ++r) {
        float s = 0.0f;
        for (int g = 0; g < groups; ++g) {
            int32_t D = 0, X = 0;
            const uint8_t* b = nib + (size_t)r * (cols / 2) + (size_t)g * 16;
            const int16_t* xg = x + (size_t)g * 32;
            for (int k = 0; k < 16; ++k) {
                D += (int32_t)(b[k] & 15) * xg[2 * k] + (int32_t)(b[k] >> 4) * xg[2 * k + 1];
                X += xg[2 * k] + xg[2 * k + 1];
            }
            float sa = (float)s16[(size_t)r * groups + g] * ps;
            float ma = (float)m16[(size_t)r * groups + g] * ps;
            float t1 = sa * (float)D, t2 = ma * (float)X;
            s = s + (t1 + t2);
        }
        v[r] = s;
    }
}

void vgxo_rowval_t3(const uint8_t* body, int rows, int cols, const float* wsr, const int16_t* x,
                    float* v) {
    const long stride = ((cols + 7) / 8) * 4;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* band = body + (long)(r / 2) * stride;
        int64_t s = 0;
        for (int c = 0; c < cols; ++c) {
            unsigned code = (band[(long)(c >> 3) * 4 + (r & 1) * 2 + ((c >> 2) & 1)] >> (2 * (c & 3))) & 3u;
            s += (int64_t)t3_level(code) * x[c];
        }
        v[r] = (float)s * wsr[r];
    }
}

void vgxo_rowval_t3_ref32(const uint8_t* body, int rows, int cols, const float* wsr,
                          const int16_t* x, float* v) {
    const long stride = ((cols + 7) / 8) * 4;
    for (int r = 0; r < rows; ++r) {
        const uint8_t* band = body + (long)(r / 2) * stride;
        float s = 0.0f;
        for (int g = 0; g < (cols + 7) / 8; ++g) {
            float part = 0.0f;
            for (int h = 0; h < 2; ++h) {
                uint8_t byte = band[(long)g * 4 + (r & 1) * 2 + h];
                float d = 0.0f;
                for (int k = 0; k < 4; ++k) {
                    int c = g * 8 + h * 4 + k;
                    float xv = c < cols ? (float)x[c] : 0.0f;
                    float t = (float)t3_level((byte >> (2 * k)) & 3u) * xv;
                    d = k == 0 ? t : d + t;
                }
                part = h == 0 ? d : part + d;
            }
            s = s + part;
        }
        v[r] = s * wsr[r];
    }
}

/* The q16 store with an optional residual in Q units: enc16(v + res), i.e.
 * clamp(floor(v + res + 0.5)) -- one rounding (matvec_q8_add_pair's inline
 * form, shaders.cpp:1188-1189; x_p2_stq for q4/t3). */
void vgxo_store(const float* v, const int16_t* res, int n, int16_t* y) {
    for (int i = 0; i < n; ++i) {
        float u = res ? v[i] + (float)res[i] : v[i];
        y[i] = vgxo_q16_round(u);
    }
}

/* fp32 output: the row value in activation units (v / 256, exact scaling). */
void vgxo_store_f32(const float* v, int n, float* y) {
    for (int i = 0; i < n; ++i) y[i] = v[i] * (1.0f / 256.0f);
}

/* SwiGLU of the fused gate (qz_sl, shaders.cpp:116-120; matvec_q8_pair_swiglu
 * :756-815): g = qz(v1), u = qz(v3), h = (a/(1+exp(-a)))*(u/256) with a = g/256,
 * times 2^-hs (metadata key 15), stored through x_st2. */
void vgxo_gate(const float* v1, const float* v3, int n, int hs, int16_t* h) {
    const float hsc = ldexpf(1.0f, -hs);
    for (int i = 0; i < n; ++i) {
        float g = (float)vgxo_q16_round(v1[i]);
        float u = (float)vgxo_q16_round(v3[i]);
        float a = g / 256.0f;
        float e = exp_d(-a);
        float d = 1.0f + e;
        float r = a / d;
        float o = r * (u / 256.0f);
        o = o * hsc;
        h[i] = vgxo_q16_store(o);
    }
}

/* The probes' acceptance reference (engine/probes/wrow_probe.cpp:356-372):
 * double accumulation, lrint, residual added after; the GPU may differ by one. */
void vgxo_probe_q8(const int8_t* w, int rows, int cols, const float* srow, float unit,
                   const int16_t* xq, const int16_t* res, int32_t* want) {
    for (int r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) acc += (double)w[(size_t)r * cols + c] * xq[c];
        double sc = srow ? (double)srow[r] * (double)unit : (double)unit;
        long v = lrint(acc * sc) + (res ? res[r] : 0);
        want[r] = clampi(v, -32768, 32767);
    }
}

/* ======================================================================
 * RMSNorm: rms_stats_split + rms_stats_reduce + rms_norm
 * (engine/src/shaders.cpp:1965-1988, 2062-2124; dispatch gpu_upload.cpp:280-365).
 * 32 partial sums of v^2 over contiguous slices of (dim+31)/32 values, each
 * stored on the 1/4096 grid, their sum (also on that grid) is ss; then
 * y = q16(x * inversesqrt(ss/dim + eps) * w).  v = x/256, so a partial is
 * P/65536 with P = sum x^2 and its stored value is floor(P/16 + 1/2).
 * ====================================================================== */
void vgxo_rmsnorm_stats(const int16_t* x, int dim, int64_t* partials32, int64_t* total) {
    const int per = (dim + 31) / 32;
    int64_t tot = 0;
    for (int p = 0; p < 32; ++p) {
        int64_t P = 0;
        for (int k = 0; k < per; ++k) {
            int i = p * per + k;
            if (i < dim) P += (int64_t)x[i] * x[i];
        }
        int64_t q = (P + 8) >> 4; /* floor(P/16 + 0.5), P >= 0 */
        if (partials32) partials32[p] = q;
        tot += q;
    }
    *total = tot;
}

void vgxo_rmsnorm(const int16_t* x, const int16_t* w, int dim, float eps, int16_t* y) {
    int64_t tot;
    vgxo_rmsnorm_stats(x, dim, 0, &tot);
    float ss = (float)tot / 4096.0f;
    float inv = rsqrt_d(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) {
        float xv = (float)x[i] / 256.0f;
        float wv = (float)w[i] / 256.0f;
        float v = (xv * inv) * wv;
        y[i] = vgxo_q16_store(v);
    }
}

/* ======================================================================
 * Attention (engine/src/shaders_attn.cpp; dispatch engine/src/gpu_attn.cpp).
 * The KV row of a position is the reference's texel row: K values then V
 * values, q16 as big-endian int16 (encKV, :133-135), q8 as two's-complement
 * bytes (encKV8, :144).  Grids: KV q16 2048, q8 16 (gpu_attn.cpp:89-90);
 * score 1024, sum 32 (shaders.h:13-14).
 * ====================================================================== */

/* Session's rope tables, engine/src/session.cpp:188-202. */
void vgxo_rope_cos_sin(float theta, int head_dim, int seq, float* rcos, float* rsin) {
    const int half = head_dim / 2;
    for (int p = 0; p < seq; ++p)
        for (int i = 0; i < half; ++i) {
            float freq = 1.0f / powf(theta, (2.0f * i) / head_dim);
            float a = p * freq;
            rcos[(size_t)p * half + i] = cosf(a);
            rsin[(size_t)p * half + i] = sinf(a);
        }
}

/* The 24-bit RoPE texture at 1/4096, engine/src/gpu_attn.cpp:142-156:
 * tab[(p*half + i)*2 + {0,1}] = lrintf(cos*4096), lrintf(sin*4096). */
void vgxo_rope_table(const float* rcos, const float* rsin, int seq, int half, int32_t* tab) {
    for (long k = 0; k < (long)seq * half; ++k) {
        tab[2 * k] = (int32_t)lrintf(rcos[k] * 4096.0f);
        tab[2 * k + 1] = (int32_t)lrintf(rsin[k] * 4096.0f);
    }
}

int vgxo_kv_row_bytes(const vgxo_attn_cfg* c) {
    const int kv_dim = c->kv_heads * c->head_dim;
    return c->kv_bits == 16 ? 4 * kv_dim : 2 * kv_dim;
}

static inline float kv_scale(const vgxo_attn_cfg* c) { return c->kv_bits == 16 ? 2048.0f : 16.0f; }

/* decKV (shaders_attn.cpp:136-138, 144-145): value idx of a row (K in
 * [0,kv_dim), V in [kv_dim, 2 kv_dim)). */
static inline int kv_int(const vgxo_attn_cfg* c, const uint8_t* row, int idx) {
    if (c->kv_bits == 16) {
        int u = ((int)row[2 * idx] << 8) | row[2 * idx + 1];
        return u >= 32768 ? u - 65536 : u;
    }
    return (int)(int8_t)row[idx];
}

float vgxo_kv_decode(const vgxo_attn_cfg* c, const uint8_t* row, int idx) {
    return (float)kv_int(c, row, idx) / kv_scale(c);
}

static inline void kv_put(const vgxo_attn_cfg* c, uint8_t* row, int idx, float v) {
    float f = floorf(v * kv_scale(c) + 0.5f);
    if (c->kv_bits == 16) {
        int q = f < -32768.0f ? -32768 : f > 32767.0f ? 32767 : (int)f;
        uint16_t u = (uint16_t)q;
        row[2 * idx] = (uint8_t)(u >> 8);
        row[2 * idx + 1] = (uint8_t)u;
    } else {
        int q = f < -128.0f ? -128 : f > 127.0f ? 127 : (int)f;
        row[idx] = (uint8_t)(int8_t)q;
    }
}

/* partner index and rope slot of element i of a head (qval / att_kv_rope). */
static inline void rope_pair(const vgxo_attn_cfg* c, int i, int* j, int* ti, int* first) {
    const int half = c->head_dim / 2;
    if (c->rope_half) {
        if (i < half) { *j = i + half; *ti = i; *first = 1; }
        else { *j = i - half; *ti = i - half; *first = 0; }
    } else {
        int even = (i & 1) == 0;
        *j = even ? i + 1 : i - 1;
        *ti = i / 2;
        *first = even;
    }
}

/* sum of squares of one head in Q units, as the fp32 value the shader forms */
static inline float head_ss(const int16_t* v, int hd) {
    int64_t s = 0;
    for (int z = 0; z < hd; ++z) s += (int64_t)v[z] * v[z];
    return (float)s * (1.0f / 65536.0f);
}

/* att_kv_rope, shaders_attn.cpp:162-241 (q16 branch :200-229, q8 :165-199):
 * K is qk-normed (inversesqrt(mean(k^2)+1e-6) times the q16 k_norm weight),
 * rotated with the 1/4096 table and packed; V is packed unchanged. */
void vgxo_kv_write(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* kn, const int32_t* rtab,
                   int pos, uint8_t* row) {
    const int hd = c->head_dim, half = hd / 2, kv_dim = c->kv_heads * hd;
    const int16_t* k = qkv + c->dim;
    const int16_t* v = qkv + c->dim + kv_dim;
    for (int h = 0; h < c->kv_heads; ++h) {
        const int16_t* kh = k + h * hd;
        float rk = 1.0f;
        if (c->qk_norm) rk = rsqrt_d(head_ss(kh, hd) / (float)hd + 1e-6f);
        for (int i = 0; i < hd; ++i) {
            int j, ti, first;
            rope_pair(c, i, &j, &ti, &first);
            float vv = (float)kh[i] / 256.0f, bb = (float)kh[j] / 256.0f;
            if (c->qk_norm) {
                vv = (vv * rk) * ((float)kn[i] / 256.0f);
                bb = (bb * rk) * ((float)kn[j] / 256.0f);
            }
            const int32_t* rt = rtab + ((size_t)pos * half + ti) * 2;
            float co = (float)rt[0] / 4096.0f, sn = (float)rt[1] / 4096.0f;
            float o = first ? (vv * co) - (bb * sn) : (bb * sn) + (vv * co);
            kv_put(c, row, h * hd + i, o);
        }
    }
    for (int i = 0; i < kv_dim; ++i) kv_put(c, row, kv_dim + i, (float)v[i] / 256.0f);
}

/* att_qnorm_scale (:259-268) and att_qrot (:270-296): the per-head q factor is
 * min(inversesqrt(mean(q^2)+1e-6), 127) stored on a 1/65536 grid; q is normed,
 * rotated and stored as q16. */
void vgxo_q_rot(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* qn, const int32_t* rtab,
                int pos, int16_t* qrot) {
    const int hd = c->head_dim, half = hd / 2;
    for (int h = 0; h < c->heads; ++h) {
        const int16_t* qh = qkv + h * hd;
        float rq = 1.0f;
        if (c->qk_norm) {
            float r = rsqrt_d(head_ss(qh, hd) / (float)hd + 1e-6f);
            if (r > 127.0f) r = 127.0f;
            rq = floorf(r * 65536.0f + 0.5f) / 65536.0f;
        }
        for (int i = 0; i < hd; ++i) {
            int j, ti, first;
            rope_pair(c, i, &j, &ti, &first);
            float qv = (float)qh[i] / 256.0f, b = (float)qh[j] / 256.0f;
            if (c->qk_norm) {
                qv = (qv * rq) * ((float)qn[i] / 256.0f);
                b = (b * rq) * ((float)qn[j] / 256.0f);
            }
            const int32_t* rt = rtab + ((size_t)pos * half + ti) * 2;
            float co = (float)rt[0] / 4096.0f, sn = (float)rt[1] / 4096.0f;
            float o = first ? (qv * co) - (b * sn) : (b * sn) + (qv * co);
            qrot[h * hd + i] = vgxo_q16_store(o);
        }
    }
}

/* att_score (:308-332): s = sum q*k over the head, times 1/sqrt(hd), on the
 * 1/1024 grid (q16 clamp).  The dot of two integer grids is exact here. */
void vgxo_attn_scores(const vgxo_attn_cfg* c, const int16_t* qrot, const uint8_t* kv, int pos,
                      int16_t* scores) {
    const int hd = c->head_dim, group = c->heads / c->kv_heads;
    const int rb = vgxo_kv_row_bytes(c);
    const float invsqrt = 1.0f / sqrtf((float)hd);
    const float unit = c->kv_bits == 16 ? 1.0f / 524288.0f : 1.0f / 4096.0f; /* 1/(256*kvscale) */
    for (int h = 0; h < c->heads; ++h) {
        const int kvh = h / group;
        for (int t = 0; t <= pos; ++t) {
            const uint8_t* row = kv + (size_t)t * rb;
            int64_t d = 0;
            for (int i = 0; i < hd; ++i) d += (int64_t)qrot[h * hd + i] * kv_int(c, row, kvh * hd + i);
            float s = (float)d * unit;
            float f = floorf((s * invsqrt) * 1024.0f + 0.5f);
            scores[(size_t)h * c->seq + t] = (int16_t)(f < -32768.0f ? -32768 : f > 32767.0f ? 32767 : (int)f);
        }
    }
}

/* att_stats (:334-369), linear sum grid: per head (max, sum exp(s - max)) as
 * two q16 values at scales 1024 and 32.  st[2h] = max, st[2h+1] = sum.
 *
 * The build's summation order for both attention sums (this one and att_v's):
 * positions in chunks of VGXO_ATTN_CHUNK, each chunk summed in double in
 * position order from 0.0, then the chunk sums added in chunk order from 0.0.
 * With at most one chunk this is the plain sequential sum. */
void vgxo_attn_stats(const vgxo_attn_cfg* c, const int16_t* scores, int pos, int16_t* st) {
    for (int h = 0; h < c->heads; ++h) {
        const int16_t* sc = scores + (size_t)h * c->seq;
        float mx = -1e30f;
        for (int t = 0; t <= pos; ++t) { float s = (float)sc[t] / 1024.0f; if (s > mx) mx = s; }
        double sum = 0.0;
        for (int t0 = 0; t0 <= pos; t0 += VGXO_ATTN_CHUNK) {
            double cs = 0.0;
            for (int t = t0; t <= pos && t < t0 + VGXO_ATTN_CHUNK; ++t)
                cs += (double)exp_d((float)sc[t] / 1024.0f - mx);
            sum += cs;
        }
        float fs = (float)sum;
        float qm = floorf(mx * 1024.0f + 0.5f), qs = floorf(fs * 32.0f + 0.5f);
        st[2 * h] = (int16_t)(qm < -32768.0f ? -32768 : qm > 32767.0f ? 32767 : (int)qm);
        st[2 * h + 1] = (int16_t)(qs < -32768.0f ? -32768 : qs > 32767.0f ? 32767 : (int)qs);
    }
}

/* att_v (:383-459): p_t = exp(s_t - max) / sum from the stored stats, out =
 * q16(sum_t p_t v_t); the build accumulates p*v in double, in the chunked
 * order of vgxo_attn_stats. */
void vgxo_attn_v(const vgxo_attn_cfg* c, const int16_t* scores, const int16_t* st, const uint8_t* kv,
                 int pos, int16_t* out) {
    const int hd = c->head_dim, group = c->heads / c->kv_heads, kv_dim = c->kv_heads * hd;
    const int rb = vgxo_kv_row_bytes(c);
    for (int h = 0; h < c->heads; ++h) {
        const int kvh = h / group;
        const float mx = (float)st[2 * h] / 1024.0f;
        const float sum = (float)st[2 * h + 1] / 32.0f;
        const float invs = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int i = 0; i < hd; ++i) {
            double a = 0.0;
            for (int t0 = 0; t0 <= pos; t0 += VGXO_ATTN_CHUNK) {
                double ca = 0.0;
                for (int t = t0; t <= pos && t < t0 + VGXO_ATTN_CHUNK; ++t) {
                    float p = exp_d((float)scores[(size_t)h * c->seq + t] / 1024.0f - mx) * invs;
                    float v = vgxo_kv_decode(c, kv + (size_t)t * rb, kv_dim + kvh * hd + i);
                    ca += (double)p * (double)v;
                }
                a += ca;
            }
            out[h * hd + i] = vgxo_q16_store((float)a);
        }
    }
}

/* attention_block after the qkv draw (gpu_attn.cpp:187-241): KV write of this
 * position into kv (seq rows of kv_row_bytes), then q, scores, stats, v. */
void vgxo_attn_block(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* qn, const int16_t* kn,
                     const int32_t* rtab, int pos, uint8_t* kv, int16_t* out) {
    const int rb = vgxo_kv_row_bytes(c);
    int16_t* qrot = (int16_t*)malloc((size_t)c->dim * sizeof(int16_t));
    int16_t* scores = (int16_t*)calloc((size_t)c->heads * c->seq, sizeof(int16_t));
    int16_t* st = (int16_t*)malloc((size_t)c->heads * 2 * sizeof(int16_t));
    vgxo_kv_write(c, qkv, kn, rtab, pos, kv + (size_t)pos * rb);
    vgxo_q_rot(c, qkv, qn, rtab, pos, qrot);
    vgxo_attn_scores(c, qrot, kv, pos, scores);
    vgxo_attn_stats(c, scores, pos, st);
    vgxo_attn_v(c, scores, st, kv, pos, out);
    free(qrot); free(scores); free(st);
}

/* ======================================================================
 * LFM2 conv block (GPU::conv_block, engine/src/gpu_conv.cpp:165-225)
 * ====================================================================== */

/* GPU::set_conv_kernel (engine/src/gpu_conv.cpp:84-101): the f32 depthwise
 * kernel w[i*k + t] as q16 taps lrintf(w*256), clamped; taps[t*dim + i]. */
void vgxo_conv_taps(const float* w, int dim, int k, int16_t* taps) {
    for (int t = 0; t < k; ++t)
        for (int i = 0; i < dim; ++i) taps[(size_t)t * dim + i] = vgxo_quantize_act(w[(size_t)i * k + t]);
}

/* One position of the conv block after in_proj.  bcx = the q16 in_proj
 * output (matvec_to stores x_i24encq, which clamps to the q16 range,
 * engine/src/shaders.cpp:61; rows B, C, x in that order, model.cpp:1314-1316);
 * s2 / s1 = the gated values of positions pos-2 / pos-1 (q16), updated in
 * place; y = the q16 input of out_proj.  Per channel:
 *   gated = x_st2(b/256 * x/256)                        (mul_act, shaders.cpp:2011)
 *   cv    = x_st2q(((k0*s2 + k1*s1) + k2*gated) * 2^-8) (conv3_act, :2025-2051;
 *           every operand in q16 units, fp32, left to right)
 *   y     = x_st2(c/256 * cv/256)                       (mul_act) */
void vgxo_conv_step(int dim, const int16_t* bcx, const int16_t* taps, int16_t* s2, int16_t* s1, int16_t* y) {
    for (int i = 0; i < dim; ++i) {
        const float bv = (float)bcx[i] / 256.0f, cvv = (float)bcx[dim + i] / 256.0f;
        const float xv = (float)bcx[2 * dim + i] / 256.0f;
        const int16_t g = vgxo_q16_store(bv * xv);
        const float k0 = (float)taps[i], k1 = (float)taps[dim + i], k2 = (float)taps[2 * dim + i];
        const float acc = ((k0 * (float)s2[i] + k1 * (float)s1[i]) + k2 * (float)g) * 0.00390625f;
        const int16_t cq = vgxo_q16_round(acc);
        y[i] = vgxo_q16_store(cvv * ((float)cq / 256.0f));
        s2[i] = s1[i];
        s1[i] = g;
    }
}

/* ======================================================================
 * Embedding, argmax
 * ====================================================================== */

/* Session::embedding, q8 row branch (engine/src/session.cpp:362-365): the
 * signed q8 row times its scale, on the host q16 grid (lrintf). */
void vgxo_embed_q8(const int8_t* emb, const float* emb_scale, int dim, int token, int16_t* x) {
    const float s = emb_scale[token];
    for (int i = 0; i < dim; ++i) x[i] = vgxo_quantize_act((float)emb[(size_t)token * dim + i] * s);
}

/* argmax_token (engine/src/sampling.cpp:160-162): the first maximum wins. */
int vgxo_argmax_i16(const int16_t* v, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i) if (v[i] > v[best]) best = i;
    return best;
}

/* ======================================================================
 * Float path (engine/tools/ref_forward.py:35-115): fp32 values, the dot
 * products accumulated in double, OpenMP over rows.
 * ====================================================================== */
void vgxo_matvec_f32(const float* w, int rows, int cols, const float* x, float* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* wr = w + (size_t)r * cols;
        double acc = 0.0;
        for (int c = 0; c < cols; ++c) acc += (double)wr[c] * (double)x[c];
        y[r] = (float)acc;
    }
}

void vgxo_rms_f32(const float* x, const float* w, int n, float eps, float* y) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    float inv = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * (w ? w[i] : 1.0f);
}

int vgxo_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void vgxo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
