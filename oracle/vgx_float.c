/*
 * The reference's float CPU path in C with OpenMP: engine/tools/ref_forward.py
 * semantics (the float32 forward over the dequantised container weights, as
 * oracle/model.py FModel restates it in numpy), for the CPU baseline of the
 * decode benchmarks.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/ use it; the
 * product never does.  The matrices are the float32 arrays FModel dequantises
 * (row-major, rows x cols); every matrix-vector product is parallel over rows,
 * each row a float32 dot product in 8-wide FMA partial sums, so the results
 * differ from numpy's in summation order only (tests/test_oracle_model.py
 * bounds the difference).
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vgx_float.h"

struct vgxf_state {
    float *kc, *vc;       /* layers x seq x kv_dim */
    float* cst;           /* layers x 2 x dim: B*x of pos-2, pos-1 (conv layers) */
    float *x, *xn, *qkv, *att, *g, *u, *bcx, *t; /* activations */
    float* sc;            /* heads x seq scores */
};

static float dot(const float* w, const float* x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    int k = 0;
    for (; k + 16 <= n; k += 16) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k), _mm256_loadu_ps(x + k), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k + 8), _mm256_loadu_ps(x + k + 8), a1);
    }
    a0 = _mm256_add_ps(a0, a1);
    float s[8];
    _mm256_storeu_ps(s, a0);
    float r = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; k < n; ++k) r += w[k] * x[k];
    return r;
}

/* y = W x, W rows x cols */
static void matvec(const float* W, const float* x, int rows, int cols, float* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) y[r] = dot(W + (size_t)r * cols, x, cols);
}

static void rms(const float* x, const float* w, int n, float eps, float* y) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    const float inv = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * w[i];
}

static void rope(float* v, const float* c, const float* s, int hd, int half_style) {
    const int h = hd / 2;
    if (half_style) {
        for (int i = 0; i < h; ++i) {
            const float a = v[i], b = v[i + h];
            v[i] = a * c[i] - b * s[i];
            v[i + h] = b * c[i] + a * s[i];
        }
    } else {
        for (int i = 0; i < h; ++i) {
            const float a = v[2 * i], b = v[2 * i + 1];
            v[2 * i] = a * c[i] - b * s[i];
            v[2 * i + 1] = b * c[i] + a * s[i];
        }
    }
}

vgxf_state* vgxf_state_new(const vgxf_model* m) {
    vgxf_state* s = (vgxf_state*)calloc(1, sizeof(vgxf_state));
    if (!s) return NULL;
    const size_t kvd = (size_t)m->kv_heads * m->head_dim;
    const size_t big = (size_t)(m->hidden > 3 * m->dim ? m->hidden : 3 * m->dim);
    s->kc = (float*)calloc((size_t)m->layers * m->seq * kvd, sizeof(float));
    s->vc = (float*)calloc((size_t)m->layers * m->seq * kvd, sizeof(float));
    s->cst = (float*)calloc((size_t)m->layers * 2 * m->dim, sizeof(float));
    s->x = (float*)calloc((size_t)m->dim, sizeof(float));
    s->xn = (float*)calloc((size_t)m->dim, sizeof(float));
    s->qkv = (float*)calloc((size_t)m->dim + 2 * kvd, sizeof(float));
    s->att = (float*)calloc((size_t)m->dim, sizeof(float));
    s->g = (float*)calloc(big, sizeof(float));
    s->u = (float*)calloc(big, sizeof(float));
    s->bcx = (float*)calloc((size_t)3 * m->dim, sizeof(float));
    s->t = (float*)calloc(big, sizeof(float));
    s->sc = (float*)calloc((size_t)m->heads * m->seq, sizeof(float));
    if (!s->kc || !s->vc || !s->cst || !s->x || !s->xn || !s->qkv || !s->att || !s->g || !s->u || !s->bcx ||
        !s->t || !s->sc) {
        vgxf_state_free(s);
        return NULL;
    }
    return s;
}

void vgxf_state_free(vgxf_state* s) {
    if (!s) return;
    free(s->kc); free(s->vc); free(s->cst); free(s->x); free(s->xn); free(s->qkv); free(s->att);
    free(s->g); free(s->u); free(s->bcx); free(s->t); free(s->sc);
    free(s);
}

/* One position of the float forward; logits (vocab floats) may be NULL. */
int vgxf_step(const vgxf_model* m, vgxf_state* s, int token, int pos, float* logits) {
    if (!m || !s || token < 0 || token >= m->vocab || pos < 0 || pos >= m->seq) return 1;
    const int D = m->dim, H = m->hidden, hd = m->head_dim, nh = m->heads, nkv = m->kv_heads;
    const int kvd = nkv * hd, half = hd / 2;
    if (pos == 0) memset(s->cst, 0, sizeof(float) * (size_t)m->layers * 2 * D);
    for (int i = 0; i < D; ++i) s->x[i] = (float)m->emb[(size_t)token * D + i] * m->es[token];
    for (int l = 0; l < m->layers; ++l) {
        rms(s->x, m->rms_att + (size_t)l * D, D, m->eps, s->xn);
        if (m->is_conv[l]) {
            /* LFM2 ShortConv: B, C, x = in_proj(xn); Bx; causal depthwise conv
             * over the last three Bx (tap 0 on pos-2); C * conv; out_proj */
            matvec(m->conv_in[l], s->xn, 3 * D, D, s->bcx);
            float* st = s->cst + (size_t)l * 2 * D;
            const float* w = m->conv_w[l];
            for (int i = 0; i < D; ++i) {
                const float bx = s->bcx[i] * s->bcx[2 * D + i];
                const float cv = w[3 * i] * st[i] + w[3 * i + 1] * st[D + i] + w[3 * i + 2] * bx;
                st[i] = st[D + i];
                st[D + i] = bx;
                s->t[i] = s->bcx[D + i] * cv;
            }
            matvec(m->conv_out[l], s->t, D, D, s->att);
        } else {
            matvec(m->qkv[l], s->xn, D + 2 * kvd, D, s->qkv);
            float* q = s->qkv;
            float* k = s->qkv + D;
            const float* v = s->qkv + D + kvd;
            const float* rc = m->rcos + (size_t)pos * half;
            const float* rsn = m->rsin + (size_t)pos * half;
            for (int h = 0; h < nh; ++h) {
                if (m->qk_norm) rms(q + h * hd, m->qn + (size_t)l * hd, hd, 1e-6f, q + h * hd);
                rope(q + h * hd, rc, rsn, hd, m->rope_half);
            }
            for (int h = 0; h < nkv; ++h) {
                if (m->qk_norm) rms(k + h * hd, m->kn + (size_t)l * hd, hd, 1e-6f, k + h * hd);
                rope(k + h * hd, rc, rsn, hd, m->rope_half);
            }
            float* kc = s->kc + (size_t)l * m->seq * kvd;
            float* vc = s->vc + (size_t)l * m->seq * kvd;
            memcpy(kc + (size_t)pos * kvd, k, sizeof(float) * kvd);
            memcpy(vc + (size_t)pos * kvd, v, sizeof(float) * kvd);
            const int rep = nh / nkv;
            const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
            for (int h = 0; h < nh; ++h) {
                const int g = h / rep;
                float* sc = s->sc + (size_t)h * m->seq;
                float mx = -1e30f;
                for (int t = 0; t <= pos; ++t) {
                    sc[t] = dot(q + h * hd, kc + (size_t)t * kvd + g * hd, hd) * scale;
                    mx = sc[t] > mx ? sc[t] : mx;
                }
                float sum = 0.0f;
                for (int t = 0; t <= pos; ++t) {
                    sc[t] = expf(sc[t] - mx);
                    sum += sc[t];
                }
                float* o = s->att + h * hd;
                for (int i = 0; i < hd; ++i) o[i] = 0.0f;
                for (int t = 0; t <= pos; ++t) {
                    const float p = sc[t] / sum;
                    const float* vv = vc + (size_t)t * kvd + g * hd;
                    for (int i = 0; i < hd; ++i) o[i] += p * vv[i];
                }
            }
            memcpy(s->t, s->att, sizeof(float) * D);
            matvec(m->wo[l], s->t, D, D, s->att);
        }
        for (int i = 0; i < D; ++i) s->x[i] += s->att[i];
        rms(s->x, m->rms_ffn + (size_t)l * D, D, m->eps, s->xn);
        matvec(m->w1[l], s->xn, H, D, s->g);
        matvec(m->w3[l], s->xn, H, D, s->u);
        for (int i = 0; i < H; ++i) s->t[i] = s->g[i] / (1.0f + expf(-s->g[i])) * s->u[i];
        matvec(m->w2[l], s->t, D, H, s->att);
        for (int i = 0; i < D; ++i) s->x[i] += s->att[i];
    }
    if (logits) {
        rms(s->x, m->rms_final, D, m->eps, s->xn);
        matvec(m->head, s->xn, m->vocab, D, logits);
    }
    return 0;
}

int vgxf_threads(void) { return omp_get_max_threads(); }
void vgxf_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}
