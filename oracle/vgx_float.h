/* The reference's float CPU path (engine/tools/ref_forward.py semantics) in C.
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg and tests/. */
#ifndef VGX_FLOAT_H
#define VGX_FLOAT_H

#include <stdint.h>

typedef struct {
    int dim, hidden, layers, heads, kv_heads, head_dim, vocab, seq;
    int rope_half, qk_norm;
    float eps;
    const int* is_conv;                    /* layers */
    const float* const* qkv;               /* per layer (dim + 2 kv_dim) x dim; NULL on conv layers */
    const float* const* wo;                /* dim x dim */
    const float* const* conv_in;           /* 3 dim x dim (conv layers) */
    const float* const* conv_out;          /* dim x dim */
    const float* const* conv_w;            /* dim x 3 */
    const float* const* w1;                /* hidden x dim */
    const float* const* w3;                /* hidden x dim */
    const float* const* w2;                /* dim x hidden */
    const float* rms_att;                  /* layers x dim */
    const float* rms_ffn;                  /* layers x dim */
    const float* rms_final;                /* dim */
    const float* qn;                       /* layers x head_dim, or NULL */
    const float* kn;
    const float* rcos;                     /* seq x head_dim/2 */
    const float* rsin;
    const int8_t* emb;                     /* vocab x dim */
    const float* es;                       /* vocab */
    const float* head;                     /* vocab x dim */
} vgxf_model;

typedef struct vgxf_state vgxf_state;

vgxf_state* vgxf_state_new(const vgxf_model* m);
void vgxf_state_free(vgxf_state* s);
int vgxf_step(const vgxf_model* m, vgxf_state* s, int token, int pos, float* logits);
int vgxf_threads(void);
void vgxf_set_threads(int n);

#endif
