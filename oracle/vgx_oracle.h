/*
 * vgx_oracle.h -- CPU restatement of the reference's quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libvgx, the engine, the
 * Python package) links, loads or calls this library.  Only tests/, the
 * smoke check in __graft_entry__.py and bench.py's cpu_baseline leg use it,
 * and only as the checker or as the timed CPU baseline.
 *
 * Every function names the reference file:line it restates.  Floating point
 * follows the reference's fp32 operation order with no contraction (the
 * library is built with -ffp-contract=off); transcendental functions are
 * evaluated as (float)f((double)x), which is the definition the HIP kernels
 * implement too.  Sums of integer-grid products are exact (int64) -- the
 * reference accumulates the same integers in fp32, which is exact while every
 * partial sum stays below 2^24 and otherwise differs by fp32 rounding; the
 * *_ref32 variants restate that fp32 order literally so tests can bound the
 * difference.
 */
#ifndef VGX_ORACLE_H
#define VGX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- activation grid (engine/src/common.h:188-195, engine/src/xformat.cpp) */
enum { VGXO_I16_1 = 0, VGXO_I16_2 = 1, VGXO_I8_4 = 2, VGXO_I24_1 = 3, VGXO_F32 = 4, VGXO_BF16 = 5 };
int16_t vgxo_quantize_act(float x);
int vgxo_x_texels(int count, int fmt);
void vgxo_x_pack(const float* v, int count, int fmt, uint8_t* out);
int16_t vgxo_q16_store(float v);
int16_t vgxo_q16_round(float q);
void vgxo_quantize_act_n(const float* v, long n, int16_t* out);

/* ---- packers (engine/tools/mmcf_hf.py) ------------------------------------ */
void vgxo_qmat(const float* w, long n, int16_t* q, double* s);
void vgxo_q8mat(const float* w, long n, int8_t* q, double* s);
void vgxo_q8_from_i16(const float* w, long n, int8_t* q, double* s);
void vgxo_q8_per_row(const float* w, int rows, int cols, int8_t* q, float* unit, float* plane);
int vgxo_q4mat(const float* w, int rows, int cols, uint8_t* packed, int16_t* s16, int16_t* m16,
               double* ps);
int vgxo_t3mat(const float* w, int rows, int cols, uint8_t* packed, float* unit, float* plane);
void vgxo_t3_codes(const uint8_t* packed, int rows, int cols, uint8_t* codes);
long vgxo_t3_bytes(int rows, int cols);

/* ---- unpack / dequantise (engine/src/model.cpp, engine/src/gpu_upload.cpp) */
void vgxo_row_scales(int rows, float scale, const float* plane, float* wsr);
void vgxo_dequant_q8(const uint8_t* body, int prebiased, int rows, int cols, const float* wsr,
                     float* out);
void vgxo_dequant_q4(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                     int rows, int cols, float* out);
void vgxo_dequant_t3(const uint8_t* body, int rows, int cols, const float* wsr, float* out);

/* ---- dequant-GEMV row values (engine/src/shaders.cpp matvec_* builders) ---- */
void vgxo_rowval_q8(const uint8_t* body, int prebiased, int rows, int cols, const float* wsr,
                    const int16_t* x, float* v);
void vgxo_rowval_q8_ref32(const uint8_t* body, int prebiased, int rows, int cols,
                          const float* wsr, const int16_t* x, float* v);
void vgxo_rowsum_q8(const uint8_t* body, int prebiased, int rows, int cols, const int16_t* x,
                    int64_t* s);
void vgxo_rowval_q4(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                    int rows, int cols, const int16_t* x, float* v);
void vgxo_rowval_q4_ref32(const uint8_t* nib, const int16_t* s16, const int16_t* m16, float ps,
                          int rows, int cols, const int16_t* x, float* v);
void vgxo_rowval_t3(const uint8_t* body, int rows, int cols, const float* wsr, const int16_t* x,
                    float* v);
void vgxo_rowval_t3_ref32(const uint8_t* body, int rows, int cols, const float* wsr,
                          const int16_t* x, float* v);
void vgxo_store(const float* v, const int16_t* res, int n, int16_t* y);
void vgxo_store_f32(const float* v, int n, float* y);
void vgxo_gate(const float* v1, const float* v3, int n, int hs, int16_t* h);
void vgxo_probe_q8(const int8_t* w, int rows, int cols, const float* srow, float unit,
                   const int16_t* xq, const int16_t* res, int32_t* want);

/* ---- RMSNorm (engine/src/shaders.cpp:1965-2124) --------------------------- */
void vgxo_rmsnorm(const int16_t* x, const int16_t* w, int dim, float eps, int16_t* y);
void vgxo_rmsnorm_stats(const int16_t* x, int dim, int64_t* partials32, int64_t* total);

/* ---- attention and KV pack/unpack (engine/src/shaders_attn.cpp) ----------- */
/* positions per chunk of the attention sums' summation order */
#define VGXO_ATTN_CHUNK 32
typedef struct {
    int dim, heads, kv_heads, head_dim, seq;
    int kv_bits;   /* 16 or 8 */
    int rope_half; /* 1 rotate-half, 0 interleaved pairs */
    int qk_norm;
} vgxo_attn_cfg;
void vgxo_rope_table(const float* rcos, const float* rsin, int seq, int half, int32_t* tab);
void vgxo_rope_cos_sin(float theta, int head_dim, int seq, float* rcos, float* rsin);
int vgxo_kv_row_bytes(const vgxo_attn_cfg* c);
void vgxo_kv_write(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* kn, const int32_t* rtab,
                   int pos, uint8_t* row);
void vgxo_q_rot(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* qn, const int32_t* rtab,
                int pos, int16_t* qrot);
void vgxo_attn_scores(const vgxo_attn_cfg* c, const int16_t* qrot, const uint8_t* kv, int pos,
                      int16_t* scores);
void vgxo_attn_stats(const vgxo_attn_cfg* c, const int16_t* scores, int pos, int16_t* st);
void vgxo_attn_v(const vgxo_attn_cfg* c, const int16_t* scores, const int16_t* st, const uint8_t* kv,
                 int pos, int16_t* out);
void vgxo_attn_block(const vgxo_attn_cfg* c, const int16_t* qkv, const int16_t* qn, const int16_t* kn,
                     const int32_t* rtab, int pos, uint8_t* kv, int16_t* out);
float vgxo_kv_decode(const vgxo_attn_cfg* c, const uint8_t* row, int idx);

/* ---- LFM2 conv block (engine/src/gpu_conv.cpp:165-225) -------------------- */
void vgxo_conv_taps(const float* w, int dim, int k, int16_t* taps);
void vgxo_conv_step(int dim, const int16_t* bcx, const int16_t* taps, int16_t* s2, int16_t* s1, int16_t* y);

/* ---- embedding and argmax (engine/src/session.cpp:342-371, sampling.cpp) -- */
void vgxo_embed_q8(const int8_t* emb, const float* emb_scale, int dim, int token, int16_t* x);
int vgxo_argmax_i16(const int16_t* v, int n);

/* ---- float path (engine/tools/ref_forward.py:35-115) --------------------- */
void vgxo_matvec_f32(const float* w, int rows, int cols, const float* x, float* y);
void vgxo_rms_f32(const float* x, const float* w, int n, float eps, float* y);

/* ---- CPU baseline helpers -------------------------------------------------- */
int vgxo_threads(void);
void vgxo_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
