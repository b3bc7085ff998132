/*
 * vgx.h -- C-ABI of libvgx, the MI355X (gfx950) quantized decode path.
 *
 * This is the boundary that replaces the reference engine's `class GPU`
 * (engine/src/gpu.h:41-633): every GLES2 draw + readback the reference's
 * Session issues for the decode hot path has one entry point here.  Plain
 * pointers and sizes only.  Activation, residual, KV and logits buffers are
 * device pointers (hipMalloc'd or torch tensors); weight bytes are passed
 * exactly as they lie in an MMCF container (host pointers) and are copied to
 * HBM at upload.
 *
 * Numbers: activations travel as the reference's q16 grid -- int16 holding
 * round(value*256) (engine/src/common.h:188-195) -- in native little-endian
 * order; the texel byte order (big-endian pairs) exists only in
 * vgx_x_pack_i16_2 and in the KV row export, where it is a persisted format.
 *
 * Errors: every call returns VGX_OK (0) or a negative status; the message of
 * the last failure on the calling thread is vgx_last_error().  No call throws
 * or aborts.  Shapes are validated at upload and at each launch.
 *
 * Streams: all device work of a context is issued on its stream in call
 * order (vgx_ctx_set_stream); only vgx_ctx_sync, vgx_kv_read_rows and
 * vgx_kv_write_rows block the host.  One context per host thread, as the
 * reference keeps one GL context per process (engine/src/gpu_internal.h:4-9).
 */
#ifndef VGX_H
#define VGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VGX_ABI_VERSION 1

enum vgx_status {
    VGX_OK = 0,
    VGX_EINVAL = -1, /* bad argument or shape */
    VGX_EHIP = -2,   /* HIP runtime error (message in vgx_last_error) */
    VGX_ENOMEM = -3, /* device allocation failed */
    VGX_ESTATE = -4, /* call out of order (e.g. attention before create) */
    VGX_ERANGE = -5  /* position / row / size outside what was created */
};

typedef struct vgx_ctx vgx_ctx;
typedef struct vgx_mat vgx_mat;
typedef struct vgx_group vgx_group;
typedef struct vgx_attn vgx_attn;
typedef struct vgx_conv vgx_conv;

int vgx_abi_version(void);
const char* vgx_strerror(int status);
const char* vgx_last_error(void);

/* ---- context: replaces GPU::GPU / init_egl (engine/src/gpu.cpp) and
 *      GPU::sync (engine/src/gpu.h:60); release_scene is vgx_ctx_destroy. */
int vgx_ctx_create(int device, vgx_ctx** out);
int vgx_ctx_destroy(vgx_ctx* ctx);
/* hipStream_t; NULL is HIP's default (null) stream.  A new context issues on
 * a stream of its own that is ordered with the null stream. */
int vgx_ctx_set_stream(vgx_ctx* ctx, void* stream);
void* vgx_ctx_stream(vgx_ctx* ctx);
int vgx_ctx_sync(vgx_ctx* ctx);

/* ---- weights: replaces GPU::upload(Mat&) (engine/src/gpu_upload.cpp:20-192).
 * The body and planes are the MMCF tensor bytes unchanged
 * (docs/checkpoint-container.md, "Tensor record"):
 *   Q8: rows x cols bytes, q8u8 (dtype 2, prebiased=1) or q8i8 (dtype 3);
 *       `scale` = record scale; `row_plane` = part 3 (rows f32) or NULL.
 *   Q4: rows x cols/2 nibble bytes (low nibble = even column); `scale` = the
 *       record's ps; `q4_scale` / `q4_min` = parts 1 and 2 (rows x cols/32 int16).
 *   T3: ceil(rows/2) x cols/8 x 4 bytes (dtype 7; cols a multiple of 8, as
 *       the packer pads them, engine/tools/mmcf_hf.py:151-156); `scale` =
 *       record scale (the kernels use scale*127, engine/src/model.cpp:927);
 *       `row_plane` = part 3.
 * Column counts: q8 a multiple of 16, q4 of 32, t3 of 8.
 * `scale_mul` is Model::apply_hidden_scale's 2^k for a w2 matrix
 * (engine/src/model.cpp:407-429), 0 or 1 for every other matrix.  */
enum vgx_kind { VGX_Q8 = 1, VGX_Q4 = 2, VGX_T3 = 3 };
typedef struct vgx_weight_desc {
    int kind;
    int rows, cols;
    const void* body;
    size_t body_bytes;
    int prebiased;
    float scale;
    const float* row_plane;
    const int16_t* q4_scale;
    const int16_t* q4_min;
    float scale_mul;
} vgx_weight_desc;

int vgx_mat_upload(vgx_ctx* ctx, const vgx_weight_desc* desc, vgx_mat** out);
/* A second device copy of an uploaded matrix (device-to-device). */
int vgx_mat_clone(vgx_ctx* ctx, const vgx_mat* src, vgx_mat** out);
int vgx_mat_free(vgx_mat* m);
int vgx_mat_shape(const vgx_mat* m, int* kind, int* rows, int* cols);
/* Bytes one GEMV over this matrix must read from HBM for the weights: body
 * plus the per-row / per-group scale planes as held on the device. */
size_t vgx_mat_weight_bytes(const vgx_mat* m);
/* The dequantised matrix, fp32 rows x cols into device memory: the value each
 * kernel multiplies by (q8/t3: level * row scale; q4: n*(s16*ps) + m16*ps). */
int vgx_dequant(vgx_ctx* ctx, const vgx_mat* m, float* out);

/* ---- dequant-GEMV family.
 * vgx_gemv: y = q16(W.x) -- matvec_q8_pair_logits / matvec_t3_pair /
 *   matvec_i4 (engine/src/shaders.cpp:704-747, 554-573, 1249-1274); with
 *   `res` (may be NULL) y = q16(W.x + res), one rounding, as
 *   matvec_q8_add_pair / matvec_i4_add_pair / matvec_t3_add_pair
 *   (:1161-1214, :1322-1354, :575-600) dispatched by GPU::matvec_add
 *   (engine/src/gpu_matvec.cpp:225-291).  x: cols int16, y/res: rows int16.  */
int vgx_gemv(vgx_ctx* ctx, const vgx_mat* W, const int16_t* x, const int16_t* res, int16_t* y);
/* fp32 activations: x is quantised to the q16 grid exactly as the host does
 * before every upload (x_pack, engine/src/xformat.cpp:87-93) and y is the row
 * value in activation units before the q16 store (the store grid / 256). */
int vgx_gemv_f32(vgx_ctx* ctx, const vgx_mat* W, const float* x, float* y);
/* Two residual adds through the column halves of one matrix:
 *   y = q16( W[:, split:].x[split:] + q16( W[:, :split].x[:split] + res ) )
 * which is GPU::matvec_add(w2a) then matvec_add(w2b) over Model::split_ffn's
 * column chunks (engine/src/session.cpp:1557-1562, model.cpp:255-265).  */
int vgx_gemv_add_split(vgx_ctx* ctx, const vgx_mat* W, int split, const int16_t* x,
                       const int16_t* res, int16_t* y);

/* A fixed list of matrices sharing one input (same kind, same cols), launched
 * as one kernel; outputs are concatenated in list order.  Replaces
 * GPU::logits_pass (one draw per <=1536-row tile, engine/src/gpu_matvec.cpp:56-82). */
int vgx_group_create(vgx_ctx* ctx, int n, const vgx_mat* const* mats, vgx_group** out);
int vgx_group_free(vgx_group* g);
int vgx_group_rows(const vgx_group* g);
int vgx_gemv_group(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, int16_t* y);
int vgx_gemv_group_f32(vgx_ctx* ctx, const vgx_group* g, const float* x, float* y);
/* The launch plan a GEMV over W (or over the group g, which is one launch)
 * takes: lanes of a wave that share a row, and rows each lane owns.  No
 * counterpart in the reference, whose draw geometry is fixed by the shader;
 * it lets a caller check which kernel variant a shape runs on. */
int vgx_gemv_plan_info(vgx_ctx* ctx, const vgx_mat* W, int* lanes_per_row, int* rows_per_lane);
int vgx_group_plan_info(const vgx_group* g, int* lanes_per_row, int* rows_per_lane);
/* The logits pass followed by argmax_token's first-maximum rule
 * (engine/src/sampling.cpp:160-162): `token` (device int) receives the
 * index into the concatenated rows; `logits` (device, may be NULL) the q16 rows. */
int vgx_logits_argmax(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, int16_t* logits,
                      int* token);

/* The candidate pass of GPU::logits_candidates_from (engine/src/gpu_matvec.cpp:
 * 152-230; kernels top2 / top2_packed, engine/src/shaders_attn.cpp:477-494, 574-594)
 * over a q16 logits row of n values (device).  For chunk c = logits
 * [16c, min(16c + 16, n)) out (device, 6 * ceil(n / 16) ints) receives
 *   v1, i1   the first maximum (q16 value, index into the row)
 *   v2, i2   the first maximum of the rest (i2 = -1: a one-logit chunk)
 *   lm       the chunk maximum (q16)
 *   sum      floor(2048 * S + 1/2), S the kernel's running sum of
 *            exp((v - max) / T) over the chunk, rescaled as the max grows,
 *            with T = max(0.0001, temp).
 * The reference's chunks are per 1536-row logits tile; with every tile but
 * the last a multiple of 16 rows they are these chunks of the whole row. */
int vgx_logits_chunks(vgx_ctx* ctx, const int16_t* logits, int n, float temp, int* out);

/* Fused FFN gate: h = q16( SiLU(qz(W1.x)) * qz(W3.x) * 2^-hs ) over all rows
 * -- matvec_q8_pair_swiglu / i4_gate_flat8b (engine/src/shaders.cpp:756-815,
 * 1539-1590) as dispatched by GPU::ffn_split_chunked (engine/src/gpu_ffn.cpp:67-132);
 * the row chunks of split_ffn are rows of the same kernel here.  */
int vgx_ffn_gate(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, const int16_t* x, int hs,
                 int16_t* h);

/* GPU::rmsnorm (engine/src/gpu_upload.cpp:280-365, shaders rms_stats_split /
 * rms_norm): w is the norm weight on the q16 grid (x_pack of the f32 vector). */
int vgx_rmsnorm(vgx_ctx* ctx, int dim, const int16_t* x, const int16_t* w, float eps, int16_t* y);

/* ---- RMSNorm fused into the GEMV that consumes it.  Each is GPU::rmsnorm
 * (engine/src/gpu_upload.cpp:280-365) over x (cols values) with weight rms_w
 * (q16, device, 16-byte aligned) and eps > 0, followed by the named GEMV on
 * its q16 output, in one launch and with identical results; the normalised
 * vector is not written out.  The pairs they replace:
 *   vgx_gemv_rms          rmsnorm + vgx_gemv (the attention norm and the qkv
 *                         draw, engine/src/session.cpp:1483 then 1502)
 *   vgx_ffn_gate_rms      rmsnorm + vgx_ffn_gate (session.cpp:1516, 1538-1569)
 *   vgx_gemv_group_rms    rmsnorm + vgx_gemv_group
 *   vgx_logits_argmax_rms the final norm + vgx_logits_argmax
 *                         (session.cpp:1580, sampling.cpp:160-162); each
 *                         workgroup leaves its best key in the group's key
 *                         slots and a one-workgroup launch on the same stream
 *                         reduces them, so launches over one group must not
 *                         overlap. */
int vgx_gemv_rms(vgx_ctx* ctx, const vgx_mat* W, const int16_t* x, const int16_t* rms_w, float eps,
                 const int16_t* res, int16_t* y);
int vgx_ffn_gate_rms(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, const int16_t* x,
                     const int16_t* rms_w, float eps, int hs, int16_t* h);
int vgx_gemv_group_rms(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                       int16_t* y);
int vgx_logits_argmax_rms(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                          int16_t* logits, int* token);
/* vgx_logits_argmax_rms with the workgroups' key slots in a static device
 * array of 4096 slots (32 KiB per device, resolved at vgx_ctx_create) instead
 * of the group's own: no counterpart in the reference; for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops).  The call allocates nothing.  A launch needing more workgroups than
 * there are slots is refused (VGX_ERANGE; the LM-head launch takes at most 5
 * per CU).  Every call on one device shares the array: calls that overlap on
 * one GPU (other streams, other threads) race; every slot a call reads is
 * written by that call first. */
int vgx_logits_argmax_rms_noalloc(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w,
                                  float eps, int16_t* logits, int* token);

/* ---- batched prefill: ntok consecutive positions per launch, every row the
 * exact result of the batch-1 entry point on that token.  Replaces
 * Session::step_group's per-position draws (engine/src/session.cpp:1741-1795)
 * and the two-position P2 kernels (matvec_q8_p2 and the pair gate,
 * engine/src/shaders.cpp:825-1072): the reference's rule for a batched path
 * is byte-identical logits to the serial one (docs/prefill-batching.md:98-113).
 * Activations are row-major, ntok rows of cols (x) or rows (y, res, h) q16
 * values; the GEMMs run on the int8 matrix cores.
 *   vgx_gemm            per token: vgx_gemv (y = q16(W.x [+ res]))
 *   vgx_gemm_add_split  per token: vgx_gemv_add_split
 *   vgx_ffn_gate_batch  per token: vgx_ffn_gate
 *   vgx_rmsnorm_batch   per token: vgx_rmsnorm (upload_hidden_grp + rmsnorm,
 *                       engine/src/gpu_upload.cpp:250)
 *   vgx_embed_q8_batch  per token: vgx_embed_q8; tokens is a device int array
 *   vgx_kv_append_batch / vgx_attn_decode_batch: positions pos0 .. pos0+ntok-1,
 *     qkv and out rows consecutive; the KV rows are written first, then every
 *     position attends to its prefix (att_stage, att_scores_batch,
 *     att_stats_row, att_v_row: engine/src/gpu_attn.cpp:433-532).
 * A vgx_gemm, vgx_gemm_add_split or vgx_ffn_gate_batch launch of at most 32
 * tokens whose row tiles leave most CUs idle and whose rows are longer than
 * 32 k-steps (of 32 columns) splits K over up to 8 workgroups
 * and adds their exact integer sums in a second launch; the sums live in a
 * workspace of the context, sized for every such launch (8 splits x 2 sets x
 * 32 tokens x num_cu/2 tiles of 32 rows, int64: 16 MiB at 256 CUs), allocated
 * at the first such call and never regrown, freed by vgx_ctx_destroy.  No
 * allocation happens under stream capture.  Results are identical either way;
 * a launch without a workspace (capture before the first, or an allocation
 * failure) runs whole. */
int vgx_gemm(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* res, int16_t* y);
int vgx_gemm_add_split(vgx_ctx* ctx, const vgx_mat* W, int split, int ntok, const int16_t* x, const int16_t* res,
                       int16_t* y);
int vgx_ffn_gate_batch(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, int ntok, const int16_t* x, int hs,
                       int16_t* h);
int vgx_rmsnorm_batch(vgx_ctx* ctx, int ntok, int dim, const int16_t* x, const int16_t* w, float eps, int16_t* y);
/* RMSNorm fused into the GEMM that consumes it: per token,
 *   vgx_gemm_rms            vgx_rmsnorm (rms_w, eps) then vgx_gemm
 *   vgx_ffn_gate_batch_rms  vgx_rmsnorm (rms_w, eps) then vgx_ffn_gate_batch
 * in one launch with identical results; the normalised rows are not written
 * out.  The pairs they replace in Session::step_group
 * (engine/src/session.cpp:1741-1795): the attention norm and the qkv draw,
 * the FFN norm and the gate.  rms_w: cols q16 values, 16-byte aligned. */
int vgx_gemm_rms(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* rms_w, float eps,
                 const int16_t* res, int16_t* y);
int vgx_ffn_gate_batch_rms(vgx_ctx* ctx, const vgx_mat* W1, const vgx_mat* W3, int ntok, const int16_t* x,
                           const int16_t* rms_w, float eps, int hs, int16_t* h);
int vgx_embed_q8_batch(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim, int ntok,
                       const int* tokens, int16_t* x);
/* The embedding rows of a batch and their RMSNorm: per token vgx_embed_q8
 * into x (the residual stream), then vgx_rmsnorm(x, rms_w, eps) into y, in
 * one launch with identical bytes -- Session::embedding
 * (engine/src/session.cpp:362-365) and the first layer's attention norm
 * (:1483).  rms_w: dim q16 values. */
int vgx_embed_q8_rms_batch(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim, int ntok,
                           const int* tokens, int16_t* x, const int16_t* rms_w, float eps, int16_t* y);
/* The other side of the same fusion: a GEMM that writes the residual stream
 * also normalises the rows it wrote, per token,
 *   vgx_gemm_norm            vgx_gemm, then vgx_rmsnorm_batch(y, rms_w, eps) -> yn
 *   vgx_gemm_add_split_norm  vgx_gemm_add_split, then the same
 * with identical bytes in y and yn.  For the decode of a batch of sequences:
 * in Session::forward_gpu_hidden, the wo residual and the FFN norm
 * (engine/src/session.cpp:1508-1516), the w2 residual (:1572) and the next
 * layer's attention norm (:1483) or the final norm (:1580), so the GEMM that
 * reads yn needs no norm of its own.  A launch whose K is split adds the RMSNorm to its
 * epilogue launch (one workgroup per token row); otherwise it is a launch of
 * its own.  rms_w: W's rows q16 values; yn: ntok rows of W's rows values. */
int vgx_gemm_norm(vgx_ctx* ctx, const vgx_mat* W, int ntok, const int16_t* x, const int16_t* res, int16_t* y,
                  const int16_t* rms_w, float eps, int16_t* yn);
int vgx_gemm_add_split_norm(vgx_ctx* ctx, const vgx_mat* W, int split, int ntok, const int16_t* x,
                            const int16_t* res, int16_t* y, const int16_t* rms_w, float eps, int16_t* yn);

/* One matrix holding the rows of n q8 or t3 matrices of equal cols, in order
 * (the LM head tiles as a single operand of vgx_gemm, for batched decode);
 * every row keeps its own scale, so its results are unchanged.  A t3 matrix
 * before the last must have an even row count. */
int vgx_mat_concat(vgx_ctx* ctx, int n, vgx_mat* const* mats, vgx_mat** out);
/* argmax_token (engine/src/sampling.cpp:160-162, the first maximum) of each
 * row of a row-major nrows x n q16 array (device); tokens: device int[nrows]. */
int vgx_argmax_rows(vgx_ctx* ctx, int nrows, int n, const int16_t* v, int* tokens);

/* Session::embedding (engine/src/session.cpp:342-371), q8 rows: x = the
 * host-grid q16 of emb[token]*emb_scale[token].  emb: vocab x dim signed
 * bytes (device), emb_scale: vocab f32 (device), token: device int. */
int vgx_embed_q8(vgx_ctx* ctx, const int8_t* emb, const float* emb_scale, int vocab, int dim,
                 const int* token, int16_t* x);

/* ---- attention over the packed KV cache: replaces GPU::init_attention,
 * attention_block, kv_rope_write (engine/src/gpu_attn.cpp:41-241, 400-421). */
typedef struct vgx_attn_desc {
    int dim, heads, kv_heads, head_dim, seq, layers;
    int kv_bits;               /* 16 (grid 1/2048) or 8 (grid 1/16) */
    int rope_half;             /* 1: rotate-half pairs (i, i+hd/2); 0: (2i, 2i+1) */
    int qk_norm;
    const float* rope_cos;     /* host [seq][head_dim/2] (Session's tables) */
    const float* rope_sin;
    const float* q_norm;       /* host [layers][head_dim] f32, NULL without qk_norm */
    const float* k_norm;
    const uint8_t* layer_is_attn; /* host [layers], NULL = every layer */
} vgx_attn_desc;
int vgx_attn_create(vgx_ctx* ctx, const vgx_attn_desc* desc, vgx_attn** out);
int vgx_attn_free(vgx_attn* a);
/* KV write of position `pos`: K qk-normed, rotated, packed; V packed. */
int vgx_kv_append(vgx_attn* a, int layer, int pos, const int16_t* qkv);
/* q prep, scores, stats and the weighted V for position `pos` (rows 0..pos
 * of the layer's KV must be written). qkv: dim + 2*kv_dim int16; out: dim. */
int vgx_attn_decode(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out);
/* vgx_kv_append then vgx_attn_decode in one launch. */
int vgx_attn_block(vgx_attn* a, int layer, int pos, const int16_t* qkv, int16_t* out);
/* Batched forms for positions pos0 .. pos0+ntok-1 (see the batched prefill
 * block above; engine/src/gpu_attn.cpp:433-532): qkv holds ntok consecutive
 * rows of dim + 2*kv_dim, out ntok rows of dim.  Append all rows first. */
int vgx_kv_append_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv);
int vgx_attn_decode_batch(vgx_attn* a, int layer, int pos0, int ntok, const int16_t* qkv, int16_t* out);

/* ---- a decode step captured once and replayed for every token (a HIP
 * graph: its kernel arguments are fixed, so the position lives in device
 * memory).  No counterpart in the reference, whose host loop issues each
 * step (engine/src/session.cpp:1827-1842).
 * vgx_attn_block_at: vgx_attn_block at the position *pos_dev (clamped into
 *   the cache; the host cannot check it).
 * vgx_decode_advance: hist[*pos + 1] = *token (when inside hist_len), then
 *   ++*pos; one thread, so a replayed step leaves the next one's position
 *   and the token history in place.
 * vgx_logits_argmax_step: vgx_logits_argmax_rms, then in the same reduction
 *   launch the step's tail: the advance above with the chosen token, and
 *   that token's q8 embedding row (vgx_embed_q8: emb, emb_scale, vocab, dim)
 *   into x_next, the next step's input (it may be x: the head's launch has
 *   read x before the reduction launch starts).  Two launches
 *   fewer per step than vgx_logits_argmax_rms + vgx_decode_advance +
 *   vgx_embed_q8, with the same results. */
int vgx_attn_block_at(vgx_attn* a, int layer, const int* pos_dev, const int16_t* qkv, int16_t* out);
int vgx_decode_advance(vgx_ctx* ctx, int* pos, const int* token, int* hist, int hist_len);
int vgx_logits_argmax_step(vgx_ctx* ctx, const vgx_group* g, const int16_t* x, const int16_t* rms_w, float eps,
                           int16_t* logits, int* token, int* pos, int* hist, int hist_len, const int8_t* emb,
                           const float* emb_scale, int vocab, int dim, int16_t* x_next);

/* ---- several sequences in lockstep (batched greedy decode).  No counterpart
 * in the reference, which decodes one sequence; each sequence's results are
 * the exact results of the single-sequence entry points on it.
 * vgx_attn_create_seqs: the KV caches of nseq sequences (each seq rows per
 *   layer); vgx_attn_create is nseq = 1.
 * vgx_attn_seq_view: a handle on sequence s's cache that every
 *   single-sequence entry point takes (its prompt's batched prefill, the
 *   MMKV1 row export/import); it shares the parent's buffers, so free it
 *   before the parent.
 * vgx_attn_block_seqs: vgx_attn_block of position pos for sequences
 *   0..nseq-1 in one launch; qkv holds nseq consecutive rows of
 *   dim + 2*kv_dim, out nseq rows of dim. */
int vgx_attn_create_seqs(vgx_ctx* ctx, const vgx_attn_desc* desc, int nseq, vgx_attn** out);
int vgx_attn_seq_view(vgx_attn* a, int s, vgx_attn** out);
int vgx_attn_block_seqs(vgx_attn* a, int layer, int pos, int nseq, const int16_t* qkv, int16_t* out);

/* ---- LFM2 gated short convolution: replaces GPU::init_conv, set_conv_kernel,
 * conv_block's gate/conv3/gate passes and clear_conv_state
 * (engine/src/gpu_conv.cpp:10-225), between the in_proj GEMV (3*dim rows:
 * B, C, x) and the out_proj GEMV.
 * vgx_conv_create: w = host f32 [layers][dim][kernel] (the container's
 *   depthwise kernel records, engine/src/model.cpp:1143-1158), kernel must be
 *   3; layer_is_conv = host [layers] (key 14) or NULL = every layer.
 * vgx_conv_step: positions in order, ntok of them: bcx = ntok rows of 3*dim
 *   q16 (the in_proj output), y = ntok rows of dim q16; the per-layer state
 *   (the last two gated vectors) advances by ntok.
 * vgx_conv_reset: every layer's state to zero (Session::zero_conv_state,
 *   engine/src/session.cpp:320-325).
 * vgx_conv_state_read / write: one layer's state, 2*dim int16 (the gated
 *   vectors of positions pos-2 and pos-1), what the prefix cache persists for
 *   a hybrid model (read_conv_state / write_conv_state, gpu_conv.cpp:24-58). */
int vgx_conv_create(vgx_ctx* ctx, int dim, int layers, int kernel, const float* w, const uint8_t* layer_is_conv,
                    vgx_conv** out);
int vgx_conv_free(vgx_conv* c);
int vgx_conv_reset(vgx_conv* c);
int vgx_conv_step(vgx_conv* c, int layer, int ntok, const int16_t* bcx, int16_t* y);
int vgx_conv_state_read(vgx_conv* c, int layer, int16_t* host);
int vgx_conv_state_write(vgx_conv* c, int layer, const int16_t* host);
/* The packed KV rows in the reference's texel byte layout (K values then V
 * values; q16 big-endian, q8 two's-complement bytes) -- what MMKV1 persists
 * (engine/src/prefix_cache.cpp:59-67).  Host buffers; these block. */
int vgx_kv_row_bytes(const vgx_attn* a);
int vgx_kv_read_rows(vgx_attn* a, int layer, int row0, int nrows, void* host);
int vgx_kv_write_rows(vgx_attn* a, int layer, int row0, int nrows, const void* host);

/* ---- host helpers (no device work) */
/* quantize_act over n values (engine/src/common.h:188-195). */
void vgx_quantize_act(const float* v, int n, int16_t* q);
/* x_pack(I16_2): the texel bytes, 4*ceil(n/2) (engine/src/xformat.cpp:87-93). */
void vgx_x_pack_i16_2(const float* v, int n, uint8_t* out);

#ifdef __cplusplus
}
#endif
#endif
