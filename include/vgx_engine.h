/*
 * vgx_engine.h -- the decode engine above libvgx: MMCF loader, layer loop
 * and greedy generation, as one C-ABI object.
 *
 * It re-provides the reference's Session (engine/src/session.h:41-93) over
 * libvgx: vgx_engine_step is Session::step (forward_gpu_hidden + the logits
 * readback, engine/src/session.cpp:1797-1821); vgx_engine_generate is the
 * chat decode loop with greedy selection (engine/src/chat.cpp:313-352,
 * argmax_token's first-maximum rule) with the token chained on the device,
 * as Session::step_greedy does with GPU_ARGMAX (engine/src/session.cpp:1827-1842).
 * Status codes are libvgx's (vgx.h).
 */
#ifndef VGX_ENGINE_H
#define VGX_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct vgx_engine vgx_engine;

/* Open an MMCF container (a path, or bytes the caller keeps alive until
 * close) on `device`.  seq: KV length, 0 = the container's; kv_bits: 16 or 8
 * (the reference's KV=q16 / KV=q8). */
int vgx_engine_open(const char* path, int device, int seq, int kv_bits, vgx_engine** out);
int vgx_engine_open_bytes(const void* data, size_t size, int device, int seq, int kv_bits,
                          vgx_engine** out);
int vgx_engine_close(vgx_engine* e);
int vgx_engine_info(const vgx_engine* e, int* dim, int* layers, int* vocab, int* seq);
/* The number of LFM2 conv layers (key 14 of the container); 0 for a model of
 * attention layers only, < 0 for a NULL engine. */
int vgx_engine_conv_layers(const vgx_engine* e);
/* One position: logits_host (vocab int16, q16 grid) and next (argmax) may be NULL. */
int vgx_engine_step(vgx_engine* e, int token, int pos, int16_t* logits_host, int* next);
/* Greedy generation: n_prompt tokens at positions 0.., then n_gen tokens into
 * out.  prefill_ms covers the prompt (its last step yields out[0]); decode_ms
 * the n_gen-1 steps after it.  Either timing pointer may be NULL. */
int vgx_engine_generate(vgx_engine* e, const int* prompt, int n_prompt, int n_gen, int* out,
                        double* prefill_ms, double* decode_ms);
/* The same with positions 0..n_cached-1 of the prompt already in the KV cache
 * (a loaded prefix cache): only positions n_cached.. are prefilled, so
 * 0 <= n_cached < n_prompt (the reference re-runs at least the last prompt
 * token for its logits, engine/src/worker.cpp:277-279). */
int vgx_engine_generate_from(vgx_engine* e, const int* prompt, int n_prompt, int n_cached, int n_gen, int* out,
                             double* prefill_ms, double* decode_ms);
/* Prompt positions pos0 .. pos0+n-1 in batches: Session::step_group
 * (engine/src/session.cpp:1741-1795) on the int8 matrix cores.  Every
 * position's result equals vgx_engine_step's, so logits_host (vocab int16 of
 * the last position, may be NULL) and next are what n serial steps give. */
int vgx_engine_prefill(vgx_engine* e, const int* tokens, int n, int pos0, int16_t* logits_host, int* next);
/* Largest batch a prompt is prefilled in (the reference's PREFILL_BATCH,
 * docs/prefill-batching.md): 0 or 1 = one position at a time; at most
 * min(seq, 512), which is also the default.  Applies to vgx_engine_prefill
 * and to vgx_engine_generate's prompt. */
int vgx_engine_set_prefill_batch(vgx_engine* e, int n);
/* Decode steps of vgx_engine_generate[_from] as one HIP graph replayed per
 * token (on: the default) or as individual launches (off); the tokens are
 * the same either way. */
int vgx_engine_set_graphs(vgx_engine* e, int on);
/* Greedy generation for nseq sequences in lockstep (no counterpart in the
 * reference, which decodes one sequence): prompts is nseq x n_prompt, out
 * nseq x n_gen, each row exactly what vgx_engine_generate gives for that
 * prompt.  Each prompt is prefilled on its own KV cache, then every step runs
 * all sequences at once (GEMMs on the int8 matrix cores over nseq rows, one
 * attention launch).  nseq at most min(seq, 512); not for conv (hybrid)
 * models. */
int vgx_engine_generate_batch(vgx_engine* e, int nseq, const int* prompts, int n_prompt, int n_gen, int* out,
                              double* prefill_ms, double* decode_ms);
/* The MMKV1 prefix cache (engine/src/prefix_cache.cpp:25-207).  save: the
 * KV rows of positions 0..n-1 (the caller has run toks[0..n) through the
 * engine) and, for a hybrid model, the conv history, under a header naming
 * the container (file size and mtime), the shape and the KV packing; plus the
 * JSON sidecar path + ".json" with system_fnv / tools_fnv as the reference
 * records them.  load: refuses a cache written for another container, shape
 * or packing (VGX_EINVAL) before touching the device state; on success the
 * KV rows, the conv history and the token history are in place, *n is the
 * cached token count and toks (cap entries, may be NULL) holds the ids. */
int vgx_engine_save_prefix(vgx_engine* e, const char* path, const int* toks, int n, uint64_t system_fnv,
                           uint64_t tools_fnv);
int vgx_engine_load_prefix(vgx_engine* e, const char* path, int* toks, int cap, int* n);
/* The message of the last failed engine call on this thread. */
const char* vgx_engine_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
