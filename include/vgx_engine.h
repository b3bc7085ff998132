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
/* Decode steps of vgx_engine_generate[_from] as replayed HIP graphs (on: the
 * default; one step a graph, and four steps a graph for runs of four tokens
 * where a step has at most 100 launches) or as individual launches (off);
 * the tokens are the same either way. */
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
/* One position with the top-k candidates of its logits instead of the logits
 * (Session::step_candidates, engine/src/session.cpp:1844-1859, over
 * GPU::logits_candidates_from, engine/src/gpu_matvec.cpp:97-230): the
 * two largest logits of every 16-logit chunk (vgx_logits_chunks), sorted by
 * value, the first topk kept in value / cand_token (cap >= topk entries, *n
 * kept); stats = {logsumexp of logit / T, the largest logit, the softmax
 * denominator}, T = max(0.0001, temp), from the chunks' (max, sum) pairs.
 * *complete = 1 when the kept candidates hold at least top_p of the
 * probability mass; otherwise full (vocab floats) receives the logits, the
 * reference's fallback to the full read-back. */
int vgx_engine_step_candidates(vgx_engine* e, int token, int pos, int topk, float temp, float top_p, float* value,
                               int* cand_token, int cap, int* n, float* stats, int* complete, float* full);

/* ---- token selection on the host (engine/src/sampling.cpp), for the
 * worker's sampled requests.  Each keeps the reference's float operations and
 * standard-library selection in order, so a seed draws the reference's token
 * from the same logits.  Logits are floats (the q16 value / 256). */
typedef struct vgx_sampler vgx_sampler;
/* A generator: std::mt19937 seeded with `seed` (the request's, engine/src/worker.cpp:337). */
int vgx_sampler_create(uint32_t seed, vgx_sampler** out);
int vgx_sampler_free(vgx_sampler* s);
/* sample_token / sample_token_report (sampling.cpp:119-142): softmax at temp,
 * top_k (0 = off) renormalised, top_p prefix, one uniform draw; temp <= 0 is
 * the first maximum.  logprob (may be NULL): of the token within the kept set. */
int vgx_sample_logits(vgx_sampler* s, const float* logits, int n, float temp, float top_p, int top_k, int* token,
                      float* logprob);
/* argmax_token_report (sampling.cpp:144-155): the first maximum and its
 * log-probability under the untempered softmax. */
int vgx_argmax_report(const float* logits, int n, int* token, float* logprob);
/* sample_candidate_result (sampling.cpp:164-199) over a candidate result
 * (value / cand_token / n, strict and stats[0] as vgx_engine_step_candidates
 * gives them); no candidates draws token 2. */
int vgx_sample_candidates(vgx_sampler* s, const float* value, const int* cand_token, int n, int strict,
                          float logsumexp, float temp, float top_p, int top_k, int* token);
/* apply_sampling_penalties (sampling.cpp:16-56) in place, with the settings
 * (1, 0, 0, 0, 0 = off) passed in; recent: the tokens generated so far. */
int vgx_apply_penalties(float* logits, int n, const int* recent, int nrecent, float repetition, float frequency,
                        float presence, int no_repeat_ngram, float min_p);

/* The message of the last failed engine call on this thread. */
const char* vgx_engine_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
