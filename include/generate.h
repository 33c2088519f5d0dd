/*
 * generate.h -- one-token GPT-2 steps with per-layer K/V caches.
 * No counterpart in gpt.c: its infer_gpt.c:339-351 runs the whole
 * block_size window through GPT2.forward for every new token and keeps one
 * row of the logits.  Under the causal rule that row depends on tokens
 * 0 .. i-1 only, so a decode step over cached keys and values returns the
 * same logits while reading each weight and cached row once per token.
 *
 * gptc_kv_cache_create(gpt, B, L)   per-layer K and V caches (B, H, L, D) on
 *                                   the GPU for B <= 8 sequences of up to
 *                                   L <= block_size tokens, and the step's
 *                                   activations.
 * gptc_gpt2_decode(gpt, kv, ids, pos)
 *                                   ids (B, 1) token ids (floats, GPU) at
 *                                   position pos of every sequence; returns
 *                                   the logits (B, 1, V) of that position (a
 *                                   new tensor) and stores the token's keys
 *                                   and values at pos.  Positions 0 .. pos-1
 *                                   must have been decoded before.
 * gptc_gpt2_generate(gpt, kv, tokens, prompt, total)
 *                                   greedy generation on the GPU: tokens is a
 *                                   (B, total) float buffer holding each
 *                                   sequence's prompt in columns 0 .. prompt-1;
 *                                   columns prompt .. total-1 receive the
 *                                   argmax tokens.  One step (positions 0 ..
 *                                   total-2) is captured once as a HIP graph
 *                                   and replayed, the position living in
 *                                   device memory, so the host does not wait
 *                                   between tokens.  Returns without
 *                                   synchronising; total <= L.  The graph
 *                                   is reused by a later call only when the
 *                                   model object, the address of every
 *                                   parameter, the token buffer, prompt,
 *                                   total and the LayerNorm eps values are
 *                                   all unchanged; otherwise it is captured
 *                                   again (a model moved between devices
 *                                   has new addresses).
 * gptc_kv_cache_free(kv)
 */
#pragma once

#include "tensor.h"
#include "transformer.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gptc_kv_cache {
    int n_layers;
    int B;
    int L;
    tensor_t **k;          // n_layers tensors (B, H, L, D)
    tensor_t **v;
    tensor_t *scratch[8];  // activations of one step, reused across steps
    tensor_t *logits;      // (B, 1, V) of the captured step
    int *pos_dev;          // device-side position of the captured step
    void *graph_exec;      // hipGraphExec_t of the captured step
    unsigned long long *graph_key;  // everything the captured launches baked in
    int graph_key_len;              // (model and buffer addresses, shapes, eps):
                                    // the graph is replayed only on an exact match
} gptc_kv_cache_t;

gptc_kv_cache_t *gptc_kv_cache_create(const gpt2_t *gpt, const int B, const int L);
void gptc_kv_cache_free(gptc_kv_cache_t *kv);
tensor_t *gptc_gpt2_decode(gpt2_t *gpt, gptc_kv_cache_t *kv, const tensor_t *ids, const int pos);
void gptc_gpt2_generate(gpt2_t *gpt, gptc_kv_cache_t *kv, tensor_t *tokens, const int prompt, const int total);

#ifdef __cplusplus
}
#endif
