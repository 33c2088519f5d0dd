/*
 * generate.h -- one-token GPT-2 steps with per-layer K/V caches.
 * No counterpart in gpt.c: its infer_gpt.c:339-351 runs the whole
 * block_size window through GPT2.forward for every new token and keeps one
 * row of the logits.  Under the causal rule that row depends on tokens
 * 0 .. i-1 only, so a decode step over cached keys and values returns the
 * same logits while reading each weight and cached row once per token.
 *
 * gptc_kv_cache_create(gpt, B, L)   per-layer K and V caches (B, H, L, D) on
 *                                   the GPU for B sequences of up to L tokens.
 * gptc_gpt2_decode(gpt, kv, ids, pos)
 *                                   ids (B, 1) token ids (floats, GPU) at
 *                                   position pos of every sequence; returns
 *                                   the logits (B, 1, V) of that position and
 *                                   stores the token's keys and values at pos.
 *                                   Positions 0 .. pos-1 must have been
 *                                   decoded before (prefill = decode them in
 *                                   order).  B <= 8, pos < L <= block_size.
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
    tensor_t **k;  // n_layers tensors (B, H, L, D)
    tensor_t **v;
    tensor_t *scratch[8];  // activations of one step, reused across steps
} gptc_kv_cache_t;

gptc_kv_cache_t *gptc_kv_cache_create(const gpt2_t *gpt, const int B, const int L);
void gptc_kv_cache_free(gptc_kv_cache_t *kv);
tensor_t *gptc_gpt2_decode(gpt2_t *gpt, gptc_kv_cache_t *kv, const tensor_t *ids, const int pos);

#ifdef __cplusplus
}
#endif
