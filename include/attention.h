/*
 * attention.h -- gpt.c's causal self-attention layer, unchanged interface
 * (/root/reference/include/attention.h:42-61).
 *
 * Attention(n_embd, n_heads, block_size) returns a layer object with the
 * same field order and function pointers as the reference:
 *   forward(attn, x)   x: (B, T, 3C) -> returns y: (B, T, C); x is consumed
 *                      (the caller must not use it afterwards);
 *   backward(attn, dy) dy: (B, T, C) -> returns dqkv: (B, T, 3C); dy is
 *                      consumed and the layer's cache is released.
 * `buffer` is the (block, block) lower-triangular mask of ones, built on
 * the host by the constructor, exactly as the reference builds it.
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct attention {
    tensor_t *buffer;
    tensor_t *cache[4];

    tensor_t *(*forward)(struct attention *, tensor_t *);
    tensor_t *(*backward)(struct attention *, tensor_t *);
    void (*description)(const struct attention *);
    int (*num_parameters)(const struct attention *);
    void (*free_layer)(struct attention *);
    void (*free_cache)(struct attention *);
    void (*to)(struct attention *, const device_t device);

    int n_embd;
    int n_heads;
} __attribute__((aligned(64))) attention_t;

attention_t *Attention(int n_embd, int n_heads, int block_size);

/* No counterpart in the reference: the layer's forward and backward with
 * the preceding qkv Linear's bias folded into the GPU kernels.  x holds
 * x W^T without the bias; the backward returns dqkv as backward does and
 * adds the bias gradient (its column sums) into db.  The library's own
 * SelfAttention uses them (gpt.c adds the bias in the Linear,
 * self_attention.c:59, and sums its gradient there). */
tensor_t *gptc_attention_forward_bias(attention_t *attn, tensor_t *x, const tensor_t *bias);
tensor_t *gptc_attention_backward_bias(attention_t *attn, tensor_t *global_grad, const tensor_t *bias, tensor_t *db);

#ifdef __cplusplus
}
#endif
