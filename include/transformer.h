/*
 * transformer.h -- gpt.c's GPT-2 model, unchanged interface
 * (/root/reference/include/transformer.h:34-79).  forward(ids (B, T)) returns
 * logits (B, T, vocab_size); backward(dlogits) accumulates every parameter
 * gradient (lm_head shares wte's weight, and its gradient is added into
 * wte's).  parameters()/gradients() list _num_param_tensors tensors in the
 * order wte, wpe, layers[0..n), ln_f.
 */
#pragma once

#include "blocks.h"
#include "embedding.h"
#include "layer_norm.h"
#include "linear.h"
#include "loss.h"
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpt2 {
    int n_embd;
    int n_heads;
    int n_layers;
    int block_size;
    int vocab_size;
    int _num_param_tensors;

    block_t **layers;
    embedding_t *wpe;
    embedding_t *wte;
    linear_t *lm_head;
    layer_norm_t *ln_f;

    tensor_t *(*forward)(struct gpt2 *, tensor_t *);
    tensor_t *(*backward)(struct gpt2 *, tensor_t *);
    void (*description)(const struct gpt2 *);
    int (*num_parameters)(const struct gpt2 *);
    void (*free_layer)(struct gpt2 *);
    void (*free_cache)(struct gpt2 *);
    tensor_t **(*parameters)(const struct gpt2 *);
    tensor_t **(*gradients)(const struct gpt2 *);
    void (*load_state_dict)(struct gpt2 *, tensor_t **);
    void (*fast_load_state_dict)(struct gpt2 *, tensor_t **);
    void (*to)(struct gpt2 *, const device_t);
} gpt2_t;

typedef struct {
    int block_size;
    int vocab_size;
    int n_layers;
    int n_heads;
    int n_embd;
} GPT2Config_t;

gpt2_t *GPT2(GPT2Config_t *config);

#ifdef __cplusplus
}
#endif
