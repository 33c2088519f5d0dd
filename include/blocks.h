/*
 * blocks.h -- gpt.c's transformer building blocks, unchanged interface
 * (/root/reference/include/blocks.h:34-113):
 *   MLP            c_fc -> GELU -> c_proj (expansion_factor * in_features wide)
 *   SelfAttention  qkv Linear -> Attention -> c_proj
 *   Block          x + attn(ln1(x)), then + mlp(ln2(.))
 * forward() consumes its input; backward() consumes the upstream gradient
 * and returns the gradient of the block input.
 */
#pragma once

#include "activation.h"
#include "attention.h"
#include "layer_norm.h"
#include "linear.h"
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mlp {
    int in_features;
    int use_bias;
    int expansion_factor;
    int _num_param_tensors;

    linear_t *c_fc;
    gelu_t *gelu;
    linear_t *c_proj;

    tensor_t *(*forward)(struct mlp *, tensor_t *);
    tensor_t *(*backward)(struct mlp *, tensor_t *);
    void (*description)(const struct mlp *);
    int (*num_parameters)(const struct mlp *);
    void (*free_layer)(struct mlp *);
    void (*free_cache)(struct mlp *);
    tensor_t **(*parameters)(const struct mlp *);
    tensor_t **(*gradients)(const struct mlp *);
    void (*load_state_dict)(struct mlp *, tensor_t **);
    void (*to)(struct mlp *, const device_t device);
} __attribute__((aligned(64))) mlp_t;

typedef struct self_attention {
    int n_embd;
    int n_heads;
    int use_bias;
    int block_size;
    int _num_param_tensors;
    char __padding[4];

    linear_t *qkv;
    attention_t *attn;
    linear_t *c_proj;

    tensor_t *(*forward)(struct self_attention *, tensor_t *);
    tensor_t *(*backward)(struct self_attention *, tensor_t *);
    void (*description)(const struct self_attention *);
    int (*num_parameters)(const struct self_attention *);
    void (*free_layer)(struct self_attention *);
    void (*free_cache)(struct self_attention *);
    tensor_t **(*parameters)(const struct self_attention *);
    tensor_t **(*gradients)(const struct self_attention *);
    void (*load_state_dict)(struct self_attention *, tensor_t **);
    void (*to)(struct self_attention *, const device_t device);
} __attribute__((aligned(64))) self_attention_t;

typedef struct block {
    int n_embd;
    int n_heads;
    int use_bias;
    int block_size;
    int _num_param_tensors;
    char __padding[4];

    layer_norm_t *ln1;
    layer_norm_t *ln2;
    mlp_t *mlp;
    self_attention_t *attn;

    tensor_t *(*forward)(struct block *, tensor_t *);
    tensor_t *(*backward)(struct block *, tensor_t *);
    void (*description)(const struct block *);
    int (*num_parameters)(const struct block *);
    void (*free_layer)(struct block *);
    void (*free_cache)(struct block *);
    tensor_t **(*parameters)(const struct block *);
    tensor_t **(*gradients)(const struct block *);
    void (*load_state_dict)(struct block *, tensor_t **);
    void (*to)(struct block *, const device_t device);
} __attribute__((aligned(64))) block_t;

mlp_t *MLP(const int in_features, int expansion_factor, const int use_bias);
self_attention_t *SelfAttention(const int n_embd, const int n_heads, const int block_size, const int use_bias);
block_t *Block(const int n_embd, const int n_heads, const int block_size, const int use_bias);

#ifdef __cplusplus
}
#endif
