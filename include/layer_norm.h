/*
 * layer_norm.h -- gpt.c's LayerNorm layer, unchanged interface
 * (/root/reference/include/layer_norm.h:34-62).  cache[0] mean, cache[1]
 * rstd (one per row), cache[2] the input (owned by the layer until backward).
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct layer_norm {
    int in_features;
    int use_bias;
    int _num_param_tensors;
    float eps;

    tensor_t *W;
    tensor_t *b;
    tensor_t *dW;
    tensor_t *db;
    tensor_t *cache[3];

    tensor_t *(*forward)(struct layer_norm *, tensor_t *);
    tensor_t *(*backward)(struct layer_norm *, tensor_t *);
    void (*description)(const struct layer_norm *);
    int (*num_parameters)(const struct layer_norm *);
    void (*free_layer)(struct layer_norm *);
    void (*free_cache)(struct layer_norm *);
    tensor_t **(*parameters)(const struct layer_norm *);
    tensor_t **(*gradients)(const struct layer_norm *);
    void (*load_state_dict)(struct layer_norm *, tensor_t **);
    void (*to)(struct layer_norm *, const device_t);
} __attribute__((aligned(64))) layer_norm_t;

layer_norm_t *LayerNorm(int in_features, const float eps, const int use_bias);

#ifdef __cplusplus
}
#endif
