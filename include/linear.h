/*
 * linear.h -- gpt.c's Linear layer, unchanged interface
 * (/root/reference/include/linear.h:34-61).  y = x W^T + b with
 * W (out_features, in_features).  forward() keeps x as the layer's cache
 * (ownership passes to the layer); backward() consumes the upstream
 * gradient and the cache and returns dx.
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct linear {
    tensor_t *W;
    tensor_t *b;
    tensor_t *dW;
    tensor_t *db;
    tensor_t *cache;

    tensor_t *(*forward)(struct linear *, tensor_t *);
    tensor_t *(*backward)(struct linear *, tensor_t *);
    void (*description)(const struct linear *);
    int (*num_parameters)(const struct linear *);
    void (*free_layer)(struct linear *);
    void (*free_cache)(struct linear *);
    tensor_t **(*parameters)(const struct linear *);
    tensor_t **(*gradients)(const struct linear *);
    void (*load_state_dict)(struct linear *, tensor_t **);
    void (*to)(struct linear *, const device_t);

    int in_features;
    int out_features;
    int use_bias;
    int _num_param_tensors;
} __attribute__((aligned(64))) linear_t;

linear_t *Linear(const int in_features, const int out_features, const int use_bias);

/* No counterpart in the reference: forward and backward without the bias
 * term, for a consumer that folds the bias into its own kernels (the
 * library's SelfAttention, with the fused attention).  forward: x W^T,
 * caching x as forward does; backward: dx = g W and dW += g^T x as backward
 * does, leaving db to the caller; it consumes g and the cache. */
tensor_t *gptc_linear_forward_nobias(linear_t *linear, tensor_t *x);
tensor_t *gptc_linear_backward_nodb(linear_t *linear, tensor_t *global_grad);

#ifdef __cplusplus
}
#endif
