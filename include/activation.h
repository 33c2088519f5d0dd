/*
 * activation.h -- gpt.c's GELU and Softmax layers, unchanged interface
 * (/root/reference/include/activation.h:34-56).  GELU caches its input,
 * Softmax its output; backward consumes the upstream gradient and the cache.
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gelu {
    tensor_t *cache;
    tensor_t *(*forward)(struct gelu *, tensor_t *);
    tensor_t *(*backward)(struct gelu *, tensor_t *);
    void (*description)(const struct gelu *);
    void (*free_layer)(struct gelu *);
    void (*free_cache)(struct gelu *);
    void (*to)(struct gelu *, const device_t device);
} __attribute__((aligned(64))) gelu_t;

typedef struct softmax {
    tensor_t *cache;
    tensor_t *(*forward)(struct softmax *, tensor_t *);
    tensor_t *(*backward)(struct softmax *, tensor_t *);
    void (*description)(const struct softmax *);
    void (*free_layer)(struct softmax *);
    void (*free_cache)(struct softmax *);
    void (*to)(struct softmax *, const device_t device);
} __attribute__((aligned(64))) softmax_t;

gelu_t *GELU(void);
softmax_t *Softmax(void);

/* No counterpart in the reference: GELU of x + bias (bias per last-dim
 * column), for the library's MLP, whose c_fc Linear then runs without its
 * bias (gptc_linear_forward_nobias): one pass over the activations instead
 * of gpt.c's bias add followed by GELU (src/mlp.c's forward).  forward
 * caches x (without the bias) as forward does; backward returns
 * dx = g * gelu'(x + bias), adds its column sums to db (c_fc's bias
 * gradient, which gptc_linear_backward_nodb then leaves alone) and consumes
 * g and the cache. */
tensor_t *gptc_gelu_forward_bias(gelu_t *gelu, tensor_t *x, const tensor_t *bias);
tensor_t *gptc_gelu_backward_bias(gelu_t *gelu, tensor_t *global_grad, const tensor_t *bias, tensor_t *db);

#ifdef __cplusplus
}
#endif
