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

#ifdef __cplusplus
}
#endif
