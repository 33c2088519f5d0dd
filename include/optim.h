/*
 * optim.h -- gpt.c's AdamW optimizer, unchanged interface
 * (/root/reference/include/optim.h:31-57).  The moment tensors m and v are
 * created (zeroed, on each gradient's device) by the first step().
 */
#pragma once

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct adamW {
    tensor_t **parameters;
    tensor_t **gradients;
    tensor_t **m;
    tensor_t **v;

    float lr;
    float beta1;
    float beta2;
    float eps;
    float weight_decay;

    int n_parameters;
    int step_t;
    char __padding[4];

    void (*step)(struct adamW *);
    void (*zero_grad)(struct adamW *);
    void (*free_layer)(struct adamW *);
} __attribute__((aligned(64))) adamW_t;

adamW_t *AdamW(tensor_t **parameters, tensor_t **gradients, const int n_parameters, const float lr,
               const float beta1, const float beta2, const float eps, const float weight_decay);

#ifdef __cplusplus
}
#endif
