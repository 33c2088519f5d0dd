/*
 * dispatch.h -- the device switch that gpt.c's layers call
 * (/root/reference/kernels/include/dispatch.h:1-13,
 *  kernels/src/core/Attention.c:6-79, kernels/src/core/Tensor.c:6-139,
 *  kernels/src/core/Alloc.c, kernels/src/core/runtime.c:5-19).
 *
 * Each *_dispatch checks that its tensors share one device (fatal
 * otherwise) and routes to the CPU or GPU implementation.  In this library
 * the GPU side is the HIP code in gpu_kernels.h.  The CPU side covers the
 * tensor data ops only: gpt.c's CPU attention kernel
 * (kernels/src/cpu/Attention.c) stays in gpt.c's own library, so
 * attention_*_dispatch with device == CPU is a fatal error here.
 */
#pragma once

#include <stddef.h>
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

void runtime_init_dispatch(const device_t device);
void runtime_destroy_dispatch(const device_t device);
void synchronize_dispatch(const device_t device);

void *alloc_dispatch(const size_t nbytes, const size_t alignment, const device_t device);
void free_dispatch(void *ptr, const device_t device);

void create_tensor_data_dispatch(tensor_t *tensor);
void zeros_tensor_data_dispatch(tensor_t *tensor);
void ones_tensor_data_dispatch(tensor_t *tensor);
void fill_tensor_data_dispatch(tensor_t *tensor, const float value);
void arange_tensor_data_dispatch(tensor_t *tensor, const int start, const int end, const int steps);
void move_tensor_data_dispatch(tensor_t *tensor, const device_t device);
void copy_tensor_data_dispatch(tensor_t *dst, const tensor_t *src);

void attention_forward_dispatch(
    const tensor_t *input,
    const tensor_t *mask,
    const int n_heads,
    tensor_t **cache,
    tensor_t *output
);

void attention_backward_dispatch(
    const tensor_t *global_grad,
    tensor_t **cache,
    const int n_heads,
    tensor_t *dout
);

#ifdef __cplusplus
}
#endif
