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
 * attention_*_dispatch with device == CPU is a fatal error here, and so
 * are the other compute dispatchers below (gpt.c's CPU kernels over
 * OpenBLAS are not part of this library).
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

/* The other layers' device switches (kernels/src/core/{Linear,LayerNorm,
 * GeLU,Softmax,Embedding,CrossEntropyLoss,AdamW,Tensor}.h).  Same rule: the
 * GPU kernels of gpu_kernels.h, device == CPU is fatal. */
void saxpy_dispatch(const int n, const float alpha, const tensor_t *x, const int offsetx, const int incx,
                    tensor_t *y, const int offsety, const int incy);
void sgemm_dispatch(const int TransA, const int TransB, const int M, const int N, const int K, const float alpha,
                    const tensor_t *A, const int offsetA, const int lda, const tensor_t *B, const int offsetB,
                    const int ldb, const float beta, tensor_t *C, const int offsetC, const int ldc);
void linear_forward_dispatch(const tensor_t *W, const tensor_t *b, const tensor_t *input, tensor_t *output);
void linear_backward_dispatch(const tensor_t *global_grad, const tensor_t *cache, const tensor_t *W, tensor_t *dW,
                              tensor_t *db, tensor_t *dout);
void layer_norm_forward_dispatch(const tensor_t *W, const tensor_t *b, const tensor_t *input, const float eps,
                                 tensor_t **cache, tensor_t *output);
void layer_norm_backward_dispatch(const tensor_t *global_grad, const tensor_t **cache, const tensor_t *W,
                                  tensor_t *dW, tensor_t *db, tensor_t *dout);
void gelu_forward_dispatch(const tensor_t *input, tensor_t *output);
void gelu_backward_dispatch(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout);
void softmax_forward_dispatch(const tensor_t *input, tensor_t *output);
void softmax_backward_dispatch(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout);
void embedding_forward_dispatch(const tensor_t *W, const tensor_t *input, tensor_t *output);
void embedding_backward_dispatch(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dW);
void cross_entropy_forward_dispatch(const tensor_t *logits, const tensor_t *targets, tensor_t **cache,
                                    tensor_t *output);
void cross_entropy_backward_dispatch(const tensor_t *global_grad, const tensor_t **cache, tensor_t *dout);
void step_adamW_dispatch(tensor_t **parameters, tensor_t **gradients, tensor_t **m, tensor_t **v, const int n,
                         const float lr, const float beta1, const float beta2, const float weight_decay,
                         const float eps, const int step);
void zero_grad_adamW_dispatch(tensor_t **gradients, const int n);

#ifdef __cplusplus
}
#endif
