// The library's rocBLAS handle, bound to its stream, and a row-major fp32
// GEMM over raw device pointers (used by the Linear kernels and sgemm_cuda).
#pragma once

#include <rocblas/rocblas.h>

// Created on first use; fatal if the runtime has not been initialised.
rocblas_handle gptc_blas_handle();
void gptc_blas_destroy();

// Row-major C (M x N) = alpha * op(A) op(B) + beta * C, op = transpose when
// trans_* == 1 (gpt.c's sgemm convention, kernels/src/cpu/Tensor.c:81-104).
void gptc_sgemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float *A, int lda, const float *B,
                int ldb, float beta, float *C, int ldc);

// Weight gradient of a Linear layer: row-major dW (out_f x in_f) += g^T x,
// g (rows x out_f), x (rows x in_f).  Deterministic: when the output has too
// few tiles to fill the GPU, the rows are split into equal slices whose
// products are added into dW in slice order.
void gptc_sgemm_wgrad(int out_f, int in_f, int rows, const float *g, const float *x, float *dW);

// Input gradient of a Linear layer: row-major dx (rows x in_f) = g W,
// g (rows x out_f), W (out_f x in_f).  Deterministic: when the output has too
// few tiles to fill the GPU and the reduction over out_f is long, it is split
// into equal slices (plus the leftover terms, added to the first) whose
// products are summed into dx in slice order.
void gptc_sgemm_dgrad(int rows, int in_f, int out_f, const float *g, const float *W, float *dx);
