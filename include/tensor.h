/*
 * tensor.h -- the device-tensor contract of gpt.c, kept binary-compatible.
 *
 * Mirrors /root/reference/include/tensor.h:42-79: the same `device_t` enum
 * (CUDA names "the GPU"; on this build that is the HIP device), the same
 * `tensor_t` field order, sizes and 64-byte alignment, and the same function
 * signatures, so code written against gpt.c's tensor API (attention.c,
 * self_attention.c, train_gpt.c, infer_gpt.c) compiles and links unchanged.
 *
 * `t` is a host pointer when device == CPU and a device pointer when
 * device == CUDA.  create_tensor() leaves the data uninitialised; zeros(),
 * ones() and fill() initialise it.  to() moves data between host and device
 * with a synchronous copy on the library's one stream.
 */
#pragma once

#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { CPU, CUDA } device_t;

typedef struct tensor {
    float *t;
    int ndims;
    int length;
    int shape[8];
    void (*to)(struct tensor *, const device_t device);
    device_t device;
} __attribute__((aligned(64))) tensor_t;

tensor_t *create_tensor(const int *shape, const int n, const device_t device);
tensor_t *randn(const int *shape, const int n, const device_t device);
tensor_t *zeros(const int *shape, const int n, const device_t device);
tensor_t *ones(const int *shape, const int n, const device_t device);
tensor_t *fill(const int *shape, const int n, const float value, const device_t device);
tensor_t *arange(const int start, const int end, const int steps, const device_t device);

void tensor_copy(tensor_t *dest, const tensor_t *src);

/* y[offsety + i*incy] += alpha * x[offsetx + i*incx] and row-major
 * C = alpha op(A) op(B) + beta C (op = transpose when Trans* == 1); both
 * run on the GPU (reference tensor.h:62-68). */
void saxpy(const int n, const float alpha, const tensor_t *x, const int offsetx, const int incx, tensor_t *y,
           const int offsety, const int incy);
void sgemm(
    const int TransA, const int TransB, const int M, const int N, const int K,
    const float alpha, const tensor_t *A, const int offsetA, const int lda,
    const tensor_t *B, const int offsetB, const int ldb,
    const float beta, tensor_t *C, const int offsetC, const int ldc
);
/* Fill a host tensor from the C library rand(), as gpt.c's uniform()
 * (src/tensor.c:36-42,164-170) does, including its (high - low + 1) range. */
void uniform(tensor_t *tensor, const float low, const float high);

void shape(const tensor_t *tensor, char *shape);
void view(tensor_t *tensor, const int *shape, const int n);

tensor_t *tensor_load(FILE *fp, const int *shape, int n, const device_t device);
void tensor_save(FILE *fp, const tensor_t *tensor);
void free_tensor(tensor_t *tensor);
void get_tensor_device(const tensor_t *tensor, char *device);
void print_tensor(const tensor_t *tensor, const int compact);
void print_shape(const tensor_t *tensor);

#ifdef __cplusplus
}
#endif
