// Dense fp32 BLAS entry points of gpt.c's device back end: sgemm,
// strided-batched sgemm (rocBLAS on the library's stream) and saxpy (a
// HIP kernel).  Replaces kernels/src/cuda/Tensor.cu:132-206, whose GEMMs go
// through cuBLAS with TF32 math on sm >= 80 (runtime.cu:20-24); here every
// product is computed in fp32 (rocBLAS's fp32 MFMA kernels for gfx950).
//
// gpt.c's matrices are row-major; rocBLAS is column-major.  A row-major
// C (M x N) = op(A) op(B) is the column-major C^T (N x M) = op(B)^T op(A)^T,
// so each call swaps the operands and the M/N sizes and keeps the leading
// dimensions, as the reference does for cuBLAS.
#include <rocblas/rocblas.h>
#include <cstdint>
#include "blas.hpp"
#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace {

rocblas_handle g_handle = nullptr;
hipStream_t g_handle_stream = nullptr;

void blas_check(rocblas_status st, const char *what) {
    CHECK_ERROR(st != rocblas_status_success, "rocBLAS %s failed: %s", what, rocblas_status_to_string(st));
}

rocblas_operation op(int trans) { return trans == 1 ? rocblas_operation_transpose : rocblas_operation_none; }

constexpr int kThreads = 256;

// y[offy + i*incy] += alpha * x[offx + i*incx], i < n.
__global__ __launch_bounds__(kThreads) void saxpy_kernel(int64_t n, float alpha, const float *__restrict__ x,
                                                        int64_t incx, float *__restrict__ y, int64_t incy) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        y[i * incy] = fmaf(alpha, x[i * incx], y[i * incy]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Unit strides and 16-byte aligned x and y: 16-byte vectors, then the tail.
__global__ __launch_bounds__(kThreads) void saxpy_vec_kernel(int64_t n, float alpha, const float *__restrict__ x,
                                                            float *__restrict__ y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t n4 = n / 4;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const f32x4 a = reinterpret_cast<const f32x4 *>(x)[i];
        f32x4 b = reinterpret_cast<f32x4 *>(y)[i];
        b[0] = fmaf(alpha, a[0], b[0]);
        b[1] = fmaf(alpha, a[1], b[1]);
        b[2] = fmaf(alpha, a[2], b[2]);
        b[3] = fmaf(alpha, a[3], b[3]);
        reinterpret_cast<f32x4 *>(y)[i] = b;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = fmaf(alpha, x[i], y[i]);
}

// The element range [off, off + (n-1)*inc] must lie inside the tensor (inc >= 1).
void check_span(const tensor_t *t, int off, int n, int inc, const char *name) {
    CHECK_ERROR(t == NULL || t->device != CUDA, "Expected %s to be a tensor on the GPU.", name);
    CHECK_ERROR(inc < 1, "%s: increment %d is not supported (must be >= 1).", name, inc);
    if (n <= 0) return;
    const int64_t last = static_cast<int64_t>(off) + static_cast<int64_t>(n - 1) * inc;
    CHECK_ERROR(off < 0 || last >= t->length,
                "%s: elements %d .. %lld fall outside a tensor of %d elements.", name, off, (long long)last,
                t->length);
}

// Elements a row-major (rows x cols) operand with leading dimension ld spans.
void check_matrix(const tensor_t *t, int64_t off, int rows, int cols, int ld, const char *name) {
    CHECK_ERROR(t == NULL || t->device != CUDA, "Expected %s to be a tensor on the GPU.", name);
    CHECK_ERROR(ld < (cols > 1 ? cols : 1), "%s: leading dimension %d is smaller than its %d columns.", name, ld, cols);
    if (rows <= 0 || cols <= 0) return;
    const int64_t last = off + static_cast<int64_t>(rows - 1) * ld + cols - 1;
    CHECK_ERROR(off < 0 || last >= t->length, "%s: a (%d x %d) operand at offset %lld with ld %d overruns %d elements.",
                name, rows, cols, (long long)off, ld, t->length);
}

}  // namespace

rocblas_handle gptc_blas_handle() {
    hipStream_t s = gptc_stream_checked();
    if (g_handle == nullptr) {
        blas_check(rocblas_create_handle(&g_handle), "create_handle");
        // Deterministic results: no split-K with atomic accumulation.
        blas_check(rocblas_set_atomics_mode(g_handle, rocblas_atomics_not_allowed), "set_atomics_mode");
    }
    if (g_handle_stream != s) {
        blas_check(rocblas_set_stream(g_handle, s), "set_stream");
        g_handle_stream = s;
    }
    return g_handle;
}

void gptc_blas_destroy() {
    if (g_handle != nullptr) blas_check(rocblas_destroy_handle(g_handle), "destroy_handle");
    g_handle = nullptr;
    g_handle_stream = nullptr;
}

void gptc_sgemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float *A, int lda, const float *B,
                int ldb, float beta, float *C, int ldc) {
    if (M <= 0 || N <= 0) return;
    blas_check(rocblas_sgemm(gptc_blas_handle(), op(trans_b), op(trans_a), N, M, K, &alpha, B, ldb, A, lda, &beta, C,
                             ldc),
               "sgemm");
}

namespace {

// out[i] (+)= p[0][i] + p[1][i] + ... + p[S-1][i], in that order; `accumulate`
// adds the sum to out, otherwise it overwrites out.
__global__ __launch_bounds__(kThreads) void add_partials_kernel(const float *__restrict__ p, float *__restrict__ out,
                                                               int64_t n, int S, bool vec, bool accumulate) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    if (vec) {
        const int64_t n4 = n / 4;
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            f32x4 acc = reinterpret_cast<const f32x4 *>(p)[i];
            for (int s = 1; s < S; ++s) acc += reinterpret_cast<const f32x4 *>(p + s * n)[i];
            if (accumulate) {
                f32x4 o = reinterpret_cast<f32x4 *>(out)[i];
                o += acc;
                acc = o;
            }
            reinterpret_cast<f32x4 *>(out)[i] = acc;
        }
    } else {
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
            float acc = p[i];
            for (int s = 1; s < S; ++s) acc += p[s * n + i];
            out[i] = accumulate ? out[i] + acc : acc;
        }
    }
}

void launch_add_partials(const float *partial, float *out, int64_t n, int S, bool accumulate, hipStream_t s) {
    int64_t blocks = (n / 4 + kThreads - 1) / kThreads;
    if (blocks > 256 * 8) blocks = 256 * 8;
    const bool vec = (n % 4) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    add_partials_kernel<<<dim3(static_cast<int>(blocks < 1 ? 1 : blocks)), dim3(kThreads), 0, s>>>(partial, out, n, S,
                                                                                                   vec, accumulate);
    hipCheck(hipGetLastError());
}

}  // namespace

void gptc_sgemm_wgrad(int out_f, int in_f, int rows, const float *g, const float *x, float *dW) {
    if (out_f <= 0 || in_f <= 0) return;
    // Output tiles of 128 x 128; below about two per CU the GEMM cannot fill
    // 256 CUs, so the row (K) range is split into S slices computed as one
    // strided-batched GEMM, and the slices are added in a fixed order.
    const int64_t tiles = static_cast<int64_t>((out_f + 127) / 128) * ((in_f + 127) / 128);
    int S = 1;
    while (S < 8 && tiles * S < 512 && rows % (2 * S) == 0 && rows / (2 * S) >= 1024) S *= 2;
    if (S == 1) {
        gptc_sgemm(1, 0, out_f, in_f, rows, 1.0f, g, out_f, x, in_f, 1.0f, dW, in_f);
        return;
    }
    hipStream_t s = gptc_stream_checked();
    const int chunk = rows / S;
    const int64_t n = static_cast<int64_t>(out_f) * in_f;
    float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * static_cast<size_t>(n) * S));
    const float one = 1.0f, zero = 0.0f;
    // Column-major view: partial_b^T (in x out) = x_b^T (in x chunk) g_b (chunk x out).
    blas_check(rocblas_sgemm_strided_batched(gptc_blas_handle(), rocblas_operation_none, rocblas_operation_transpose,
                                             in_f, out_f, chunk, &one, x, in_f,
                                             static_cast<rocblas_stride>(chunk) * in_f, g, out_f,
                                             static_cast<rocblas_stride>(chunk) * out_f, &zero, partial, in_f, n, S),
               "sgemm_strided_batched (weight gradient)");
    launch_add_partials(partial, dW, n, S, true, s);
    free_cuda(partial);
}

void gptc_sgemm_dgrad(int rows, int in_f, int out_f, const float *g, const float *W, float *dx) {
    if (rows <= 0 || in_f <= 0) return;
    // With rocBLAS's atomics off, a product with few 128 x 128 output tiles and
    // a long reduction runs on one wave of tiles with a third of the CUs idle
    // (GPT-2's lm_head input gradient: 384 tiles, K = 50257, 113 TFLOP/s).  The
    // reduction is then split into S equal slices, as in the weight gradient,
    // while every slice keeps at least 8192 terms: below that the extra passes
    // over the slices cost more than the fuller GPU gains (measured at K = 2304
    // and 3072).  The K - S*chunk leftover terms are added into slice 0.
    const int64_t tiles = static_cast<int64_t>((rows + 127) / 128) * ((in_f + 127) / 128);
    int S = 1;
    while (S < 8 && tiles * S < 512 && out_f / (2 * S) >= 8192) S *= 2;
    if (S == 1) {
        gptc_sgemm(0, 0, rows, in_f, out_f, 1.0f, g, out_f, W, in_f, 0.0f, dx, in_f);
        return;
    }
    hipStream_t s = gptc_stream_checked();
    const int chunk = out_f / S, rest = out_f - S * chunk;
    const int64_t n = static_cast<int64_t>(rows) * in_f;
    float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * static_cast<size_t>(n) * S));
    const float one = 1.0f, zero = 0.0f;
    // Column-major view: partial_b^T (in x rows) = W_b^T (in x chunk) g_b^T (chunk x rows),
    // W_b = rows [b*chunk, (b+1)*chunk) of W, g_b = the same columns of g.
    blas_check(rocblas_sgemm_strided_batched(gptc_blas_handle(), rocblas_operation_none, rocblas_operation_none, in_f,
                                             rows, chunk, &one, W, in_f, static_cast<rocblas_stride>(chunk) * in_f, g,
                                             out_f, chunk, &zero, partial, in_f, n, S),
               "sgemm_strided_batched (input gradient)");
    if (rest > 0) {
        const int64_t k0 = static_cast<int64_t>(S) * chunk;
        blas_check(rocblas_sgemm(gptc_blas_handle(), rocblas_operation_none, rocblas_operation_none, in_f, rows, rest,
                                 &one, W + k0 * in_f, in_f, g + k0, out_f, &one, partial, in_f),
                   "sgemm (input gradient, leftover terms)");
    }
    launch_add_partials(partial, dx, n, S, false, s);
    free_cuda(partial);
}

extern "C" void sgemm_cuda(const int TransA, const int TransB, const int M, const int N, const int K,
                           const float alpha, const tensor_t *A, const int offsetA, const int lda, const tensor_t *B,
                           const int offsetB, const int ldb, const float beta, tensor_t *C, const int offsetC,
                           const int ldc) {
    CHECK_ERROR(M < 0 || N < 0 || K < 0, "sgemm: negative size M=%d N=%d K=%d.", M, N, K);
    // op(A) is M x K: A itself is (K x M) when transposed.
    check_matrix(A, offsetA, TransA == 1 ? K : M, TransA == 1 ? M : K, lda, "sgemm A");
    check_matrix(B, offsetB, TransB == 1 ? N : K, TransB == 1 ? K : N, ldb, "sgemm B");
    check_matrix(C, offsetC, M, N, ldc, "sgemm C");
    gptc_sgemm(TransA, TransB, M, N, K, alpha, A->t + offsetA, lda, B->t + offsetB, ldb, beta, C->t + offsetC, ldc);
}

extern "C" void sgemm_strided_batched_cuda(const int TransA, const int TransB, const int M, const int N, const int K,
                                           const float alpha, const tensor_t *A, const int lda, const int strideA,
                                           const tensor_t *B, const int ldb, const int strideB, const float beta,
                                           tensor_t *C, const int ldc, const int strideC, const int batch_count) {
    CHECK_ERROR(M < 0 || N < 0 || K < 0 || batch_count < 0, "sgemm_strided_batched: negative size.");
    if (M == 0 || N == 0 || batch_count == 0) return;
    const int64_t nb = batch_count - 1;
    check_matrix(A, nb * strideA, TransA == 1 ? K : M, TransA == 1 ? M : K, lda, "sgemm_strided_batched A");
    check_matrix(B, nb * strideB, TransB == 1 ? N : K, TransB == 1 ? K : N, ldb, "sgemm_strided_batched B");
    check_matrix(C, nb * strideC, M, N, ldc, "sgemm_strided_batched C");
    blas_check(rocblas_sgemm_strided_batched(gptc_blas_handle(), op(TransB), op(TransA), N, M, K, &alpha, B->t, ldb,
                                             strideB, A->t, lda, strideA, &beta, C->t, ldc, strideC, batch_count),
               "sgemm_strided_batched");
}

extern "C" void saxpy_cuda(const int n, const float alpha, const tensor_t *x, const int offsetx, const int incx,
                           tensor_t *y, const int offsety, const int incy) {
    if (n <= 0) return;
    check_span(x, offsetx, n, incx, "saxpy x");
    check_span(y, offsety, n, incy, "saxpy y");
    hipStream_t s = gptc_stream_checked();
    const float *xp = x->t + offsetx;
    float *yp = y->t + offsety;
    int64_t g = (static_cast<int64_t>(n) + kThreads * 4 - 1) / (kThreads * 4);
    if (g > 256 * 8) g = 256 * 8;
    const bool vec = incx == 1 && incy == 1 && (reinterpret_cast<uintptr_t>(xp) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(yp) & 15) == 0;
    if (vec)
        saxpy_vec_kernel<<<dim3(static_cast<int>(g)), dim3(kThreads), 0, s>>>(n, alpha, xp, yp);
    else
        saxpy_kernel<<<dim3(static_cast<int>(g)), dim3(kThreads), 0, s>>>(n, alpha, xp, incx, yp, incy);
    hipCheck(hipGetLastError());
}
