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
// rocblas_gemm_ex's solution_index is part of the stable API; only the
// listing of solutions (used by the tuner, not here) is a beta feature.
#include <rocblas/rocblas.h>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <set>
#include <tuple>
#include "blas.hpp"
#include "gemm_tuned.hpp"
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

namespace {

// Tuned solutions.  rocBLAS picks a Tensile kernel for a GEMM by a heuristic;
// for the GEMMs of a GPT-2 small training step that pick runs 5-24 % slower
// than the fastest solution rocBLAS itself lists for the same problem.  The
// table gemm_tuned.inc (written by tune_gemm from a log of the library's own
// calls, see gemm_tuned.hpp) names that solution per problem.  A listed
// problem is run with its solution, checked by rocBLAS on first use; a
// solution that this rocBLAS rejects (another version) is dropped with one
// warning and the problem runs on the default pick, as every unlisted one
// does.  The choice is fixed per problem, so results stay deterministic.
const gptc::GemmTuned kTuned[] = {
    {{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, 0},  // never matches: GEMMs with m = 0 return before the lookup
#include "gemm_tuned.inc"
};
constexpr int kNumTuned = sizeof(kTuned) / sizeof(kTuned[0]);
std::atomic<signed char> g_tuned_state[kNumTuned > 0 ? kNumTuned : 1];  // 0 untried, 1 accepted, -1 rejected

int find_tuned(const gptc::GemmProblem &p) {
    for (int i = 0; i < kNumTuned; ++i)
        if (kTuned[i].problem == p) return i;
    return -1;
}

// GPTC_GEMM_LOG=path: append each distinct problem this process runs to
// path, one line each (the tuner's input).
void log_problem(const gptc::GemmProblem &p) {
    static const char *path = std::getenv("GPTC_GEMM_LOG");
    if (path == nullptr || *path == '\0') return;
    static std::mutex mu;
    static std::set<std::tuple<int, int, int, int, int, int, int, int, long long, long long, long long, int, int, int>>
        seen;
    std::lock_guard<std::mutex> lk(mu);
    if (!seen.insert(std::make_tuple(p.ta, p.tb, p.m, p.n, p.k, p.lda, p.ldb, p.ldc, p.sa, p.sb, p.sc, p.batch,
                                     p.beta_zero, p.alpha_one))
             .second)
        return;
    FILE *f = std::fopen(path, "a");
    if (f == nullptr) return;
    std::fprintf(f, "%d %d %d %d %d %d %d %d %lld %lld %lld %d %d %d\n", p.ta, p.tb, p.m, p.n, p.k, p.lda, p.ldb, p.ldc,
                 p.sa, p.sb, p.sc, p.batch, p.beta_zero, p.alpha_one);
    std::fclose(f);
}

// rocblas_gemm_ex / _strided_batched_ex of p with solution sol and flags.
rocblas_status gemm_ex(const gptc::GemmProblem &p, int sol, uint32_t flags, float alpha, const float *A,
                       const float *B, float beta, float *C) {
    const rocblas_operation ta = p.ta ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_operation tb = p.tb ? rocblas_operation_transpose : rocblas_operation_none;
    const rocblas_datatype f32 = rocblas_datatype_f32_r;
    if (p.batch == 0)
        return rocblas_gemm_ex(gptc_blas_handle(), ta, tb, p.m, p.n, p.k, &alpha, A, f32, p.lda, B, f32, p.ldb, &beta,
                               C, f32, p.ldc, C, f32, p.ldc, f32, rocblas_gemm_algo_solution_index, sol, flags);
    return rocblas_gemm_strided_batched_ex(gptc_blas_handle(), ta, tb, p.m, p.n, p.k, &alpha, A, f32, p.lda, p.sa, B,
                                           f32, p.ldb, p.sb, &beta, C, f32, p.ldc, p.sc, C, f32, p.ldc, p.sc, p.batch,
                                           f32, rocblas_gemm_algo_solution_index, sol, flags);
}

// The tuned solution of p, run; false when p has none (or it was rejected).
// On first use the solution is validated (rocblas_gemm_flags_check_solution_index
// only checks the index; it does not compute), then every call runs it.
bool run_tuned(const gptc::GemmProblem &p, float alpha, const float *A, const float *B, float beta, float *C) {
    const int i = find_tuned(p);
    if (i < 0) return false;
    const signed char state = g_tuned_state[i].load(std::memory_order_relaxed);
    if (state < 0) return false;
    if (state == 0) {
        const rocblas_status st =
            gemm_ex(p, kTuned[i].solution, rocblas_gemm_flags_check_solution_index, alpha, A, B, beta, C);
        if (st != rocblas_status_success) {
            g_tuned_state[i].store(-1, std::memory_order_relaxed);
            std::fprintf(stderr,
                         "gptc: rocBLAS rejects tuned solution %d for a %dx%dx%d GEMM (%s); using its default pick.\n",
                         kTuned[i].solution, p.m, p.n, p.k, rocblas_status_to_string(st));
            return false;
        }
        g_tuned_state[i].store(1, std::memory_order_relaxed);
    }
    blas_check(gemm_ex(p, kTuned[i].solution, rocblas_gemm_flags_none, alpha, A, B, beta, C),
               "gemm_ex (tuned solution)");
    return true;
}

gptc::GemmProblem problem(rocblas_operation ta, rocblas_operation tb, int m, int n, int k, int lda, int ldb, int ldc,
                          long long sa, long long sb, long long sc, int batch, float alpha, float beta) {
    gptc::GemmProblem p;
    p.ta = ta == rocblas_operation_transpose;
    p.tb = tb == rocblas_operation_transpose;
    p.m = m, p.n = n, p.k = k, p.lda = lda, p.ldb = ldb, p.ldc = ldc;
    p.sa = sa, p.sb = sb, p.sc = sc, p.batch = batch;
    p.beta_zero = beta == 0.0f;
    p.alpha_one = alpha == 1.0f;
    return p;
}

// Column-major rocBLAS GEMM / strided-batched GEMM, through the tuned table.
void colmajor_gemm(rocblas_operation ta, rocblas_operation tb, int m, int n, int k, float alpha, const float *A,
                   int lda, const float *B, int ldb, float beta, float *C, int ldc, const char *what) {
    const gptc::GemmProblem p = problem(ta, tb, m, n, k, lda, ldb, ldc, 0, 0, 0, 0, alpha, beta);
    log_problem(p);
    if (run_tuned(p, alpha, A, B, beta, C)) return;
    blas_check(rocblas_sgemm(gptc_blas_handle(), ta, tb, m, n, k, &alpha, A, lda, B, ldb, &beta, C, ldc), what);
}

void colmajor_gemm_batched(rocblas_operation ta, rocblas_operation tb, int m, int n, int k, float alpha,
                           const float *A, int lda, long long sa, const float *B, int ldb, long long sb, float beta,
                           float *C, int ldc, long long sc, int batch, const char *what) {
    const gptc::GemmProblem p = problem(ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, batch, alpha, beta);
    log_problem(p);
    if (run_tuned(p, alpha, A, B, beta, C)) return;
    blas_check(rocblas_sgemm_strided_batched(gptc_blas_handle(), ta, tb, m, n, k, &alpha, A, lda, sa, B, ldb, sb,
                                             &beta, C, ldc, sc, batch),
               what);
}

}  // namespace

void gptc_sgemm(int trans_a, int trans_b, int M, int N, int K, float alpha, const float *A, int lda, const float *B,
                int ldb, float beta, float *C, int ldc) {
    if (M <= 0 || N <= 0) return;
    colmajor_gemm(op(trans_b), op(trans_a), N, M, K, alpha, B, ldb, A, lda, beta, C, ldc, "sgemm");
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
    // Output tiles of 128 x 128; below about two per CU rocBLAS's default
    // pick cannot fill 256 CUs, so the row (K) range is split into S slices
    // computed as one strided-batched GEMM, and the slices are added in a
    // fixed order.
    // A tuned solution for one of the split counts 1, 2, 4, 8 fixes S: the
    // table holds one per weight gradient, chosen with the slices' add pass
    // counted (with tuned kernels GPT-2's c_fc and c_proj products fill the
    // GPU unsplit).
    const int64_t n_out = static_cast<int64_t>(out_f) * in_f;
    int S = 0;
    for (int s = 1; s <= 8 && S == 0; s *= 2) {
        if (rows % s != 0) continue;
        const int c = rows / s;
        const gptc::GemmProblem p =
            s == 1 ? problem(rocblas_operation_none, rocblas_operation_transpose, in_f, out_f, rows, in_f, out_f, in_f,
                             0, 0, 0, 0, 1.0f, 1.0f)
                   : problem(rocblas_operation_none, rocblas_operation_transpose, in_f, out_f, c, in_f, out_f, in_f,
                             static_cast<long long>(c) * in_f, static_cast<long long>(c) * out_f, n_out, s, 1.0f, 0.0f);
        if (find_tuned(p) >= 0) S = s;
    }
    if (S == 0) {
        const int64_t tiles = static_cast<int64_t>((out_f + 127) / 128) * ((in_f + 127) / 128);
        S = 1;
        while (S < 8 && tiles * S < 512 && rows % (2 * S) == 0 && rows / (2 * S) >= 1024) S *= 2;
    }
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
    colmajor_gemm_batched(rocblas_operation_none, rocblas_operation_transpose, in_f, out_f, chunk, one, x, in_f,
                          static_cast<long long>(chunk) * in_f, g, out_f, static_cast<long long>(chunk) * out_f, zero,
                          partial, in_f, n, S, "sgemm_strided_batched (weight gradient)");
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
    colmajor_gemm_batched(rocblas_operation_none, rocblas_operation_none, in_f, rows, chunk, one, W, in_f,
                          static_cast<long long>(chunk) * in_f, g, out_f, chunk, zero, partial, in_f, n, S,
                          "sgemm_strided_batched (input gradient)");
    if (rest > 0) {
        const int64_t k0 = static_cast<int64_t>(S) * chunk;
        colmajor_gemm(rocblas_operation_none, rocblas_operation_none, in_f, rows, rest, one, W + k0 * in_f, in_f,
                      g + k0, out_f, one, partial, in_f, "sgemm (input gradient, leftover terms)");
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
    colmajor_gemm_batched(op(TransB), op(TransA), N, M, K, alpha, B->t, ldb, strideB, A->t, lda, strideA, beta, C->t,
                          ldc, strideC, batch_count, "sgemm_strided_batched");
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
