// Linear layer kernels, y = x W^T + b (replaces kernels/src/cuda/Linear.cu:40-95,
// semantics of kernels/src/cpu/Linear.c:4-80):
//   forward   one fp32 GEMM (rocBLAS) then a bias pass over y;
//   backward  dx = g W (overwrites dout), dW += g^T x, db += column sums of g.
// dW's GEMM has a small output (out x in) and a long reduction (B*T rows):
// it is split over row slices (one strided-batched GEMM) and the slices are
// added into dW in a fixed order, so it fills the GPU and stays deterministic.
// dx's GEMM is split the same way over its reduction (out features) when that
// is long and the output small: GPT-2's lm_head (K = 50257, 8192 x 768).
// The column sums are deterministic: workgroups sum fixed row ranges into a
// partial buffer, and a second kernel adds the partials in a fixed order
// (the reference uses one atomicAdd per workgroup and column); float4
// columns where the shape allows.
#include "blas.hpp"
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;

// y[r, c] += b[c] over rows x cols; vec: cols % 4 == 0 and 16-byte aligned rows.
__global__ __launch_bounds__(kThreads) void bias_add_kernel(float *__restrict__ y, const float *__restrict__ b,
                                                           int64_t rows, int cols, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    if (vec) {
        const int c4 = cols / 4;
        const int64_t n4 = rows * c4;
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            const int c = static_cast<int>(i % c4);
            f32x4_t v = reinterpret_cast<f32x4_t *>(y)[i];
            const f32x4_t bb = reinterpret_cast<const f32x4_t *>(b)[c];
            v += bb;
            reinterpret_cast<f32x4_t *>(y)[i] = v;
        }
    } else {
        const int64_t n = rows * cols;
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] += b[i % cols];
    }
}

// partial[blockIdx.y, c] = sum of g[r, c] over the rows r this workgroup
// owns (r = blockIdx.y * 4 + wave, stepping 4 * gridDim.y).  A wave reads 64
// consecutive columns of one row per step.
__global__ __launch_bounds__(kThreads) void colsum_partial_kernel(const float *__restrict__ g,
                                                                 float *__restrict__ partial, int rows, int cols) {
    __shared__ float red[kThreads / kWave][kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    float s = 0.0f;
    if (c < cols)
        for (int r = blockIdx.y * (kThreads / kWave) + w; r < rows; r += gridDim.y * (kThreads / kWave))
            s += g[static_cast<int64_t>(r) * cols + c];
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < cols) {
        float t = red[0][lane];
#pragma unroll
        for (int i = 1; i < kThreads / kWave; ++i) t += red[i][lane];
        partial[static_cast<int64_t>(blockIdx.y) * cols + c] = t;
    }
}

constexpr int kPartialWaves = 8;

// out[c] += sum over p < parts of partial[p, c].  A workgroup owns 64
// columns; wave w adds rows p = w, w + 8, ... and the 8 wave sums are then
// added in wave order, so the result does not depend on scheduling.
__global__ __launch_bounds__(kPartialWaves * kWave) void add_column_partials_kernel(const float *__restrict__ partial,
                                                                                  float *__restrict__ out, int parts,
                                                                                  int cols) {
    __shared__ float red[kPartialWaves][kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    float s = 0.0f;
    if (c < cols)
        for (int p = w; p < parts; p += kPartialWaves) s += partial[static_cast<int64_t>(p) * cols + c];
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < cols) {
        float t = red[0][lane];
#pragma unroll
        for (int i = 1; i < kPartialWaves; ++i) t += red[i][lane];
        out[c] += t;
    }
}

// The same two reductions on float4 columns (cols % 4 == 0, 16-byte aligned
// rows), with several loads in flight per lane.
// partial[blockIdx.y, c] = sum of g[r, c] over rows r0 .. r0+rpp-1 of part
// blockIdx.y: wave w takes rows r0 + w, r0 + w + 4, ... into two alternating
// sums; the sums are added in a fixed order (sum 0 + sum 1 per wave, then
// waves 0..3).
__global__ __launch_bounds__(kThreads) void colsum_partial4_kernel(const float *__restrict__ g,
                                                                  float *__restrict__ partial, int rows, int cols,
                                                                  int rpp) {
    __shared__ f32x4_t red[kThreads / kWave][kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int n4 = cols / 4, c4 = blockIdx.x * kWave + lane;
    const int r0 = blockIdx.y * rpp, r1 = min(rows, r0 + rpp);
    const f32x4_t *g4 = reinterpret_cast<const f32x4_t *>(g);
    f32x4_t a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
    if (c4 < n4) {
        int r = r0 + w;
        for (; r + 4 < r1; r += 8) {
            a0 += g4[static_cast<int64_t>(r) * n4 + c4];
            a1 += g4[static_cast<int64_t>(r + 4) * n4 + c4];
        }
        if (r < r1) a0 += g4[static_cast<int64_t>(r) * n4 + c4];
    }
    red[w][lane] = a0 + a1;
    __syncthreads();
    if (w == 0 && c4 < n4) {
        f32x4_t t = red[0][lane];
#pragma unroll
        for (int i = 1; i < kThreads / kWave; ++i) t += red[i][lane];
        reinterpret_cast<f32x4_t *>(partial)[static_cast<int64_t>(blockIdx.y) * n4 + c4] = t;
    }
}

constexpr int kSlices = 32;  // part slices per workgroup of add_column_partials4_kernel

// out[c] += sum over p < parts of partial[p, c]: thread (slice sl, float4
// column c4) adds parts sl, sl + 32, ... into four alternating sums (added in
// order), and the 32 slice sums are then added in slice order.
__global__ __launch_bounds__(kThreads) void add_column_partials4_kernel(const float *__restrict__ partial,
                                                                       float *__restrict__ out, int parts, int cols) {
    constexpr int kGroups = kThreads / kSlices;  // float4 columns per workgroup
    __shared__ f32x4_t red[kSlices][kGroups];
    const int cl = threadIdx.x % kGroups, sl = threadIdx.x / kGroups;
    const int n4 = cols / 4, c4 = blockIdx.x * kGroups + cl;
    const f32x4_t *p4 = reinterpret_cast<const f32x4_t *>(partial);
    f32x4_t a[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (c4 < n4) {
        int p = sl;
        for (; p + 3 * kSlices < parts; p += 4 * kSlices)
#pragma unroll
            for (int k = 0; k < 4; ++k) a[k] += p4[static_cast<int64_t>(p + k * kSlices) * n4 + c4];
#pragma unroll
        for (int k = 0; k < 3; ++k)  // at most three parts are left
            if (p + k * kSlices < parts) a[k] += p4[static_cast<int64_t>(p + k * kSlices) * n4 + c4];
    }
    red[sl][cl] = (a[0] + a[1]) + (a[2] + a[3]);
    __syncthreads();
    if (sl == 0 && c4 < n4) {
        f32x4_t t = red[0][cl];
#pragma unroll
        for (int i = 1; i < kSlices; ++i) t += red[i][cl];
        f32x4_t o = reinterpret_cast<f32x4_t *>(out)[c4];
        o += t;
        reinterpret_cast<f32x4_t *>(out)[c4] = o;
    }
}

bool aligned16p(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void launch_bias_add(float *y, const float *b, int64_t rows, int cols, hipStream_t s) {
    const bool vec = (cols % 4) == 0 && aligned16(y) && aligned16(b);
    const int64_t items = vec ? rows * (cols / 4) : rows * cols;
    bias_add_kernel<<<dim3(blocks_for(items, kThreads * 4)), dim3(kThreads), 0, s>>>(y, b, rows, cols, vec);
    hipCheck(hipGetLastError());
}

// out[c] += sum_r g[r, c] for a row-major (rows x cols) g, deterministic.
void launch_column_sum_add(const float *g, float *out, int rows, int cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    if (cols % 4 == 0 && aligned16p(g) && aligned16p(out)) {
        // About 1024 workgroups of 256 float4 columns x rpp rows.
        const int cblocks = (cols / 4 + kWave - 1) / kWave;
        int parts = (1024 + cblocks - 1) / cblocks;
        if (parts > rows) parts = rows;
        const int rpp = (rows + parts - 1) / parts;
        parts = (rows + rpp - 1) / rpp;
        float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * static_cast<size_t>(parts) * cols));
        colsum_partial4_kernel<<<dim3(cblocks, parts), dim3(kThreads), 0, s>>>(g, partial, rows, cols, rpp);
        hipCheck(hipGetLastError());
        launch_add_column_partials(partial, out, parts, cols, s);
        free_cuda(partial);
        return;
    }
    const int cblocks = (cols + kWave - 1) / kWave;
    int parts = 1024 / cblocks;
    const int max_parts = (rows + 3) / 4;
    if (parts > max_parts) parts = max_parts;
    if (parts > 256) parts = 256;
    if (parts < 1) parts = 1;
    float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * static_cast<size_t>(parts) * cols));
    colsum_partial_kernel<<<dim3(cblocks, parts), dim3(kThreads), 0, s>>>(g, partial, rows, cols);
    hipCheck(hipGetLastError());
    launch_add_column_partials(partial, out, parts, cols, s);
    free_cuda(partial);
}

void launch_add_column_partials(const float *partial, float *out, int parts, int cols, hipStream_t s) {
    if (parts <= 0 || cols <= 0) return;
    if (cols % 4 == 0 && aligned16p(partial) && aligned16p(out)) {
        const int groups = kThreads / kSlices;
        add_column_partials4_kernel<<<dim3((cols / 4 + groups - 1) / groups), dim3(kThreads), 0, s>>>(partial, out,
                                                                                                     parts, cols);
        hipCheck(hipGetLastError());
        return;
    }
    add_column_partials_kernel<<<dim3((cols + kWave - 1) / kWave), dim3(kPartialWaves * kWave), 0, s>>>(partial, out,
                                                                                                     parts, cols);
    hipCheck(hipGetLastError());
}

}  // namespace gptc

using namespace gptc;

extern "C" void linear_forward_cuda_kernel(const tensor_t *W, const tensor_t *b, const tensor_t *input,
                                           tensor_t *output) {
    check_gpu(W, "W");
    check_gpu(input, "input");
    check_gpu(output, "output");
    CHECK_ERROR(W->ndims != 2, "Expected W to be (out_features, in_features), but got %d dims.", W->ndims);
    const int out_f = W->shape[0], in_f = W->shape[1];
    CHECK_ERROR(last_dim(input) != in_f, "Expected input's last dimension to be %d, but got %d.", in_f,
                last_dim(input));
    const int rows = leading_rows(input);
    CHECK_ERROR(static_cast<int64_t>(rows) * out_f != output->length,
                "Expected output to hold %d x %d elements, but it holds %d.", rows, out_f, output->length);
    if (b != NULL) {
        check_gpu(b, "b");
        CHECK_ERROR(b->length != out_f, "Expected b to hold %d elements, but got %d.", out_f, b->length);
    }
    hipStream_t s = gptc_stream_checked();
    gptc_sgemm(0, 1, rows, out_f, in_f, 1.0f, input->t, in_f, W->t, in_f, 0.0f, output->t, out_f);
    if (b != NULL && rows > 0) launch_bias_add(output->t, b->t, rows, out_f, s);
}

extern "C" void linear_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, const tensor_t *W,
                                            tensor_t *dW, tensor_t *db, tensor_t *dout) {
    check_gpu(global_grad, "global_grad");
    check_gpu(cache, "cache");
    check_gpu(W, "W");
    check_gpu(dW, "dW");
    check_gpu(dout, "dout");
    CHECK_ERROR(W->ndims != 2, "Expected W to be (out_features, in_features), but got %d dims.", W->ndims);
    const int out_f = W->shape[0], in_f = W->shape[1];
    const int rows = leading_rows(global_grad);
    CHECK_ERROR(last_dim(global_grad) != out_f, "Expected global_grad's last dimension to be %d, but got %d.", out_f,
                last_dim(global_grad));
    CHECK_ERROR(static_cast<int64_t>(rows) * in_f != cache->length || cache->length != dout->length,
                "Expected the cached input and dout to hold %d x %d elements.", rows, in_f);
    CHECK_ERROR(dW->length != W->length, "Expected dW to match W's %d elements, but got %d.", W->length, dW->length);
    if (db != NULL) {
        check_gpu(db, "db");
        CHECK_ERROR(db->length != out_f, "Expected db to hold %d elements, but got %d.", out_f, db->length);
    }
    hipStream_t s = gptc_stream_checked();
    // dx = g W : (rows x out) (out x in), split over out when the reduction is long and the output small
    gptc_sgemm_dgrad(rows, in_f, out_f, global_grad->t, W->t, dout->t);
    // dW += g^T x : (out x rows) (rows x in), split over rows when the output is small
    gptc_sgemm_wgrad(out_f, in_f, rows, global_grad->t, cache->t, dW->t);
    if (db != NULL) launch_column_sum_add(global_grad->t, db->t, rows, out_f, s);
}
