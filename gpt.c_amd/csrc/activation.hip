// GELU (tanh form) and row softmax (replaces kernels/src/cuda/GeLU.cu and
// Softmax.cu, semantics of kernels/src/cpu/GeLU.c:7-42 and
// kernels/src/cpu/Softmax.c:7-63).
//   gelu fwd   y = 0.5 x (1 + tanh(k (x + 0.044715 x^3))), k = sqrt(2/pi)
//   gelu bwd   dout = g * d/dx gelu(x), written (not accumulated)
//   with bias  the same of x + b per column (the MLP's c_fc bias folded in),
//              the backward also adding dout's column sums to db
//   softmax    rows of the last dimension: one online (max, sum) pass over the
//              row, then y = exp(x - max) * (1/sum), the reciprocal-multiply
//              normalisation of the reference
//   softmax bwd dout = (g - sum(g p)) p
// Elementwise kernels are grid-stride loops over 16-byte vectors; row kernels
// give each row one 256-thread workgroup.
#include <cmath>
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// sqrt(2) * (2/sqrt(pi)) * 0.5 = sqrt(2/pi), rounded to float once.
constexpr float kBeta = static_cast<float>(M_SQRT2 * M_2_SQRTPI * 0.5);

__device__ __forceinline__ float gelu_f(float x) {
    const float cube = 0.044715f * x * x * x;
    return 0.5f * x * (1.0f + tanhf(kBeta * (x + cube)));
}

__device__ __forceinline__ float gelu_grad(float x) {
    const float x_sq = x * x;
    const float x_cube = x_sq * x;
    const float inner = kBeta * (x + 0.044715f * x_cube);
    const float th = tanhf(inner);
    const float left = 0.5f * x;
    const float right = 1.0f + th;
    const float left_d = 0.5f * right;
    const float tanh_d = 1.0f - th * th;
    const float inner_d = kBeta * (1.0f + 3.0f * 0.044715f * x_sq);
    return left_d + left * tanh_d * inner_d;
}

__global__ __launch_bounds__(kThreads) void gelu_fwd_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                           int64_t n, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t n4 = vec ? n / 4 : 0;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        f32x4_t v = reinterpret_cast<const f32x4_t *>(x)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_f(v[e]);
        reinterpret_cast<f32x4_t *>(y)[i] = v;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = gelu_f(x[i]);
}

__global__ __launch_bounds__(kThreads) void gelu_bwd_kernel(const float *__restrict__ g, const float *__restrict__ x,
                                                           float *__restrict__ dout, int64_t n, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    const int64_t n4 = vec ? n / 4 : 0;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
        const f32x4_t xv = reinterpret_cast<const f32x4_t *>(x)[i];
        f32x4_t gv = reinterpret_cast<const f32x4_t *>(g)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = gv[e] * gelu_grad(xv[e]);
        reinterpret_cast<f32x4_t *>(dout)[i] = gv;
    }
    for (int64_t i = 4 * n4 + blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) dout[i] = g[i] * gelu_grad(x[i]);
}

// The MLP's c_fc bias folded into GELU (the Linear runs without it):
// y = gelu(h + b[c]) over rows x cols, h kept as GELU's cache.  float4
// columns (cols % 4 == 0, 16-byte aligned rows) or one element per thread.
// Element indices fit 32 bits (a tensor holds at most 2^31 - 1 elements).
__global__ __launch_bounds__(kThreads) void gelu_bias_fwd_kernel(const float *__restrict__ h,
                                                                const float *__restrict__ b, float *__restrict__ y,
                                                                int64_t rows, int cols, bool vec) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    if (vec) {
        const int c4 = cols / 4;
        const int64_t n4 = rows * c4;
        for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n4; i += stride) {
            f32x4_t v = reinterpret_cast<const f32x4_t *>(h)[i] + reinterpret_cast<const f32x4_t *>(b)[static_cast<uint32_t>(i) % static_cast<uint32_t>(c4)];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_f(v[e]);
            reinterpret_cast<f32x4_t *>(y)[i] = v;
        }
        return;
    }
    const int64_t n = rows * cols;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) y[i] = gelu_f(h[i] + b[static_cast<uint32_t>(i) % static_cast<uint32_t>(cols)]);
}

// The same on float4 columns with a fixed column per thread: workgroup
// (x, y) covers float4 columns [256 x, 256 x + 256) of rows y, y + gridDim.y,
// ..., four rows per round with their loads issued together; the bias is
// loaded once per thread and no index is divided.
__global__ __launch_bounds__(kThreads) void gelu_bias_fwd4_kernel(const float *__restrict__ h,
                                                                 const float *__restrict__ b, float *__restrict__ y,
                                                                 int rows, int c4n) {
    const int c4 = blockIdx.x * kThreads + threadIdx.x;
    if (c4 >= c4n) return;
    const f32x4_t *h4 = reinterpret_cast<const f32x4_t *>(h);
    f32x4_t *y4 = reinterpret_cast<f32x4_t *>(y);
    const f32x4_t bv = reinterpret_cast<const f32x4_t *>(b)[c4];
    const int ry = gridDim.y;
    for (int r0 = blockIdx.y; r0 < rows; r0 += 4 * ry) {
        f32x4_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = min(r0 + u * ry, rows - 1);  // past the end: repeats a row, not stored
            v[u] = h4[static_cast<int64_t>(r) * c4n + c4];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = r0 + u * ry;
            if (r < rows) {
                f32x4_t o = v[u] + bv;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = gelu_f(o[e]);
                y4[static_cast<int64_t>(r) * c4n + c4] = o;
            }
        }
    }
}

// dout = g * gelu'(h + b[c]) over rows x cols (float4 columns, 16-byte
// aligned), and partial[blockIdx.y, c] = the column sums of dout over rows
// r0 .. r0 + rpp - 1 of part blockIdx.y (the bias gradient's partials, added
// in a fixed order afterwards).  Workgroup (x, y) owns 64 float4 columns;
// wave w takes rows r0 + w, r0 + w + 4, ... four at a time (their loads
// issued together), the four waves' sums are added in wave order.
__global__ __launch_bounds__(kThreads) void gelu_bias_bwd_kernel(const float *__restrict__ g,
                                                                const float *__restrict__ h,
                                                                const float *__restrict__ b,
                                                                float *__restrict__ dout,
                                                                float *__restrict__ partial, int rows, int cols,
                                                                int rpp) {
    __shared__ f32x4_t red[kWaves][kWave];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int n4 = cols / 4, c4 = blockIdx.x * kWave + lane;
    const int r0 = blockIdx.y * rpp, r1 = min(rows, r0 + rpp);
    const f32x4_t *g4 = reinterpret_cast<const f32x4_t *>(g);
    const f32x4_t *h4 = reinterpret_cast<const f32x4_t *>(h);
    f32x4_t *d4 = reinterpret_cast<f32x4_t *>(dout);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (c4 < n4) {
        const f32x4_t bv = reinterpret_cast<const f32x4_t *>(b)[c4];
        for (int r = r0 + w; r < r1; r += 4 * kWaves) {
            f32x4_t gv[4], hv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int ru = min(r + u * kWaves, r1 - 1);  // past r1: repeats a row, not used
                gv[u] = g4[static_cast<int64_t>(ru) * n4 + c4];
                hv[u] = h4[static_cast<int64_t>(ru) * n4 + c4];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int ru = r + u * kWaves;
                if (ru < r1) {
                    const f32x4_t x = hv[u] + bv;
                    f32x4_t d;
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[e] = gv[u][e] * gelu_grad(x[e]);
                    d4[static_cast<int64_t>(ru) * n4 + c4] = d;
                    acc += d;
                }
            }
        }
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w == 0 && c4 < n4) {
        f32x4_t t = red[0][lane];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) t += red[i][lane];
        reinterpret_cast<f32x4_t *>(partial)[static_cast<int64_t>(blockIdx.y) * n4 + c4] = t;
    }
}

// The same without float4 columns: dout only (the column sums follow in
// launch_column_sum_add).
__global__ __launch_bounds__(kThreads) void gelu_bias_bwd_scalar_kernel(const float *__restrict__ g,
                                                                       const float *__restrict__ h,
                                                                       const float *__restrict__ b,
                                                                       float *__restrict__ dout, int64_t rows,
                                                                       int cols) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads, n = rows * cols;
    for (int64_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        dout[i] = g[i] * gelu_grad(h[i] + b[static_cast<uint32_t>(i) % static_cast<uint32_t>(cols)]);
}

// Workgroup-wide online (max, sum) of a row; every thread gets the result.
__device__ __forceinline__ void block_online(float &m, float &s) {
    __shared__ float sm[kWaves], ss[kWaves];
    wave_online(m, s);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sm[w] = m;
        ss[w] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) online_merge(m, s, sm[i], ss[i]);
}

__device__ __forceinline__ float block_sum(float v) {
    __shared__ float sv[kWaves];
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) sv[w] = v;
    __syncthreads();
    float t = sv[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) t += sv[i];
    return t;
}

__global__ __launch_bounds__(kThreads) void softmax_fwd_kernel(const float *__restrict__ x, float *__restrict__ y,
                                                              int C) {
    const float *xr = x + static_cast<int64_t>(blockIdx.x) * C;
    float *yr = y + static_cast<int64_t>(blockIdx.x) * C;
    float m = -INFINITY, s = 0.0f;
    for (int j = threadIdx.x; j < C; j += kThreads) {
        const float v = xr[j];
        if (v > m) {
            s = s * expf(m - v) + 1.0f;
            m = v;
        } else if (v != -INFINITY) {  // -inf entries add nothing (and -inf - -inf is NaN)
            s += expf(v - m);
        }
    }
    block_online(m, s);
    const float inv = 1.0f / s;
    for (int j = threadIdx.x; j < C; j += kThreads) yr[j] = expf(xr[j] - m) * inv;
}

__global__ __launch_bounds__(kThreads) void softmax_bwd_kernel(const float *__restrict__ g, const float *__restrict__ p,
                                                              float *__restrict__ dout, int C) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * C;
    float acc = 0.0f;
    for (int j = threadIdx.x; j < C; j += kThreads) acc += g[base + j] * p[base + j];
    const float sum = block_sum(acc);
    for (int j = threadIdx.x; j < C; j += kThreads) dout[base + j] = (g[base + j] - sum) * p[base + j];
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void gelu_forward_cuda_kernel(const tensor_t *input, tensor_t *output) {
    check_gpu(input, "input");
    check_gpu(output, "output");
    CHECK_ERROR(output->length != input->length, "Expected output to match input's %d elements.", input->length);
    const int64_t n = input->length;
    if (n == 0) return;
    const bool vec = aligned16(input->t) && aligned16(output->t);
    gelu_fwd_kernel<<<dim3(blocks_for(vec ? n / 4 : n, kThreads)), dim3(kThreads), 0, gptc_stream_checked()>>>(
        input->t, output->t, n, vec);
    hipCheck(hipGetLastError());
}

extern "C" void gelu_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout) {
    check_gpu(global_grad, "global_grad");
    check_gpu(cache, "cache");
    check_gpu(dout, "dout");
    CHECK_ERROR(global_grad->length != cache->length || dout->length != cache->length,
                "Expected global_grad, cache and dout to hold %d elements each.", cache->length);
    const int64_t n = cache->length;
    if (n == 0) return;
    const bool vec = aligned16(global_grad->t) && aligned16(cache->t) && aligned16(dout->t);
    gelu_bwd_kernel<<<dim3(blocks_for(vec ? n / 4 : n, kThreads)), dim3(kThreads), 0, gptc_stream_checked()>>>(
        global_grad->t, cache->t, dout->t, n, vec);
    hipCheck(hipGetLastError());
}

extern "C" void gptc_gelu_forward_bias_cuda(const tensor_t *input, const tensor_t *bias, tensor_t *output) {
    check_gpu(input, "input");
    check_gpu(bias, "bias");
    check_gpu(output, "output");
    const int cols = last_dim(input), rows = leading_rows(input);
    CHECK_ERROR(bias->length != cols, "Expected the bias to hold %d elements, but got %d.", cols, bias->length);
    CHECK_ERROR(output->length != input->length, "Expected output to match input's %d elements.", input->length);
    if (rows == 0 || cols == 0) return;
    const bool vec = cols % 4 == 0 && aligned16(input->t) && aligned16(bias->t) && aligned16(output->t);
    if (vec) {
        // About 2048 workgroups: the column blocks times row strides.
        const int cblocks = (cols / 4 + kThreads - 1) / kThreads;
        int ry = (2048 + cblocks - 1) / cblocks;
        if (ry > rows) ry = rows;
        if (ry > 65535) ry = 65535;
        gelu_bias_fwd4_kernel<<<dim3(cblocks, ry), dim3(kThreads), 0, gptc_stream_checked()>>>(
            input->t, bias->t, output->t, rows, cols / 4);
    } else {
        gelu_bias_fwd_kernel<<<dim3(blocks_for(static_cast<int64_t>(rows) * cols, kThreads)), dim3(kThreads), 0,
                               gptc_stream_checked()>>>(input->t, bias->t, output->t, rows, cols, false);
    }
    hipCheck(hipGetLastError());
}

extern "C" void gptc_gelu_backward_bias_cuda(const tensor_t *global_grad, const tensor_t *cache, const tensor_t *bias,
                                             tensor_t *dout, tensor_t *db) {
    check_gpu(global_grad, "global_grad");
    check_gpu(cache, "cache");
    check_gpu(bias, "bias");
    check_gpu(dout, "dout");
    check_gpu(db, "db");
    const int cols = last_dim(cache), rows = leading_rows(cache);
    CHECK_ERROR(global_grad->length != cache->length || dout->length != cache->length,
                "Expected global_grad, cache and dout to hold %d elements each.", cache->length);
    CHECK_ERROR(bias->length != cols || db->length != cols, "Expected the bias and db to hold %d elements.", cols);
    if (rows == 0 || cols == 0) return;
    hipStream_t s = gptc_stream_checked();
    if (cols % 4 == 0 && aligned16(global_grad->t) && aligned16(cache->t) && aligned16(bias->t) &&
        aligned16(dout->t) && aligned16(db->t)) {
        // About 1024 workgroups of 64 float4 columns x rpp rows.
        const int cblocks = (cols / 4 + kWave - 1) / kWave;
        int parts = (1024 + cblocks - 1) / cblocks;
        if (parts > rows) parts = rows;
        const int rpp = (rows + parts - 1) / parts;
        parts = (rows + rpp - 1) / rpp;
        float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * static_cast<size_t>(parts) * cols));
        gelu_bias_bwd_kernel<<<dim3(cblocks, parts), dim3(kThreads), 0, s>>>(global_grad->t, cache->t, bias->t,
                                                                             dout->t, partial, rows, cols, rpp);
        hipCheck(hipGetLastError());
        launch_add_column_partials(partial, db->t, parts, cols, s);
        free_cuda(partial);
        return;
    }
    gelu_bias_bwd_scalar_kernel<<<dim3(blocks_for(static_cast<int64_t>(rows) * cols, kThreads)), dim3(kThreads), 0,
                                  s>>>(global_grad->t, cache->t, bias->t, dout->t, rows, cols);
    hipCheck(hipGetLastError());
    launch_column_sum_add(dout->t, db->t, rows, cols, s);
}

extern "C" void softmax_forward_cuda_kernel(const tensor_t *input, tensor_t *output) {
    check_gpu(input, "input");
    check_gpu(output, "output");
    CHECK_ERROR(output->length != input->length, "Expected output to match input's %d elements.", input->length);
    const int C = last_dim(input), rows = leading_rows(input);
    if (rows == 0 || C == 0) return;
    softmax_fwd_kernel<<<dim3(rows), dim3(kThreads), 0, gptc_stream_checked()>>>(input->t, output->t, C);
    hipCheck(hipGetLastError());
}

extern "C" void softmax_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dout) {
    check_gpu(global_grad, "global_grad");
    check_gpu(cache, "cache");
    check_gpu(dout, "dout");
    CHECK_ERROR(global_grad->length != cache->length || dout->length != cache->length,
                "Expected global_grad, cache and dout to hold %d elements each.", cache->length);
    const int C = last_dim(global_grad), rows = leading_rows(global_grad);
    if (rows == 0 || C == 0) return;
    softmax_bwd_kernel<<<dim3(rows), dim3(kThreads), 0, gptc_stream_checked()>>>(global_grad->t, cache->t, dout->t, C);
    hipCheck(hipGetLastError());
}
