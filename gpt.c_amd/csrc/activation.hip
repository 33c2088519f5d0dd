// GELU (tanh form) and row softmax (replaces kernels/src/cuda/GeLU.cu and
// Softmax.cu, semantics of kernels/src/cpu/GeLU.c:7-42 and
// kernels/src/cpu/Softmax.c:7-63).
//   gelu fwd   y = 0.5 x (1 + tanh(k (x + 0.044715 x^3))), k = sqrt(2/pi)
//   gelu bwd   dout = g * d/dx gelu(x), written (not accumulated)
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
