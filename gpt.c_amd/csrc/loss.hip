// Cross-entropy loss over (B, T, V) logits and (B, T) float targets
// (replaces kernels/src/cuda/CrossEntropyLoss.cu, semantics of
// kernels/src/cpu/CrossEntropyLoss.c:7-97):
//   forward   cache[0] = log_softmax(logits) per row; output[0] = mean over
//             rows of -log_softmax[target];
//   backward  with s = -g / (B T):  dout[j] = [j == target] s - exp(lsm[j]) s.
// A row is one 256-thread workgroup: one online (max, sum) pass over the
// logits, then a pass that writes the log-softmax.  The per-row losses go to
// a buffer and one workgroup adds them in a fixed order, so the mean is
// deterministic.  A target outside [0, V) makes that row's loss NaN (the
// reference would read outside the row) and its gradient row is the softmax
// part only.
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

__global__ __launch_bounds__(kThreads) void ce_fwd_kernel(const float *__restrict__ logits,
                                                         const float *__restrict__ targets, float *__restrict__ lsm,
                                                         float *__restrict__ row_loss, int V) {
    __shared__ float sm[kWaves], ss[kWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * V;
    const float *xr = logits + base;
    float m = -INFINITY, s = 0.0f;
    for (int j = threadIdx.x; j < V; j += kThreads) {
        const float v = xr[j];
        if (v > m) {
            s = s * expf(m - v) + 1.0f;
            m = v;
        } else if (v != -INFINITY) {
            s += expf(v - m);
        }
    }
    wave_online(m, s);
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sm[w] = m;
        ss[w] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) online_merge(m, s, sm[i], ss[i]);
    const float logsum = logf(s);
    float *lr = lsm + base;
    for (int j = threadIdx.x; j < V; j += kThreads) lr[j] = xr[j] - m - logsum;
    if (threadIdx.x == 0) {
        const int t = static_cast<int>(targets[blockIdx.x]);
        row_loss[blockIdx.x] = (t >= 0 && t < V) ? -(xr[t] - m - logsum) : NAN;
    }
}

// output[0] = (sum of row_loss, fixed order) / rows.
__global__ __launch_bounds__(kThreads) void ce_mean_kernel(const float *__restrict__ row_loss, float *__restrict__ out,
                                                          int rows) {
    __shared__ float part[kThreads];
    // Thread i adds rows i, i + 256, ...; then thread 0 adds the 256 partials.
    float t = 0.0f;
    for (int r = threadIdx.x; r < rows; r += kThreads) t += row_loss[r];
    part[threadIdx.x] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
        float acc = 0.0f;
        for (int i = 0; i < kThreads; ++i) acc += part[i];
        out[0] = acc / rows;
    }
}

__global__ __launch_bounds__(kThreads) void ce_bwd_kernel(const float *__restrict__ g, const float *__restrict__ lsm,
                                                         const float *__restrict__ targets, float *__restrict__ dout,
                                                         int V, float rows_f) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * V;
    const float s = -g[blockIdx.x] / rows_f;
    const int t = static_cast<int>(targets[blockIdx.x]);
    for (int j = threadIdx.x; j < V; j += kThreads) {
        const float d = j == t ? s : 0.0f;
        dout[base + j] = d - expf(lsm[base + j]) * s;
    }
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void cross_entropy_forward_cuda_kernel(const tensor_t *logits, const tensor_t *targets, tensor_t **cache,
                                                  tensor_t *output) {
    check_gpu(logits, "logits");
    check_gpu(targets, "targets");
    check_gpu(output, "output");
    CHECK_ERROR(cache == NULL, "Expected **cache to be a tensor_t pointer, but got NULL.");
    check_gpu(cache[0], "cache[0] (log-softmax)");
    const int V = last_dim(logits), rows = leading_rows(logits);
    CHECK_ERROR(targets->length != rows, "Expected %d targets, but got %d.", rows, targets->length);
    CHECK_ERROR(cache[0]->length != logits->length, "Expected cache[0] to match the logits' %d elements.",
                logits->length);
    CHECK_ERROR(output->length < 1, "Expected output to hold the loss.");
    CHECK_ERROR(rows < 1 || V < 1, "Expected at least one row of logits.");
    hipStream_t s = gptc_stream_checked();
    float *row_loss = static_cast<float *>(alloc_cuda(sizeof(float) * rows));
    ce_fwd_kernel<<<dim3(rows), dim3(kThreads), 0, s>>>(logits->t, targets->t, cache[0]->t, row_loss, V);
    hipCheck(hipGetLastError());
    ce_mean_kernel<<<dim3(1), dim3(kThreads), 0, s>>>(row_loss, output->t, rows);
    hipCheck(hipGetLastError());
    free_cuda(row_loss);
}

extern "C" void cross_entropy_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t **cache,
                                                   tensor_t *dout) {
    check_gpu(global_grad, "global_grad");
    CHECK_ERROR(cache == NULL, "Expected **cache to be a tensor_t pointer, but got NULL.");
    check_gpu(cache[0], "cache[0] (log-softmax)");
    check_gpu(cache[1], "cache[1] (targets)");
    check_gpu(dout, "dout");
    const tensor_t *lsm = cache[0];
    const int V = last_dim(lsm), rows = leading_rows(lsm);
    CHECK_ERROR(cache[1]->length != rows || global_grad->length != rows,
                "Expected %d targets and %d upstream gradients.", rows, rows);
    CHECK_ERROR(dout->length != lsm->length, "Expected dout to match the logits' %d elements.", lsm->length);
    if (rows == 0) return;
    // The reference divides by the int B*T (cpu/CrossEntropyLoss.c:67-72).
    ce_bwd_kernel<<<dim3(rows), dim3(kThreads), 0, gptc_stream_checked()>>>(
        global_grad->t, lsm->t, cache[1]->t, dout->t, V, static_cast<float>(rows));
    hipCheck(hipGetLastError());
}
