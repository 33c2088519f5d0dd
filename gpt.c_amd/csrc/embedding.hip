// Embedding lookup (replaces kernels/src/cuda/Embedding.cu, semantics of
// kernels/src/cpu/Embedding.c:3-47):
//   forward   out[i, :] = W[ids[i], :] with float ids truncated to int;
//   backward  dW[ids[i % L], :] += g[i, :] for every row i of g, where L is the
//             id tensor's length (L = T for the position table, whose ids
//             are one arange(T) shared by the B sequences).
// The backward is deterministic and atomic-free: the wave of row i scans the
// ids before it, and only the first row holding a given id goes on; it then
// adds, in increasing row order, the gradient rows of every row with that id
// into dW -- the order of the reference's sequential loop.
// Ids outside [0, V) are not read or written: the forward fills that output
// row with NaN (the reference reads outside W), the backward skips it.
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

__global__ __launch_bounds__(kThreads) void embedding_fwd_kernel(const float *__restrict__ W,
                                                                const float *__restrict__ ids,
                                                                float *__restrict__ out, int rows, int C, int V,
                                                                bool vec) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWaves + static_cast<int>(threadIdx.x / kWave);
    if (row >= rows) return;
    const int ix = static_cast<int>(ids[row]);
    float *o = out + static_cast<int64_t>(row) * C;
    if (ix < 0 || ix >= V) {
        for (int j = lane; j < C; j += kWave) o[j] = NAN;
        return;
    }
    const float *w = W + static_cast<int64_t>(ix) * C;
    if (vec) {
        for (int j = lane; j < C / 4; j += kWave)
            reinterpret_cast<f32x4_t *>(o)[j] = reinterpret_cast<const f32x4_t *>(w)[j];
    } else {
        for (int j = lane; j < C; j += kWave) o[j] = w[j];
    }
}

__global__ __launch_bounds__(kThreads) void embedding_bwd_kernel(const float *__restrict__ g,
                                                                const float *__restrict__ ids,
                                                                float *__restrict__ dW, int rows, int L, int C,
                                                                int V) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWaves + static_cast<int>(threadIdx.x / kWave);
    if (row >= rows) return;
    const int ix = static_cast<int>(ids[row % L]);
    if (ix < 0 || ix >= V) return;
    // Is an earlier row holding the same id?  Then that row's wave owns dW[ix].
    for (int j0 = 0; j0 < row; j0 += kWave) {
        const int j = j0 + lane;
        const bool same = j < row && static_cast<int>(ids[j % L]) == ix;
        if (__any(same)) return;
    }
    float *dw = dW + static_cast<int64_t>(ix) * C;
    for (int j0 = row; j0 < rows; j0 += kWave) {
        const int j = j0 + lane;
        uint64_t match = __ballot(j < rows && static_cast<int>(ids[j % L]) == ix);
        while (match) {
            const int bit = __builtin_ctzll(match);
            match &= match - 1;
            const float *gr = g + static_cast<int64_t>(j0 + bit) * C;
            for (int c = lane; c < C; c += kWave) dw[c] += gr[c];
        }
    }
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void embedding_forward_cuda_kernel(const tensor_t *W, const tensor_t *input, tensor_t *output) {
    check_gpu(W, "W");
    check_gpu(input, "input");
    check_gpu(output, "output");
    CHECK_ERROR(W->ndims != 2, "Expected W to be (num_embeddings, embedding_dim), but got %d dims.", W->ndims);
    const int V = W->shape[0], C = W->shape[1];
    CHECK_ERROR(last_dim(output) != C, "Expected output's last dimension to be %d, but got %d.", C, last_dim(output));
    const int rows = leading_rows(output);
    CHECK_ERROR(input->length != rows, "Expected %d ids for a (%d x %d) output, but got %d.", rows, rows, C,
                input->length);
    if (rows == 0) return;
    const bool vec = (C % 4) == 0 && aligned16(W->t) && aligned16(output->t);
    embedding_fwd_kernel<<<dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0, gptc_stream_checked()>>>(
        W->t, input->t, output->t, rows, C, V, vec);
    hipCheck(hipGetLastError());
}

extern "C" void embedding_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t *cache, tensor_t *dW) {
    check_gpu(global_grad, "global_grad");
    check_gpu(cache, "cache");
    check_gpu(dW, "dW");
    CHECK_ERROR(dW->ndims != 2, "Expected dW to be (num_embeddings, embedding_dim), but got %d dims.", dW->ndims);
    const int V = dW->shape[0], C = dW->shape[1];
    CHECK_ERROR(last_dim(global_grad) != C, "Expected global_grad's last dimension to be %d, but got %d.", C,
                last_dim(global_grad));
    const int rows = leading_rows(global_grad);
    CHECK_ERROR(cache->length < 1 && rows > 0, "Expected at least one cached id.");
    if (rows == 0) return;
    embedding_bwd_kernel<<<dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0, gptc_stream_checked()>>>(
        global_grad->t, cache->t, dW->t, rows, cache->length, C, V);
    hipCheck(hipGetLastError());
}
