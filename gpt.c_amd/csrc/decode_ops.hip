// Kernels of the one-token model step (KV-cache generation), where every
// activation is a handful of rows and every weight is read once per token:
//   gptc_linear_rows_cuda   y = act(x W^T + b) (+ r) for few rows of x: a wave
//                           per output feature reads its weight row once
//                           (16-byte loads) and dots it with each of the rows;
//                           GELU (the tanh form of GeLU.c) and a residual add
//                           are applied in the same pass;
//   gptc_embed_token_cuda   wte[id] + wpe[pos] for each sequence;
//   gptc_argmax_cuda        greedy token of each logits row (first maximum).
// No counterpart in gpt.c, whose infer_gpt.c recomputes the whole window
// through the training kernels for every token.
#include <cmath>
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxRows = 8;
constexpr float kGeluBeta = static_cast<float>(M_SQRT2 * M_2_SQRTPI * 0.5);

__device__ __forceinline__ float gelu_tanh(float x) {
    const float cube = 0.044715f * x * x * x;
    return 0.5f * x * (1.0f + tanhf(kGeluBeta * (x + cube)));
}

// One wave per output feature o: acc[r] = W[o, :] . x[r, :] for r < rows.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void linear_rows_kernel(const float *__restrict__ W,
                                                              const float *__restrict__ b,
                                                              const float *__restrict__ x,
                                                              const float *__restrict__ res, float *__restrict__ y,
                                                              int rows, int in_f, int out_f, int act) {
    const int lane = threadIdx.x & (kWave - 1);
    const int o = blockIdx.x * kWaves + static_cast<int>(threadIdx.x / kWave);
    if (o >= out_f) return;
    const float *w = W + static_cast<int64_t>(o) * in_f;
    float acc[kMaxRows];
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r) acc[r] = 0.0f;
    if (kVec) {
        const int n4 = in_f / 4;
        for (int j = lane; j < n4; j += kWave) {
            const f32x4_t wv = reinterpret_cast<const f32x4_t *>(w)[j];
#pragma unroll
            for (int r = 0; r < kMaxRows; ++r) {
                if (r < rows) {
                    const f32x4_t xv = reinterpret_cast<const f32x4_t *>(x + static_cast<int64_t>(r) * in_f)[j];
                    acc[r] = fmaf(wv[0], xv[0], acc[r]);
                    acc[r] = fmaf(wv[1], xv[1], acc[r]);
                    acc[r] = fmaf(wv[2], xv[2], acc[r]);
                    acc[r] = fmaf(wv[3], xv[3], acc[r]);
                }
            }
        }
    } else {
        for (int j = lane; j < in_f; j += kWave) {
            const float wv = w[j];
#pragma unroll
            for (int r = 0; r < kMaxRows; ++r)
                if (r < rows) acc[r] = fmaf(wv, x[static_cast<int64_t>(r) * in_f + j], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r) {
        if (r < rows) {
            float v = wave_sum(acc[r]);
            if (lane == 0) {
                if (b != nullptr) v += b[o];
                if (act == 1) v = gelu_tanh(v);
                if (res != nullptr) v += res[static_cast<int64_t>(r) * out_f + o];
                y[static_cast<int64_t>(r) * out_f + o] = v;
            }
        }
    }
}

// out[r, :] = wte[ids[r], :] + wpe[pos, :]; an id outside [0, V) gives NaN.
__global__ __launch_bounds__(kThreads) void embed_token_kernel(const float *__restrict__ wte,
                                                              const float *__restrict__ wpe,
                                                              const float *__restrict__ ids, float *__restrict__ out,
                                                              int C, int V, int pos) {
    const int r = blockIdx.x;
    const int ix = static_cast<int>(ids[r]);
    const bool ok = ix >= 0 && ix < V;
    for (int j = threadIdx.x; j < C; j += kThreads)
        out[static_cast<int64_t>(r) * C + j] =
            ok ? wte[static_cast<int64_t>(ix) * C + j] + wpe[static_cast<int64_t>(pos) * C + j] : NAN;
}

constexpr int kArgThreads = 1024;
constexpr int kArgWaves = kArgThreads / kWave;

// ids[r] = the first index of the largest value of logits row r (NaN never wins).
// 1024 threads; each takes 4 strided elements per round with the 4 loads
// issued together, so a 50257-wide row is about 13 memory round trips.
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float *__restrict__ logits,
                                                            float *__restrict__ ids, int V) {
    __shared__ float sv[kArgWaves];
    __shared__ int si[kArgWaves];
    const float *row = logits + static_cast<int64_t>(blockIdx.x) * V;
    float best = -INFINITY;
    int bi = V;  // none yet
    for (int j0 = threadIdx.x; j0 < V; j0 += 4 * kArgThreads) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + u * kArgThreads;
            v[u] = j < V ? row[j] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (v[u] > best) {  // strictly greater, indices rising: keeps the first index per thread
                best = v[u];
                bi = j0 + u * kArgThreads;
            }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < kArgWaves; ++i)
            if (sv[i] > best || (sv[i] == best && si[i] < bi)) {
                best = sv[i];
                bi = si[i];
            }
        ids[blockIdx.x] = static_cast<float>(bi < V ? bi : 0);
    }
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void gptc_linear_rows_cuda(const tensor_t *W, const tensor_t *b, const tensor_t *x,
                                      const tensor_t *residual, const int act, tensor_t *y) {
    check_gpu(W, "W");
    check_gpu(x, "x");
    check_gpu(y, "y");
    CHECK_ERROR(W->ndims != 2, "Expected W to be (out_features, in_features), but got %d dims.", W->ndims);
    const int out_f = W->shape[0], in_f = W->shape[1];
    CHECK_ERROR(last_dim(x) != in_f, "Expected x's last dimension to be %d, but got %d.", in_f, last_dim(x));
    const int rows = leading_rows(x);
    CHECK_ERROR(rows < 1 || rows > kMaxRows, "gptc_linear_rows_cuda takes 1 .. %d rows, but got %d.", kMaxRows, rows);
    CHECK_ERROR(y->length != rows * out_f, "Expected y to hold %d x %d elements.", rows, out_f);
    CHECK_ERROR(act != 0 && act != 1, "act must be 0 (none) or 1 (GELU), got %d.", act);
    if (b != NULL) {
        check_gpu(b, "b");
        CHECK_ERROR(b->length != out_f, "Expected b to hold %d elements.", out_f);
    }
    if (residual != NULL) {
        check_gpu(residual, "residual");
        CHECK_ERROR(residual->length != y->length, "Expected the residual to match y's %d elements.", y->length);
    }
    const bool vec = (in_f % 4) == 0 && aligned16(W->t) && aligned16(x->t);
    const dim3 grid((out_f + kWaves - 1) / kWaves);
    hipStream_t s = gptc_stream_checked();
    const float *bp = b != NULL ? b->t : nullptr;
    const float *rp = residual != NULL ? residual->t : nullptr;
    if (vec)
        linear_rows_kernel<true><<<grid, dim3(kThreads), 0, s>>>(W->t, bp, x->t, rp, y->t, rows, in_f, out_f, act);
    else
        linear_rows_kernel<false><<<grid, dim3(kThreads), 0, s>>>(W->t, bp, x->t, rp, y->t, rows, in_f, out_f, act);
    hipCheck(hipGetLastError());
}

extern "C" void gptc_embed_token_cuda(const tensor_t *wte, const tensor_t *wpe, const tensor_t *ids, const int pos,
                                      tensor_t *out) {
    check_gpu(wte, "wte");
    check_gpu(wpe, "wpe");
    check_gpu(ids, "ids");
    check_gpu(out, "out");
    const int V = wte->shape[0], C = wte->shape[1];
    CHECK_ERROR(wpe->shape[1] != C, "Expected wte and wpe to share their width.");
    CHECK_ERROR(pos < 0 || pos >= wpe->shape[0], "Expected 0 <= pos < %d, but got pos = %d.", wpe->shape[0], pos);
    CHECK_ERROR(out->length != ids->length * C, "Expected out to hold %d x %d elements.", ids->length, C);
    if (ids->length == 0) return;
    embed_token_kernel<<<dim3(ids->length), dim3(kThreads), 0, gptc_stream_checked()>>>(wte->t, wpe->t, ids->t,
                                                                                        out->t, C, V, pos);
    hipCheck(hipGetLastError());
}

extern "C" void gptc_argmax_cuda(const tensor_t *logits, tensor_t *ids) {
    check_gpu(logits, "logits");
    check_gpu(ids, "ids");
    const int V = last_dim(logits), rows = leading_rows(logits);
    CHECK_ERROR(ids->length != rows, "Expected %d ids, but got %d.", rows, ids->length);
    if (rows == 0) return;
    argmax_kernel<<<dim3(rows), dim3(kArgThreads), 0, gptc_stream_checked()>>>(logits->t, ids->t, V);
    hipCheck(hipGetLastError());
}
