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

struct RowsArgs {
    const float *W, *b, *x, *res;
    float *y;
    const float *ln_w, *ln_b;  // LayerNorm of x fused in front (ln_w set)
    float eps;
    int rows, in_f, out_f, act;
};

// The 4 waves of a workgroup own `kOuts` groups of kPer output features;
// for each group, the kSplit = 4 / kOuts waves on it take equal slices of the
// in_f inputs (so a narrow output still puts work on every CU), and the
// slices' sums meet in LDS.  acc[p][r] = W[o_p, :] . xn[r, :] for r < rows,
// where xn = x, or with kLN the LayerNorm of each x row (mean and rstd
// computed by the workgroup: the decode step's rows are at most 8 of a few
// thousand features).  kPer > 1 (wide outputs): a wave reads its normalised
// x vector once for kPer weight rows, with kPer loads in flight.
//
// A step is a chain of short kernels, so each one's time is mostly memory
// latency: everything that does not depend on the LayerNorm statistics (the
// wave's first kIt 16-byte weight vectors, the LayerNorm weights, the bias
// and residual of the output this thread finishes) is requested before
// them, and the sums keep the order of a plain loop over the inputs.
template <bool kVec, bool kLN, int kOuts, int kPer>
__global__ __launch_bounds__(kThreads) void linear_rows_kernel(const RowsArgs a) {
    constexpr int kSplit = kWaves / kOuts;
    // 16-byte steps per lane loaded up front (in_f <= 1024 kSplit).  Wide
    // outputs (kPer > 1: the vocabulary projection, bandwidth-bound) stream
    // instead: their registers buy occupancy there (34 against 40 us).
    constexpr int kIt = kPer == 1 ? 4 : 0;
    constexpr int kItN = kIt > 0 ? kIt : 1;
    __shared__ float part[kWaves * kPer][kMaxRows];
    __shared__ float stat[2][kMaxRows];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int in_f = a.in_f, rows = a.rows;
    const int grp = w / kSplit, slice = w % kSplit;
    const int o0 = (blockIdx.x * kOuts + grp) * kPer;  // this wave's first output
    const int per = (in_f + kSplit - 1) / kSplit;
    const int j0 = slice * per, j1 = min(in_f, j0 + per);

    // The bias and residual of the (output, row) this thread finishes.
    const int n_fin = kOuts * kPer * rows;
    float fin_b = 0.0f, fin_r = 0.0f;
    if (static_cast<int>(threadIdx.x) < n_fin) {
        const int oo = threadIdx.x / rows, r = threadIdx.x % rows;
        const int out = blockIdx.x * kOuts * kPer + oo;
        if (out < a.out_f) {
            if (a.b != nullptr) fin_b = a.b[out];
            if (a.res != nullptr) fin_r = a.res[static_cast<int64_t>(r) * a.out_f + out];
        }
    }
    // kVec: the wave's first kIt weight vectors per output (and LayerNorm vectors).
    const int jb = j0 / 4 + lane, je = j1 / 4;
    f32x4_t wv[kItN][kPer], lw[kItN], lb[kItN];
    if (kVec && o0 < a.out_f) {
#pragma unroll
        for (int it = 0; it < kIt; ++it) {
            const int j = jb + it * kWave;
#pragma unroll
            for (int p = 0; p < kPer; ++p)
                wv[it][p] = j < je && o0 + p < a.out_f
                                ? reinterpret_cast<const f32x4_t *>(a.W + static_cast<int64_t>(o0 + p) * in_f)[j]
                                : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            lw[it] = f32x4_t{1.0f, 1.0f, 1.0f, 1.0f};
            lb[it] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if (kLN && j < je) {
                lw[it] = reinterpret_cast<const f32x4_t *>(a.ln_w)[j];
                if (a.ln_b != nullptr) lb[it] = reinterpret_cast<const f32x4_t *>(a.ln_b)[j];
            }
        }
    }
    if (kLN) {
        // Mean and E[x^2] - mean^2 of each row, as layer_norm_forward_cuda_kernel
        // (and gpt.c's LayerNorm.c) compute them; wave r handles rows r, r+4, ...
        for (int r = w; r < rows; r += kWaves) {
            const float *xr = a.x + static_cast<int64_t>(r) * in_f;
            float s = 0.0f, ss = 0.0f;
            if (kVec) {  // 16-byte loads, all of a lane's loads issued together
                constexpr int kU = 4;
                for (int j0s = lane; j0s < in_f / 4; j0s += kU * kWave) {
                    f32x4_t v[kU];
#pragma unroll
                    for (int u = 0; u < kU; ++u) {
                        const int j = j0s + u * kWave;
                        v[u] = j < in_f / 4 ? reinterpret_cast<const f32x4_t *>(xr)[j] : f32x4_t{0, 0, 0, 0};
                    }
#pragma unroll
                    for (int u = 0; u < kU; ++u)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            s += v[u][e];
                            ss += v[u][e] * v[u][e];
                        }
                }
            } else {
                for (int j = lane; j < in_f; j += kWave) {
                    s += xr[j];
                    ss += xr[j] * xr[j];
                }
            }
            s = wave_sum(s);
            ss = wave_sum(ss);
            const float scale = 1.0f / in_f;
            const float mean = s * scale;
            const float var = ss * scale - mean * mean;
            if (lane == 0) {
                stat[0][r] = mean;
                stat[1][r] = 1.0f / sqrtf(var + a.eps);
            }
        }
        __syncthreads();
    }
    float acc[kPer][kMaxRows];
#pragma unroll
    for (int p = 0; p < kPer; ++p)
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r) acc[p][r] = 0.0f;
    if (o0 < a.out_f) {
        if (kVec) {  // in_f % (4 kSplit) == 0: slices are whole 16-byte vectors
            auto step = [&](int j, const f32x4_t(&w4)[kPer], const f32x4_t &lw4, const f32x4_t &lb4) {
#pragma unroll
                for (int r = 0; r < kMaxRows; ++r) {
                    if (r < rows) {
                        f32x4_t xv = reinterpret_cast<const f32x4_t *>(a.x + static_cast<int64_t>(r) * in_f)[j];
                        if (kLN) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) xv[e] = (xv[e] - stat[0][r]) * stat[1][r] * lw4[e] + lb4[e];
                        }
#pragma unroll
                        for (int p = 0; p < kPer; ++p) {
                            acc[p][r] = fmaf(w4[p][0], xv[0], acc[p][r]);
                            acc[p][r] = fmaf(w4[p][1], xv[1], acc[p][r]);
                            acc[p][r] = fmaf(w4[p][2], xv[2], acc[p][r]);
                            acc[p][r] = fmaf(w4[p][3], xv[3], acc[p][r]);
                        }
                    }
                }
            };
#pragma unroll
            for (int it = 0; it < kIt; ++it)
                if (jb + it * kWave < je) step(jb + it * kWave, wv[it], lw[it], lb[it]);
            // Inputs past the first kIt steps (in_f > 1024 kSplit): streamed.
            for (int j = jb + kIt * kWave; j < je; j += kWave) {
                f32x4_t w4[kPer];
#pragma unroll
                for (int p = 0; p < kPer; ++p)
                    w4[p] = o0 + p < a.out_f
                                ? reinterpret_cast<const f32x4_t *>(a.W + static_cast<int64_t>(o0 + p) * in_f)[j]
                                : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                f32x4_t lw4 = {1.0f, 1.0f, 1.0f, 1.0f}, lb4 = {0.0f, 0.0f, 0.0f, 0.0f};
                if (kLN) {
                    lw4 = reinterpret_cast<const f32x4_t *>(a.ln_w)[j];
                    if (a.ln_b != nullptr) lb4 = reinterpret_cast<const f32x4_t *>(a.ln_b)[j];
                }
                step(j, w4, lw4, lb4);
            }
        } else {
            for (int j = j0 + lane; j < j1; j += kWave) {
#pragma unroll
                for (int r = 0; r < kMaxRows; ++r) {
                    if (r < rows) {
                        float xv = a.x[static_cast<int64_t>(r) * in_f + j];
                        if (kLN)
                            xv = (xv - stat[0][r]) * stat[1][r] * a.ln_w[j] + (a.ln_b != nullptr ? a.ln_b[j] : 0.0f);
#pragma unroll
                        for (int p = 0; p < kPer; ++p)
                            if (o0 + p < a.out_f)
                                acc[p][r] = fmaf(a.W[static_cast<int64_t>(o0 + p) * in_f + j], xv, acc[p][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int p = 0; p < kPer; ++p)
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r)
            if (r < rows) {
                const float v = wave_sum(acc[p][r]);
                if (lane == 0) part[(grp * kPer + p) * kSplit + slice][r] = v;
            }
    __syncthreads();
    // One thread per (output, row) adds the slices in order and finishes.
    for (int t = threadIdx.x; t < n_fin; t += kThreads) {
        const int oo = t / rows, r = t % rows;
        const int out = blockIdx.x * kOuts * kPer + oo;
        if (out < a.out_f) {
            float v = part[oo * kSplit][r];
#pragma unroll
            for (int s = 1; s < kSplit; ++s) v += part[oo * kSplit + s][r];
            const bool first = t == static_cast<int>(threadIdx.x);
            if (a.b != nullptr) v += first ? fin_b : a.b[out];
            if (a.act == 1) v = gelu_tanh(v);
            if (a.res != nullptr) v += first ? fin_r : a.res[static_cast<int64_t>(r) * a.out_f + out];
            a.y[static_cast<int64_t>(r) * a.out_f + out] = v;
        }
    }
}

template <bool kLN, int kOuts, int kPer>
void launch_rows(const RowsArgs &a, bool vec, hipStream_t s) {
    const dim3 grid((a.out_f + kOuts * kPer - 1) / (kOuts * kPer));
    if (vec)
        linear_rows_kernel<true, kLN, kOuts, kPer><<<grid, dim3(kThreads), 0, s>>>(a);
    else
        linear_rows_kernel<false, kLN, kOuts, kPer><<<grid, dim3(kThreads), 0, s>>>(a);
    hipCheck(hipGetLastError());
}

// Narrow outputs (under 1024 features) split each dot product over the 4
// waves of a workgroup; medium ones (under 4096) give each wave a feature of
// its own, wide ones 4 features.
void run_rows(const RowsArgs &a, hipStream_t s) {
    const int kind = a.out_f < 1024 ? 0 : a.out_f < 4096 ? 1 : 2;
    const int split = kind == 0 ? 4 : 1;
    const bool vec = (a.in_f % (4 * split)) == 0 && aligned16(a.W) && aligned16(a.x) &&
                     (a.ln_w == nullptr || (aligned16(a.ln_w) && aligned16(a.ln_b)));
    if (a.ln_w != nullptr) {
        if (kind == 0) launch_rows<true, 1, 1>(a, vec, s);
        else if (kind == 1) launch_rows<true, 4, 1>(a, vec, s);
        else launch_rows<true, 4, 4>(a, vec, s);
    } else {
        if (kind == 0) launch_rows<false, 1, 1>(a, vec, s);
        else if (kind == 1) launch_rows<false, 4, 1>(a, vec, s);
        else launch_rows<false, 4, 4>(a, vec, s);
    }
}

// out[r, :] = wte[id, :] + wpe[pos, :] with id = ids[r * ids_stride + pos]
// (pos_dev set: the position is *pos_dev) or ids[r] (host position); an id
// outside [0, V) gives NaN.
__global__ __launch_bounds__(kThreads) void embed_token_kernel(const float *__restrict__ wte,
                                                              const float *__restrict__ wpe,
                                                              const float *__restrict__ ids, float *__restrict__ out,
                                                              int C, int V, int pos, const int *pos_dev,
                                                              int ids_stride, int P) {
    const int r = blockIdx.x;
    if (pos_dev != nullptr) {
        pos = *pos_dev;
        if (pos < 0 || pos >= P) return;  // P: rows of the position table and of the id buffer
    }
    const int ix = static_cast<int>(ids[pos_dev != nullptr ? static_cast<int64_t>(r) * ids_stride + pos : r]);
    const bool ok = ix >= 0 && ix < V;
    for (int j = threadIdx.x; j < C; j += kThreads)
        out[static_cast<int64_t>(r) * C + j] =
            ok ? wte[static_cast<int64_t>(ix) * C + j] + wpe[static_cast<int64_t>(pos) * C + j] : NAN;
}

constexpr int kArgThreads = 1024;
constexpr int kArgWaves = kArgThreads / kWave;
constexpr int kArgU = 16;  // elements per thread per round, loads issued together

// ids[r] = the first index of the largest value of logits row r (NaN never wins).
// 1024 threads; each takes kArgU strided elements per round with all their
// loads issued together, so a 50257-wide row is 4 memory round trips.
// With pos_dev set, the token goes to ids[r * stride + *pos_dev + 1], and only
// once the prompt (positions < prompt) has been consumed and while it is
// below total.
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float *__restrict__ logits,
                                                            float *__restrict__ ids, int V, const int *pos_dev,
                                                            int stride, int prompt, int total) {
    __shared__ float sv[kArgWaves];
    __shared__ int si[kArgWaves];
    const float *row = logits + static_cast<int64_t>(blockIdx.x) * V;
    float best = -INFINITY;
    int bi = V;  // none yet
    for (int j0 = threadIdx.x; j0 < V; j0 += kArgU * kArgThreads) {
        float v[kArgU];
#pragma unroll
        for (int u = 0; u < kArgU; ++u) {
            const int j = j0 + u * kArgThreads;
            v[u] = j < V ? row[j] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < kArgU; ++u)
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
        const float tok = static_cast<float>(bi < V ? bi : 0);
        if (pos_dev == nullptr) {
            ids[blockIdx.x] = tok;
        } else {
            const int nxt = *pos_dev + 1;
            if (nxt >= prompt && nxt < total) ids[static_cast<int64_t>(blockIdx.x) * stride + nxt] = tok;
        }
    }
}

// The step's last node: the next position.
__global__ void advance_pos_kernel(int *pos_dev) {
    if (threadIdx.x == 0) *pos_dev += 1;
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void gptc_linear_rows_cuda(const tensor_t *W, const tensor_t *b, const tensor_t *x,
                                      const tensor_t *residual, const int act, tensor_t *y) {
    gptc::ln_linear_rows(nullptr, nullptr, 0.0f, W, b, x, residual, act, y);
}

void gptc::ln_linear_rows(const tensor_t *ln_w, const tensor_t *ln_b, float eps, const tensor_t *W, const tensor_t *b,
                          const tensor_t *x, const tensor_t *residual, int act, tensor_t *y) {
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
    if (ln_w != nullptr) {
        check_gpu(ln_w, "ln_w");
        CHECK_ERROR(ln_w->length != in_f || (ln_b != nullptr && ln_b->length != in_f),
                    "Expected the LayerNorm parameters to hold %d elements.", in_f);
    }
    RowsArgs a;
    a.W = W->t;
    a.b = b != NULL ? b->t : nullptr;
    a.x = x->t;
    a.res = residual != NULL ? residual->t : nullptr;
    a.y = y->t;
    a.ln_w = ln_w != nullptr ? ln_w->t : nullptr;
    a.ln_b = ln_w != nullptr && ln_b != nullptr ? ln_b->t : nullptr;
    a.eps = eps;
    a.rows = rows;
    a.in_f = in_f;
    a.out_f = out_f;
    a.act = act;
    run_rows(a, gptc_stream_checked());
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
    embed_token_kernel<<<dim3(ids->length), dim3(kThreads), 0, gptc_stream_checked()>>>(
        wte->t, wpe->t, ids->t, out->t, C, V, pos, nullptr, 1, wpe->shape[0]);
    hipCheck(hipGetLastError());
}

extern "C" void gptc_argmax_cuda(const tensor_t *logits, tensor_t *ids) {
    check_gpu(logits, "logits");
    check_gpu(ids, "ids");
    const int V = last_dim(logits), rows = leading_rows(logits);
    CHECK_ERROR(ids->length != rows, "Expected %d ids, but got %d.", rows, ids->length);
    if (rows == 0) return;
    argmax_kernel<<<dim3(rows), dim3(kArgThreads), 0, gptc_stream_checked()>>>(logits->t, ids->t, V, nullptr, 1, 0,
                                                                                 0);
    hipCheck(hipGetLastError());
}

// ---- the device-position forms used by the captured generation step ----

void gptc::launch_embed_tokens_devpos(const tensor_t *wte, const tensor_t *wpe, const float *tokens, int B,
                                      int stride, const int *pos_dev, tensor_t *out) {
    const int V = wte->shape[0], C = wte->shape[1];
    const int limit = stride < wpe->shape[0] ? stride : wpe->shape[0];
    embed_token_kernel<<<dim3(B), dim3(kThreads), 0, gptc_stream_checked()>>>(wte->t, wpe->t, tokens, out->t, C, V,
                                                                              0, pos_dev, stride, limit);
    hipCheck(hipGetLastError());
}

void gptc::launch_argmax_next(const tensor_t *logits, float *tokens, int stride, const int *pos_dev, int prompt,
                              int total) {
    const int V = last_dim(logits), rows = leading_rows(logits);
    argmax_kernel<<<dim3(rows), dim3(kArgThreads), 0, gptc_stream_checked()>>>(logits->t, tokens, V, pos_dev, stride,
                                                                                 prompt, total);
    hipCheck(hipGetLastError());
}

void gptc::launch_advance_pos(int *pos_dev) {
    advance_pos_kernel<<<dim3(1), dim3(64), 0, gptc_stream_checked()>>>(pos_dev);
    hipCheck(hipGetLastError());
}
