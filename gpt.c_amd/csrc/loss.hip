// Cross-entropy loss over (B, T, V) logits and (B, T) float targets
// (replaces kernels/src/cuda/CrossEntropyLoss.cu, semantics of
// kernels/src/cpu/CrossEntropyLoss.c:7-97):
//   forward   cache[0] = log_softmax(logits) per row; output[0] = mean over
//             rows of -log_softmax[target];
//   backward  with s = -g / (B T):  dout[j] = [j == target] s - exp(lsm[j]) s.
// Forward: a row is one workgroup.  Rows of up to 65536 logits (16-byte
// aligned buffers) are held in the registers of a 512-thread workgroup: one
// read of the logits, then the max, the sum and the log-softmax from
// registers.  Longer rows take one online (max, sum) pass over the logits,
// then a pass that writes the log-softmax (float4 accesses and exp2 where
// aligned).  The per-row losses go to a buffer and one workgroup adds them
// in a fixed order, so the mean is deterministic.  Backward: elementwise,
// several workgroups per row.  A target outside [0, V) makes that row's loss
// NaN (the reference would read outside the row) and its gradient row is the
// softmax part only.
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

// The same two kernels on float4 vectors, for 16-byte aligned buffers.  Row r
// starts at element r V; its first `head` elements (up to the next 16-byte
// boundary) and its last V - head - 4 n4 are handled one per thread, the rest
// as float4.  The exponentials are exp2 of log2(e)-scaled values
// (v_exp_f32), and the running (max, sum) is kept in log2 units.
constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kLn2F = 0.6931471805599453f;

__device__ __forceinline__ void online_merge2(float &m, float &s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;  // both empty
    s = s * __builtin_amdgcn_exp2f(m - mn) + s2 * __builtin_amdgcn_exp2f(m2 - mn);
    m = mn;
}

__device__ __forceinline__ void row_split(int64_t base, int V, int &head, int &n4) {
    head = static_cast<int>((4 - (base & 3)) & 3);
    if (head > V) head = V;
    n4 = (V - head) / 4;
}

// Index of the single element this thread handles at the row's unaligned
// ends (threads 0..2: the head, 3..5: the tail), or -1.
__device__ __forceinline__ int row_end_index(int head, int tail, int V) {
    const int t = threadIdx.x;
    if (t < head) return t;
    if (t >= 3 && t < 6 && tail + (t - 3) < V) return tail + (t - 3);
    return -1;
}

__global__ __launch_bounds__(kThreads) void ce_fwd4_kernel(const float *__restrict__ logits,
                                                          const float *__restrict__ targets, float *__restrict__ lsm,
                                                          float *__restrict__ row_loss, int V) {
    __shared__ float sm[kWaves], ss[kWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * V;
    const float *xr = logits + base;
    int head, n4;
    row_split(base, V, head, n4);
    const int je = row_end_index(head, head + 4 * n4, V);
    const f32x4_t *x4 = reinterpret_cast<const f32x4_t *>(xr + head);
    float m = -INFINITY, s = 0.0f;
    for (int i = threadIdx.x; i < n4; i += kThreads) {
        const f32x4_t v = x4[i] * kLog2eF;
        const float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if (mx > m) {
            s *= __builtin_amdgcn_exp2f(m - mx);
            m = mx;
        }
        if (m != -INFINITY)
            s += (__builtin_amdgcn_exp2f(v[0] - m) + __builtin_amdgcn_exp2f(v[1] - m)) +
                 (__builtin_amdgcn_exp2f(v[2] - m) + __builtin_amdgcn_exp2f(v[3] - m));
    }
    if (je >= 0) {
        const float v = xr[je] * kLog2eF;
        if (v > m) {
            s = s * __builtin_amdgcn_exp2f(m - v) + 1.0f;
            m = v;
        } else if (v != -INFINITY) {
            s += __builtin_amdgcn_exp2f(v - m);
        }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
        online_merge2(m, s, m2, s2);
    }
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sm[w] = m;
        ss[w] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) online_merge2(m, s, sm[i], ss[i]);
    const float shift = (m + log2f(s)) * kLn2F;  // log of the row's sum of exp
    float *lr = lsm + base;
    f32x4_t *l4 = reinterpret_cast<f32x4_t *>(lr + head);
    for (int i = threadIdx.x; i < n4; i += kThreads) l4[i] = x4[i] - shift;
    if (je >= 0) lr[je] = xr[je] - shift;
    if (threadIdx.x == 0) {
        const int t = static_cast<int>(targets[blockIdx.x]);
        row_loss[blockIdx.x] = (t >= 0 && t < V) ? -(xr[t] - shift) : NAN;
    }
}

__global__ __launch_bounds__(kThreads) void ce_bwd4_kernel(const float *__restrict__ g, const float *__restrict__ lsm,
                                                          const float *__restrict__ targets, float *__restrict__ dout,
                                                          int V, float rows_f) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * V;
    const float s = -g[blockIdx.x] / rows_f;
    const int t = static_cast<int>(targets[blockIdx.x]);
    int head, n4;
    row_split(base, V, head, n4);
    const int je = row_end_index(head, head + 4 * n4, V);
    const float *lr = lsm + base;
    float *dr = dout + base;
    const f32x4_t *l4 = reinterpret_cast<const f32x4_t *>(lr + head);
    f32x4_t *d4 = reinterpret_cast<f32x4_t *>(dr + head);
    for (int i = threadIdx.x; i < n4; i += kThreads) {
        const f32x4_t l = l4[i] * kLog2eF;
        f32x4_t d;
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = (head + 4 * i + c == t ? s : 0.0f) - __builtin_amdgcn_exp2f(l[c]) * s;
        d4[i] = d;
    }
    if (je >= 0) dr[je] = (je == t ? s : 0.0f) - __builtin_amdgcn_exp2f(lr[je] * kLog2eF) * s;
}

// Row-resident forward for rows of at most 512 NPT float4 (GPT-2's
// V = 50257 takes NPT = 25): a 512-thread workgroup issues every load of its
// row before the first use and keeps the row in registers, so the logits are
// read once (max, then the sum of exponentials, then the output, all from
// registers; 8 V bytes per row instead of 12 V).
constexpr int kRowThreads = 512;
constexpr int kRowWaves = kRowThreads / kWave;

// Block-wide max / sum of one value per thread (sum in wave order, fixed).
__device__ __forceinline__ float row_max(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; ++i) r = fmaxf(r, red[i]);
    __syncthreads();  // red is reused by the next reduction
    return r;
}
__device__ __forceinline__ float row_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kRowWaves; ++i) r += red[i];
    return r;
}

template <int NPT>
__global__ __launch_bounds__(kRowThreads) void ce_fwd_row_kernel(const float *__restrict__ logits,
                                                                const float *__restrict__ targets,
                                                                float *__restrict__ lsm, float *__restrict__ row_loss,
                                                                int V) {
    __shared__ float red[kRowWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * V;
    const float *xr = logits + base;
    int head, n4;
    row_split(base, V, head, n4);
    const int je = row_end_index(head, head + 4 * n4, V);
    const f32x4_t *x4 = reinterpret_cast<const f32x4_t *>(xr + head);
    const f32x4_t ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    f32x4_t v[NPT];
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const int i = threadIdx.x + k * kRowThreads;
        v[k] = i < n4 ? x4[i] : ninf;
    }
    const float ve = je >= 0 ? xr[je] : -INFINITY;
    float mx = ve;
#pragma unroll
    for (int k = 0; k < NPT; ++k) mx = fmaxf(mx, fmaxf(fmaxf(v[k][0], v[k][1]), fmaxf(v[k][2], v[k][3])));
    const float M = row_max(mx, red);
    // exp(x - M) = exp2(x log2(e) - M log2(e)); a row of -inf only sums to 0.
    const float ml2 = M == -INFINITY ? 0.0f : M * kLog2eF;
    float s = __builtin_amdgcn_exp2f(fmaf(ve, kLog2eF, -ml2));
#pragma unroll
    for (int k = 0; k < NPT; ++k)
        s += (__builtin_amdgcn_exp2f(fmaf(v[k][0], kLog2eF, -ml2)) + __builtin_amdgcn_exp2f(fmaf(v[k][1], kLog2eF, -ml2))) +
             (__builtin_amdgcn_exp2f(fmaf(v[k][2], kLog2eF, -ml2)) + __builtin_amdgcn_exp2f(fmaf(v[k][3], kLog2eF, -ml2)));
    const float S = row_sum(s, red);
    const float shift = M + logf(S);  // log of the row's sum of exp
    float *lr = lsm + base;
    f32x4_t *l4 = reinterpret_cast<f32x4_t *>(lr + head);
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const int i = threadIdx.x + k * kRowThreads;
        if (i < n4) l4[i] = v[k] - shift;
    }
    if (je >= 0) lr[je] = ve - shift;
    if (threadIdx.x == 0) {
        const int t = static_cast<int>(targets[blockIdx.x]);
        row_loss[blockIdx.x] = (t >= 0 && t < V) ? -(xr[t] - shift) : NAN;
    }
}

// The backward is elementwise once a row's scale s is known: a row is cut
// into chunks of kBwdChunk float4 (4 per thread, their loads issued
// together), one workgroup per (chunk, row); chunk 0 also takes the row's
// unaligned ends.
constexpr int kBwdVecs = 4;
constexpr int kBwdChunk = kThreads * kBwdVecs;

__global__ __launch_bounds__(kThreads) void ce_bwd_chunk_kernel(const float *__restrict__ g,
                                                               const float *__restrict__ lsm,
                                                               const float *__restrict__ targets,
                                                               float *__restrict__ dout, int V, float rows_f) {
    const int row = blockIdx.y;
    const int64_t base = static_cast<int64_t>(row) * V;
    const float s = -g[row] / rows_f;
    const int t = static_cast<int>(targets[row]);
    int head, n4;
    row_split(base, V, head, n4);
    const float *lr = lsm + base;
    float *dr = dout + base;
    const f32x4_t *l4 = reinterpret_cast<const f32x4_t *>(lr + head);
    f32x4_t *d4 = reinterpret_cast<f32x4_t *>(dr + head);
    const int i0 = blockIdx.x * kBwdChunk + threadIdx.x;
    f32x4_t l[kBwdVecs];
#pragma unroll
    for (int k = 0; k < kBwdVecs; ++k) {
        const int i = i0 + k * kThreads;
        l[k] = i < n4 ? l4[i] : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int k = 0; k < kBwdVecs; ++k) {
        const int i = i0 + k * kThreads;
        if (i < n4) {
            f32x4_t d;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                d[c] = (head + 4 * i + c == t ? s : 0.0f) - __builtin_amdgcn_exp2f(l[k][c] * kLog2eF) * s;
            d4[i] = d;
        }
    }
    if (blockIdx.x == 0) {
        const int je = row_end_index(head, head + 4 * n4, V);
        if (je >= 0) dr[je] = (je == t ? s : 0.0f) - __builtin_amdgcn_exp2f(lr[je] * kLog2eF) * s;
    }
}

// NPT for a row of n4 float4 (0: too long, use the streaming kernels).
int row_npt(int V) {
    const int n4 = V / 4;
    if (n4 <= 8 * kRowThreads) return 8;
    if (n4 <= 25 * kRowThreads) return 25;
    if (n4 <= 32 * kRowThreads) return 32;
    return 0;
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void cross_entropy_forward_cuda_kernel(const tensor_t *logits, const tensor_t *targets, tensor_t **cache,
                                                  tensor_t *output) {
    check_gpu(logits, "logits");
    check_gpu(targets, "targets");
    check_gpu(output, "output");
    REQUIRE_ARG(cache);
    check_gpu(cache[0], "cache[0] (log-softmax)");
    const int V = last_dim(logits), rows = leading_rows(logits);
    CHECK_ERROR(targets->length != rows, "Expected %d targets, but got %d.", rows, targets->length);
    CHECK_ERROR(cache[0]->length != logits->length, "Expected cache[0] to match the logits' %d elements.",
                logits->length);
    CHECK_ERROR(output->length < 1, "Expected output to hold the loss.");
    CHECK_ERROR(rows < 1 || V < 1, "Expected at least one row of logits.");
    hipStream_t s = gptc_stream_checked();
    float *row_loss = static_cast<float *>(alloc_cuda(sizeof(float) * rows));
    const int npt = row_npt(V);
    if (aligned16(logits->t) && aligned16(cache[0]->t) && npt > 0) {
        auto k = npt == 8 ? ce_fwd_row_kernel<8> : npt == 25 ? ce_fwd_row_kernel<25> : ce_fwd_row_kernel<32>;
        k<<<dim3(rows), dim3(kRowThreads), 0, s>>>(logits->t, targets->t, cache[0]->t, row_loss, V);
    } else if (aligned16(logits->t) && aligned16(cache[0]->t))
        ce_fwd4_kernel<<<dim3(rows), dim3(kThreads), 0, s>>>(logits->t, targets->t, cache[0]->t, row_loss, V);
    else
        ce_fwd_kernel<<<dim3(rows), dim3(kThreads), 0, s>>>(logits->t, targets->t, cache[0]->t, row_loss, V);
    hipCheck(hipGetLastError());
    ce_mean_kernel<<<dim3(1), dim3(kThreads), 0, s>>>(row_loss, output->t, rows);
    hipCheck(hipGetLastError());
    free_cuda(row_loss);
}

extern "C" void cross_entropy_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t **cache,
                                                   tensor_t *dout) {
    check_gpu(global_grad, "global_grad");
    REQUIRE_ARG(cache);
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
    if (aligned16(lsm->t) && aligned16(dout->t) && rows <= 65535) {
        const dim3 grid(V / 4 >= 1 ? (V / 4 + kBwdChunk - 1) / kBwdChunk : 1, rows);  // chunk 0 also takes the ends
        ce_bwd_chunk_kernel<<<grid, dim3(kThreads), 0, gptc_stream_checked()>>>(global_grad->t, lsm->t, cache[1]->t,
                                                                                dout->t, V, static_cast<float>(rows));
    } else if (aligned16(lsm->t) && aligned16(dout->t))
        ce_bwd4_kernel<<<dim3(rows), dim3(kThreads), 0, gptc_stream_checked()>>>(
            global_grad->t, lsm->t, cache[1]->t, dout->t, V, static_cast<float>(rows));
    else
        ce_bwd_kernel<<<dim3(rows), dim3(kThreads), 0, gptc_stream_checked()>>>(
            global_grad->t, lsm->t, cache[1]->t, dout->t, V, static_cast<float>(rows));
    hipCheck(hipGetLastError());
}
