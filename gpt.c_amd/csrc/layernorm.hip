// LayerNorm over the last dimension (replaces kernels/src/cuda/LayerNorm.cu,
// semantics of kernels/src/cpu/LayerNorm.c:5-124):
//   forward   mean, var = E[x^2] - mean^2, rstd = 1/sqrt(var + eps),
//             y = (x - mean) * rstd * W + b; mean and rstd go to cache[0..1];
//   backward  dout += a g W + b' x + c' (per-row a = rstd and the two row sums
//             of g x W and g W), dW += sum_rows g (a x - a mean), db += sum_rows g.
// One wave per row, the row held in registers (lane j holds columns
// j, j + 64, ...).  The backward's dW / db row sums go through a partial
// buffer (one row per workgroup, its 4 waves combined in LDS) and a fixed-
// order final pass, so results do not depend on scheduling.
#include "gpu_kernels.h"
#include "ops_common.hpp"

namespace gptc {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxCols = 2048;  // 32 columns per lane

template <int K>
__global__ __launch_bounds__(kThreads) void layernorm_fwd_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ W,
                                                                const float *__restrict__ b, float *__restrict__ y,
                                                                float *__restrict__ mean_out,
                                                                float *__restrict__ rstd_out, int rows, int C,
                                                                float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWaves + static_cast<int>(threadIdx.x / kWave);
    if (row >= rows) return;
    const float *xr = x + static_cast<int64_t>(row) * C;
    // Every load of the row and of W, b is issued before the first use (clamped
    // indices, no branches around them), so a row costs one memory latency:
    // at the decode step's single row that latency is the whole kernel.
    float v[K], wv[K], bv[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int jc = min(lane + k * kWave, C - 1);
        v[k] = xr[jc];
        wv[k] = W[jc];
        bv[k] = b != nullptr ? b[jc] : 0.0f;
    }
    float s = 0.0f, ss = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const bool in = lane + k * kWave < C;
        v[k] = in ? v[k] : 0.0f;
        s += v[k];
        ss += v[k] * v[k];
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    const float scale = 1.0f / C;
    const float mean = s * scale;
    const float var = ss * scale - mean * mean;
    const float rstd = 1.0f / sqrtf(var + eps);
    float *yr = y + static_cast<int64_t>(row) * C;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = lane + k * kWave;
        if (j < C) {
            const float n = (v[k] - mean) * rstd * wv[k];
            yr[j] = b != nullptr ? n + bv[k] : n;
        }
    }
    if (lane == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// The same forward on float4 columns (C % 4 == 0, 16-byte aligned x, W, b
// and y): lane l holds float4 columns l, l + 64, ... of its wave's row.
template <int K4>
__global__ __launch_bounds__(kThreads) void layernorm_fwd4_kernel(const float *__restrict__ x,
                                                                 const float *__restrict__ W,
                                                                 const float *__restrict__ b, float *__restrict__ y,
                                                                 float *__restrict__ mean_out,
                                                                 float *__restrict__ rstd_out, int rows, int C,
                                                                 float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * kWaves + static_cast<int>(threadIdx.x / kWave);
    if (row >= rows) return;
    const int n4 = C / 4;
    const f32x4_t *xr = reinterpret_cast<const f32x4_t *>(x + static_cast<int64_t>(row) * C);
    const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t v[K4], wv[K4], bv[K4];
#pragma unroll
    for (int k = 0; k < K4; ++k) {  // every load issued before the first use (clamped, no branches)
        const int c = min(lane + k * kWave, n4 - 1);
        v[k] = xr[c];
        wv[k] = reinterpret_cast<const f32x4_t *>(W)[c];
        bv[k] = b != nullptr ? reinterpret_cast<const f32x4_t *>(b)[c] : zero;
    }
    float s = 0.0f, ss = 0.0f;
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        if (lane + k * kWave >= n4) v[k] = zero;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s += v[k][e];
            ss += v[k][e] * v[k][e];
        }
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    const float scale = 1.0f / C;
    const float mean = s * scale;
    const float var = ss * scale - mean * mean;
    const float rstd = 1.0f / sqrtf(var + eps);
    f32x4_t *yr = reinterpret_cast<f32x4_t *>(y + static_cast<int64_t>(row) * C);
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = lane + k * kWave;
        if (c < n4) {
            f32x4_t o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float n = (v[k][e] - mean) * rstd * wv[k][e];
                o[e] = b != nullptr ? n + bv[k][e] : n;
            }
            yr[c] = o;
        }
    }
    if (lane == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// Workgroup blockIdx.x owns rows [r0, r1); its waves take every 4th row.
// partial: (2, gridDim.x, C) = dW then db sums of this workgroup.
// acc: dout += dx (the reference's semantics); otherwise dout = dx.
template <int K>
__global__ __launch_bounds__(kThreads) void layernorm_bwd_kernel(
    const float *__restrict__ g, const float *__restrict__ x, const float *__restrict__ mean_in,
    const float *__restrict__ rstd_in, const float *__restrict__ W, float *__restrict__ dout,
    float *__restrict__ partial, int rows, int C, int rows_per_block, bool acc) {
    extern __shared__ float red[];  // (kWaves, 2, C)
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int r0 = blockIdx.x * rows_per_block;
    const int r1 = min(rows, r0 + rows_per_block);
    const float scale = 1.0f / C;
    float wv[K], dw[K], dbs[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = lane + k * kWave;
        wv[k] = j < C ? W[j] : 0.0f;
        dw[k] = 0.0f;
        dbs[k] = 0.0f;
    }
    for (int row = r0 + w; row < r1; row += kWaves) {
        const float *xr = x + static_cast<int64_t>(row) * C;
        const float *gr = g + static_cast<int64_t>(row) * C;
        float xv[K], gv[K];
        float ds = 0.0f, dbacc = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int j = lane + k * kWave;
            xv[k] = j < C ? xr[j] : 0.0f;
            gv[k] = j < C ? gr[j] : 0.0f;
            ds += gv[k] * xv[k] * wv[k];
            dbacc += gv[k] * wv[k];
        }
        ds = wave_sum(ds);
        dbacc = wave_sum(dbacc);
        const float mean = mean_in[row], a = rstd_in[row];
        const float bn = -a * mean;
        const float bb = (dbacc * mean - ds) * a * a * a * scale;
        const float cc = -bb * mean - dbacc * a * scale;
        float *dr = dout + static_cast<int64_t>(row) * C;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int j = lane + k * kWave;
            if (j < C) {
                dw[k] += gv[k] * (a * xv[k] + bn);
                dbs[k] += gv[k];
                const float d = a * gv[k] * wv[k] + bb * xv[k] + cc;
                dr[j] = acc ? dr[j] + d : d;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = lane + k * kWave;
        if (j < C) {
            red[(w * 2 + 0) * C + j] = dw[k];
            red[(w * 2 + 1) * C + j] = dbs[k];
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < C; j += kThreads) {
        float sw = red[j], sb = red[C + j];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) {
            sw += red[(i * 2 + 0) * C + j];
            sb += red[(i * 2 + 1) * C + j];
        }
        partial[static_cast<int64_t>(blockIdx.x) * C + j] = sw;
        partial[(static_cast<int64_t>(gridDim.x) + blockIdx.x) * C + j] = sb;
    }
}

// The same backward on float4 columns (C % 4 == 0, 16-byte aligned rows and
// W): lane l holds float4 columns l, l + 64, ...  A wave takes ROWS of its
// rows per step (r, r + 4, ...) and issues every load of them, dout's
// included, before the first use, so a step costs one memory latency.
// ACC: dout += dx (the reference's semantics); otherwise dout = dx and
// dout is not read.  The dW / db sums of a column see the rows in the same
// order as in the kernel above.
template <int K4, int ROWS, bool ACC>
__global__ __launch_bounds__(kThreads) void layernorm_bwd4_kernel(
    const float *__restrict__ g, const float *__restrict__ x, const float *__restrict__ mean_in,
    const float *__restrict__ rstd_in, const float *__restrict__ W, float *__restrict__ dout,
    float *__restrict__ partial, int rows, int C, int rows_per_block) {
    extern __shared__ float red[];  // (kWaves, 2, C)
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int n4 = C / 4;
    const int r0 = blockIdx.x * rows_per_block;
    const int r1 = min(rows, r0 + rows_per_block);
    const float scale = 1.0f / C;
    const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t wv[K4], dw[K4], dbs[K4];
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = lane + k * kWave;
        wv[k] = c < n4 ? reinterpret_cast<const f32x4_t *>(W)[c] : zero;
        dw[k] = zero;
        dbs[k] = zero;
    }
    for (int row = r0 + w; row < r1; row += ROWS * kWaves) {
        f32x4_t xv[ROWS][K4], gv[ROWS][K4], ov[ROWS][K4];
        float mean[ROWS], a[ROWS];
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            // A row past r1 repeats row's loads; its results are not used.
            const int ri = min(row + i * kWaves, r1 - 1);
            const f32x4_t *xr = reinterpret_cast<const f32x4_t *>(x + static_cast<int64_t>(ri) * C);
            const f32x4_t *gr = reinterpret_cast<const f32x4_t *>(g + static_cast<int64_t>(ri) * C);
            const f32x4_t *dr = reinterpret_cast<const f32x4_t *>(dout + static_cast<int64_t>(ri) * C);
#pragma unroll
            for (int k = 0; k < K4; ++k) {
                const int c = min(lane + k * kWave, n4 - 1);
                xv[i][k] = xr[c];
                gv[i][k] = gr[c];
                if (ACC) ov[i][k] = dr[c];
            }
            mean[i] = mean_in[ri];
            a[i] = rstd_in[ri];
        }
        float ds[ROWS], dbacc[ROWS];
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            ds[i] = 0.0f;
            dbacc[i] = 0.0f;
#pragma unroll
            for (int k = 0; k < K4; ++k) {
                if (lane + k * kWave >= n4) {  // the clamped loads above: not this lane's columns
                    xv[i][k] = zero;
                    gv[i][k] = zero;
                }
                const f32x4_t gw = gv[i][k] * wv[k];
                const f32x4_t gxw = gw * xv[i][k];
                ds[i] += (gxw[0] + gxw[1]) + (gxw[2] + gxw[3]);
                dbacc[i] += (gw[0] + gw[1]) + (gw[2] + gw[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            ds[i] = wave_sum(ds[i]);
            dbacc[i] = wave_sum(dbacc[i]);
        }
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int r = row + i * kWaves;
            if (i > 0 && r >= r1) break;
            const float m = mean[i], ai = a[i];
            const float bn = -ai * m;
            const float bb = (dbacc[i] * m - ds[i]) * ai * ai * ai * scale;
            const float cc = -bb * m - dbacc[i] * ai * scale;
            f32x4_t *dr = reinterpret_cast<f32x4_t *>(dout + static_cast<int64_t>(r) * C);
#pragma unroll
            for (int k = 0; k < K4; ++k) {
                const int c = lane + k * kWave;
                if (c < n4) {
                    dw[k] += gv[i][k] * (ai * xv[i][k] + bn);
                    dbs[k] += gv[i][k];
                    const f32x4_t d = ai * gv[i][k] * wv[k] + bb * xv[i][k] + cc;
                    dr[c] = ACC ? ov[i][k] + d : d;
                }
            }
        }
    }
    f32x4_t *red4 = reinterpret_cast<f32x4_t *>(red);
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int c = lane + k * kWave;
        if (c < n4) {
            red4[(w * 2 + 0) * n4 + c] = dw[k];
            red4[(w * 2 + 1) * n4 + c] = dbs[k];
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < C; j += kThreads) {
        float sw = red[j], sb = red[C + j];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) {
            sw += red[(i * 2 + 0) * C + j];
            sb += red[(i * 2 + 1) * C + j];
        }
        partial[static_cast<int64_t>(blockIdx.x) * C + j] = sw;
        partial[(static_cast<int64_t>(gridDim.x) + blockIdx.x) * C + j] = sb;
    }
}

int cols_per_lane(int C) {
    const int k = (C + kWave - 1) / kWave;
    if (k <= 4) return 4;
    if (k <= 8) return 8;
    if (k <= 12) return 12;
    if (k <= 16) return 16;
    if (k <= 25) return 25;
    return 32;
}

template <template <int> class F, typename... Args>
void by_cols(int C, Args... args) {
    switch (cols_per_lane(C)) {
        case 4: F<4>::run(args...); break;
        case 8: F<8>::run(args...); break;
        case 12: F<12>::run(args...); break;
        case 16: F<16>::run(args...); break;
        case 25: F<25>::run(args...); break;
        default: F<32>::run(args...); break;
    }
}

template <int K>
struct FwdLaunch {
    static void run(const float *x, const float *W, const float *b, float *y, float *mean, float *rstd, int rows,
                    int C, float eps, hipStream_t s) {
        layernorm_fwd_kernel<K><<<dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0, s>>>(x, W, b, y, mean, rstd,
                                                                                            rows, C, eps);
        hipCheck(hipGetLastError());
    }
};

template <int K>
struct BwdLaunch {
    static void run(const float *g, const float *x, const float *mean, const float *rstd, const float *W, float *dout,
                    float *partial, int rows, int C, int parts, int rows_per_block, bool acc, hipStream_t s) {
        const size_t lds = sizeof(float) * kWaves * 2 * C;
        layernorm_bwd_kernel<K><<<dim3(parts), dim3(kThreads), lds, s>>>(g, x, mean, rstd, W, dout, partial, rows, C,
                                                                        rows_per_block, acc);
        hipCheck(hipGetLastError());
    }
};

// Float4 columns per lane of layernorm_bwd4_kernel: 1, 2, 3, 4, 6 or 8
// (C <= 256, 512, 768, 1024, 1536, 2048); two rows per step up to 4.
template <int K4>
void bwd4_launch(const float *g, const float *x, const float *mean, const float *rstd, const float *W, float *dout,
                 float *partial, int rows, int C, int parts, int rows_per_block, bool acc, hipStream_t s) {
    constexpr int R = K4 <= 4 ? 2 : 1;
    const size_t lds = sizeof(float) * kWaves * 2 * C;
    if (acc)
        layernorm_bwd4_kernel<K4, R, true><<<dim3(parts), dim3(kThreads), lds, s>>>(g, x, mean, rstd, W, dout,
                                                                                   partial, rows, C, rows_per_block);
    else
        layernorm_bwd4_kernel<K4, R, false><<<dim3(parts), dim3(kThreads), lds, s>>>(g, x, mean, rstd, W, dout,
                                                                                    partial, rows, C, rows_per_block);
    hipCheck(hipGetLastError());
}

// dout (+)= dx, dW += ..., db += ... of rows x C (1 <= C <= kMaxCols).
void layer_norm_backward(const float *g, const float *x, const float *mean, const float *rstd, const float *W,
                         float *dout, float *dW, float *db, int rows, int C, bool acc, hipStream_t s) {
    // About 4 rows per wave: 512 workgroups (two per CU) at GPT-2's 8192 rows.
    int parts = (rows + 15) / 16;
    if (parts > 1024) parts = 1024;
    const int rows_per_block = (rows + parts - 1) / parts;
    parts = (rows + rows_per_block - 1) / rows_per_block;
    float *partial = static_cast<float *>(alloc_cuda(sizeof(float) * 2 * static_cast<size_t>(parts) * C));
    if (C % 4 == 0 && aligned16(g) && aligned16(x) && aligned16(W) && aligned16(dout)) {
        const int k4 = (C / 4 + kWave - 1) / kWave;
        auto f = k4 <= 1 ? bwd4_launch<1> : k4 <= 2 ? bwd4_launch<2> : k4 <= 3 ? bwd4_launch<3>
               : k4 <= 4 ? bwd4_launch<4> : k4 <= 6 ? bwd4_launch<6> : bwd4_launch<8>;
        f(g, x, mean, rstd, W, dout, partial, rows, C, parts, rows_per_block, acc, s);
    } else {
        by_cols<BwdLaunch>(C, g, x, mean, rstd, W, dout, partial, rows, C, parts, rows_per_block, acc, s);
    }
    launch_add_column_partials(partial, dW, parts, C, s);
    if (db != nullptr) launch_add_column_partials(partial + static_cast<size_t>(parts) * C, db, parts, C, s);
    free_cuda(partial);
}

void check_cols(int C) {
    CHECK_ERROR(C < 1 || C > kMaxCols, "LayerNorm supports 1 .. %d features, but got %d.", kMaxCols, C);
}

}  // namespace

}  // namespace gptc

using namespace gptc;

extern "C" void layer_norm_forward_cuda_kernel(const tensor_t *W, const tensor_t *b, const tensor_t *input,
                                               const float eps, tensor_t **cache, tensor_t *output) {
    check_gpu(W, "W");
    check_gpu(input, "input");
    check_gpu(output, "output");
    REQUIRE_ARG(cache);
    check_gpu(cache[0], "cache[0] (mean)");
    check_gpu(cache[1], "cache[1] (rstd)");
    const int C = last_dim(input), rows = leading_rows(input);
    check_cols(C);
    CHECK_ERROR(W->length != C, "Expected W to hold %d elements, but got %d.", C, W->length);
    if (b != NULL) {
        check_gpu(b, "b");
        CHECK_ERROR(b->length != C, "Expected b to hold %d elements, but got %d.", C, b->length);
    }
    CHECK_ERROR(output->length != input->length, "Expected output to match input's %d elements.", input->length);
    CHECK_ERROR(cache[0]->length < rows || cache[1]->length < rows, "Expected cache[0..1] to hold %d rows.", rows);
    if (rows == 0) return;
    hipStream_t s = gptc_stream_checked();
    const float *bp = b != NULL ? b->t : nullptr;
    if (C % 4 == 0 && aligned16(input->t) && aligned16(W->t) && (bp == nullptr || aligned16(bp)) &&
        aligned16(output->t)) {
        const int k4 = (C / 4 + kWave - 1) / kWave;
        auto f = k4 <= 1 ? layernorm_fwd4_kernel<1> : k4 <= 2 ? layernorm_fwd4_kernel<2>
               : k4 <= 3 ? layernorm_fwd4_kernel<3> : k4 <= 4 ? layernorm_fwd4_kernel<4>
               : k4 <= 6 ? layernorm_fwd4_kernel<6> : layernorm_fwd4_kernel<8>;
        f<<<dim3((rows + kWaves - 1) / kWaves), dim3(kThreads), 0, s>>>(input->t, W->t, bp, output->t, cache[0]->t,
                                                                       cache[1]->t, rows, C, eps);
        hipCheck(hipGetLastError());
        return;
    }
    by_cols<FwdLaunch>(C, static_cast<const float *>(input->t), static_cast<const float *>(W->t), bp, output->t,
                       cache[0]->t, cache[1]->t, rows, C, eps, s);
}

namespace {

void layer_norm_backward_checked(const tensor_t *global_grad, const tensor_t **cache, const tensor_t *W, tensor_t *dW,
                                 tensor_t *db, tensor_t *dout, bool acc) {
    check_gpu(global_grad, "global_grad");
    REQUIRE_ARG(cache);
    check_gpu(cache[0], "cache[0] (mean)");
    check_gpu(cache[1], "cache[1] (rstd)");
    check_gpu(cache[2], "cache[2] (input)");
    check_gpu(W, "W");
    check_gpu(dW, "dW");
    check_gpu(dout, "dout");
    const int C = last_dim(global_grad), rows = leading_rows(global_grad);
    check_cols(C);
    CHECK_ERROR(W->length != C || dW->length != C, "Expected W and dW to hold %d elements.", C);
    CHECK_ERROR(cache[2]->length != global_grad->length || dout->length != global_grad->length,
                "Expected the cached input and dout to match global_grad's %d elements.", global_grad->length);
    CHECK_ERROR(cache[0]->length < rows || cache[1]->length < rows, "Expected cache[0..1] to hold %d rows.", rows);
    if (db != NULL) {
        check_gpu(db, "db");
        CHECK_ERROR(db->length != C, "Expected db to hold %d elements, but got %d.", C, db->length);
    }
    if (rows == 0) return;
    layer_norm_backward(global_grad->t, cache[2]->t, cache[0]->t, cache[1]->t, W->t, dout->t, dW->t,
                        db != NULL ? db->t : nullptr, rows, C, acc, gptc_stream_checked());
}

}  // namespace

extern "C" void layer_norm_backward_cuda_kernel(const tensor_t *global_grad, const tensor_t **cache,
                                                const tensor_t *W, tensor_t *dW, tensor_t *db, tensor_t *dout) {
    layer_norm_backward_checked(global_grad, cache, W, dW, db, dout, true);
}

extern "C" void gptc_layer_norm_backward_set(const tensor_t *global_grad, const tensor_t **cache, const tensor_t *W,
                                             tensor_t *dW, tensor_t *db, tensor_t *dout) {
    layer_norm_backward_checked(global_grad, cache, W, dW, db, dout, false);
}
