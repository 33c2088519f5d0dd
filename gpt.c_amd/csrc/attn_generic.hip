// Causal attention for head sizes past 128 (up to kGenericMaxD), which the
// MFMA kernels are not built for: gpt.c accepts any head size with
// n_embd % n_heads == 0 (src/attention.c:23, kernels/src/cpu/Attention.c:78),
// so these kernels serve the rest with plain fp32 FMAs.  They are correct and
// general, not fast: no configuration of the benchmark uses such heads.
//
// Forward and backward keep the LSE-only state (no probability blocks):
//   attn_fwd_generic_kernel   one wave per query (4 per workgroup, one head);
//                             key chunks of KC rows of K and V staged in LDS;
//                             lane j scores key k0 + j (a dot product over D
//                             from LDS), the online softmax over chunks (wave
//                             max and sum), o += sum_j p_j v_j with lanes over
//                             dims; y = o / l and the natural-log LSE.
//   attn_bwd_dq_generic_kernel   the same loop per query: s, dP = dO . v_j,
//                             P = exp(s - LSE), dS = P (dP - delta), dQ +=
//                             sum_j dS_j k_j.
//   attn_bwd_dkdv_generic_kernel one wave per key over query chunks from the
//                             key on: dV += sum_i P_i dO_i, dK += sum_i dS_i q_i.
// delta = rowsum(dO o O) comes from attn_bwd_delta_kernel as for every head
// size.  Math as kernels/src/cpu/Attention.c:46-301 (P = softmax over keys
// j <= i of q_i . k_j / sqrt(D)).
#include "attn_common.hpp"
#include "attn_kernels.hpp"
#include "hip_check.hpp"

#include <mutex>

namespace gptc {

namespace {

constexpr int kGenWaves = 4;  // queries (or keys) per workgroup

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Keys (or queries) per staged chunk for head size D: the largest of 64, 32,
// 16 and 8 with which the two tiles of KC x (D + 1) and KC x D floats, the
// waves' rows and weights (and 2 KB of static LDS) stay within 150 KB.
__host__ __device__ inline int generic_chunk(int D) {
    const int kc = (150 * 1024 / 4 - 2 * kGenWaves * D - kGenWaves * 64 - 512) / (2 * D + 1);
    return kc >= 64 ? 64 : (kc >= 32 ? 32 : (kc >= 16 ? 16 : 8));
}

// Dynamic LDS of the generic kernels: [A tile KC x (D+1)] [B tile KC x D]
// [4 rows of D (the waves' own vectors)] [4 more rows of D] [4 x 64 weights].
__host__ __device__ inline size_t generic_lds_floats(int D) {
    const int kc = generic_chunk(D);
    return static_cast<size_t>(kc) * (D + 1) + static_cast<size_t>(kc) * D + 2 * kGenWaves * D + kGenWaves * 64;
}

// Rows [r0, r0 + kc) of two (B, H, T, D)-viewed tensors of head (b, h) into
// LDS (rows past T as zeros): A with row stride D + 1, B with stride D.
__device__ __forceinline__ void stage_rows(const HeadView &va, const HeadView &vb, int b, int h, int r0, int kc,
                                           int T, int D, float *a_s, float *b_s) {
    const float *pa = va.p + b * va.sb + h * va.sh;
    const float *pb = vb.p + b * vb.sb + h * vb.sh;
    for (int e = threadIdx.x; e < kc * D; e += blockDim.x) {
        const int r = e / D, d = e - r * D, t = r0 + r;
        const bool ok = t < T;
        a_s[r * (D + 1) + d] = ok ? pa[t * va.st + d] : 0.0f;
        b_s[r * D + d] = ok ? pb[t * vb.st + d] : 0.0f;
    }
}

}  // namespace

__global__ __launch_bounds__(256) void attn_fwd_generic_kernel(const FwdParams a) {
    extern __shared__ float lds[];
    const int D = a.D, T = a.T, kc = generic_chunk(D);
    float *k_s = lds, *v_s = k_s + kc * (D + 1), *q_s = v_s + kc * D, *p_s = q_s + 2 * kGenWaves * D;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ngrp = (T + kGenWaves - 1) / kGenWaves;
    const int bh = blockIdx.x / ngrp, i0 = (blockIdx.x - bh * ngrp) * kGenWaves;
    const int b = bh / a.H, h = bh - b * a.H;
    const int i = i0 + w;
    const bool row_ok = i < T;
    float *qw = q_s + w * D;
    for (int d = lane; d < D; d += 64) qw[d] = row_ok ? a.q.p[b * a.q.sb + i * a.q.st + h * a.q.sh + d] : 0.0f;
    // The reference cache layout: this workgroup's rows of q, k, v, permuted.
    if (a.qp != nullptr && row_ok) {
        const size_t off = (static_cast<size_t>(bh) * T + i) * D;
        for (int d = lane; d < D; d += 64) {
            a.qp[off + d] = qw[d];
            a.kp[off + d] = a.k.p[b * a.k.sb + i * a.k.st + h * a.k.sh + d];
            a.vp[off + d] = a.v.p[b * a.v.sb + i * a.v.st + h * a.v.sh + d];
        }
    }
    const float c2 = a.scale_log2;
    float m = -INFINITY, l = 0.0f;
    float o[kGenericMaxD / 64];
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) o[x] = 0.0f;
    const int last = min(i0 + kGenWaves, T) - 1;  // the workgroup's last query
    for (int k0 = 0; k0 <= last; k0 += kc) {
        __syncthreads();
        stage_rows(a.k, a.v, b, h, k0, kc, T, D, k_s, v_s);
        __syncthreads();
        const int key = k0 + lane;
        float s = -INFINITY;
        if (lane < kc && row_ok && key <= i) {
            float acc = 0.0f;
            for (int d = 0; d < D; ++d) acc = fmaf(qw[d], k_s[lane * (D + 1) + d], acc);
            s = acc * c2;
        }
        const float mc = wave_max(s);
        const float m_new = fmaxf(m, mc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2(m - m_use);
        const float p = fast_exp2(s - m_use);
        l = l * alpha + wave_sum(p);
        p_s[w * 64 + lane] = p;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int x = 0; x < kGenericMaxD / 64; ++x) {
            const int d = lane + 64 * x;
            if (d < D) {
                float acc = o[x] * alpha;
                for (int j = 0; j < kc; ++j) acc = fmaf(p_s[w * 64 + j], v_s[j * D + d], acc);
                o[x] = acc;
            }
        }
        __builtin_amdgcn_wave_barrier();
        m = m_new;
    }
    if (!row_ok) return;
    const float inv = 1.0f / l;
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) {
        const int d = lane + 64 * x;
        if (d < D) {
            a.o.p[b * a.o.sb + i * a.o.st + h * a.o.sh + d] = o[x] * inv;
            if (a.o2) a.o2[b * a.o.sb + i * a.o.st + h * a.o.sh + d] = o[x] * inv;
        }
    }
    if (lane == 0) a.lse[static_cast<size_t>(bh) * T + i] = (m + log2f(l)) * kLn2;
}

__global__ __launch_bounds__(256) void attn_bwd_dq_generic_kernel(const BwdParams a) {
    extern __shared__ float lds[];
    const int D = a.D, T = a.T, kc = generic_chunk(D);
    float *k_s = lds, *v_s = k_s + kc * (D + 1), *q_s = v_s + kc * D, *do_s = q_s + kGenWaves * D;
    float *p_s = q_s + 2 * kGenWaves * D;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ngrp = (T + kGenWaves - 1) / kGenWaves;
    const int bh = blockIdx.x / ngrp, i0 = (blockIdx.x - bh * ngrp) * kGenWaves;
    const int b = bh / a.H, h = bh - b * a.H;
    const int i = i0 + w;
    const bool row_ok = i < T;
    float *qw = q_s + w * D, *gw = do_s + w * D;
    for (int d = lane; d < D; d += 64) {
        qw[d] = row_ok ? a.q.p[b * a.q.sb + i * a.q.st + h * a.q.sh + d] : 0.0f;
        gw[d] = row_ok ? a.dout.p[b * a.dout.sb + i * a.dout.st + h * a.dout.sh + d] : 0.0f;
    }
    const float c2 = a.scale * kLog2e;
    const float lse2 = row_ok ? a.lse[static_cast<size_t>(bh) * T + i] * kLog2e : 0.0f;
    const float dl = row_ok ? a.delta[static_cast<size_t>(bh) * T + i] : 0.0f;
    float acc_q[kGenericMaxD / 64];
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) acc_q[x] = 0.0f;
    const int last = min(i0 + kGenWaves, T) - 1;
    for (int k0 = 0; k0 <= last; k0 += kc) {
        __syncthreads();
        stage_rows(a.k, a.v, b, h, k0, kc, T, D, k_s, v_s);
        __syncthreads();
        const int key = k0 + lane;
        float ds = 0.0f;
        if (lane < kc && row_ok && key <= i) {
            float s = 0.0f, dp = 0.0f;
            for (int d = 0; d < D; ++d) {
                s = fmaf(qw[d], k_s[lane * (D + 1) + d], s);
                dp = fmaf(gw[d], v_s[lane * D + d], dp);
            }
            const float p = fast_exp2(fmaf(s, c2, -lse2));
            ds = p * (dp - dl);
        }
        p_s[w * 64 + lane] = ds;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int x = 0; x < kGenericMaxD / 64; ++x) {
            const int d = lane + 64 * x;
            if (d < D) {
                float acc = acc_q[x];
                for (int j = 0; j < kc; ++j) acc = fmaf(p_s[w * 64 + j], k_s[j * (D + 1) + d], acc);
                acc_q[x] = acc;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (!row_ok) return;
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) {
        const int d = lane + 64 * x;
        if (d < D) a.dq.p[b * a.dq.sb + i * a.dq.st + h * a.dq.sh + d] = acc_q[x] * a.scale;
    }
}

__global__ __launch_bounds__(256) void attn_bwd_dkdv_generic_kernel(const BwdParams a) {
    extern __shared__ float lds[];
    const int D = a.D, T = a.T, kc = generic_chunk(D);
    // A tile: Q rows (stride D + 1), B tile: dO rows; per wave its K and V
    // rows; p_s: each wave's P of the chunk's queries (dS in ds_s).
    float *q_s = lds, *g_s = q_s + kc * (D + 1), *k_s = g_s + kc * D, *v_s = k_s + kGenWaves * D;
    float *p_s = k_s + 2 * kGenWaves * D;  // [w][64]: P of the chunk's queries
    __shared__ float ds_s[kGenWaves][64];    // dS of the chunk's queries
    __shared__ float st_s[2][64];            // LSE log2(e) and delta of the chunk's queries
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ngrp = (T + kGenWaves - 1) / kGenWaves;
    const int bh = blockIdx.x / ngrp, j0 = (blockIdx.x - bh * ngrp) * kGenWaves;
    const int b = bh / a.H, h = bh - b * a.H;
    const int j = j0 + w;
    const bool key_ok = j < T;
    float *kw = k_s + w * D, *vw = v_s + w * D;
    for (int d = lane; d < D; d += 64) {
        kw[d] = key_ok ? a.k.p[b * a.k.sb + j * a.k.st + h * a.k.sh + d] : 0.0f;
        vw[d] = key_ok ? a.v.p[b * a.v.sb + j * a.v.st + h * a.v.sh + d] : 0.0f;
    }
    const float c2 = a.scale * kLog2e;
    float acc_k[kGenericMaxD / 64], acc_v[kGenericMaxD / 64];
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) acc_k[x] = acc_v[x] = 0.0f;
    for (int q0 = j0; q0 < T; q0 += kc) {
        __syncthreads();
        stage_rows(a.q, a.dout, b, h, q0, kc, T, D, q_s, g_s);
        if (threadIdx.x < kc) {
            const int q = q0 + threadIdx.x;
            st_s[0][threadIdx.x] = q < T ? a.lse[static_cast<size_t>(bh) * T + q] * kLog2e : INFINITY;
            st_s[1][threadIdx.x] = q < T ? a.delta[static_cast<size_t>(bh) * T + q] : 0.0f;
        }
        __syncthreads();
        const int q = q0 + lane;
        float p = 0.0f, ds = 0.0f;
        if (lane < kc && key_ok && q < T && q >= j) {
            float s = 0.0f, dp = 0.0f;
            for (int d = 0; d < D; ++d) {
                s = fmaf(q_s[lane * (D + 1) + d], kw[d], s);
                dp = fmaf(g_s[lane * D + d], vw[d], dp);
            }
            p = fast_exp2(fmaf(s, c2, -st_s[0][lane]));
            ds = p * (dp - st_s[1][lane]);
        }
        p_s[w * 64 + lane] = p;
        ds_s[w][lane] = ds;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int x = 0; x < kGenericMaxD / 64; ++x) {
            const int d = lane + 64 * x;
            if (d < D) {
                float ak = acc_k[x], av = acc_v[x];
                for (int r = 0; r < kc; ++r) {
                    ak = fmaf(ds_s[w][r], q_s[r * (D + 1) + d], ak);
                    av = fmaf(p_s[w * 64 + r], g_s[r * D + d], av);
                }
                acc_k[x] = ak;
                acc_v[x] = av;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    if (!key_ok) return;
#pragma unroll
    for (int x = 0; x < kGenericMaxD / 64; ++x) {
        const int d = lane + 64 * x;
        if (d < D) {
            a.dk.p[b * a.dk.sb + j * a.dk.st + h * a.dk.sh + d] = acc_k[x] * a.scale;
            a.dv.p[b * a.dv.sb + j * a.dv.st + h * a.dv.sh + d] = acc_v[x];
        }
    }
}

namespace {

// Dynamic LDS of D, allowed past the default limit for `kernel` (once per
// kernel; the three kernels' largest need is under 152 KB).
size_t generic_lds_bytes(const void *kernel, int D) {
    static std::once_flag once[3];
    static const void *kernels[3] = {reinterpret_cast<const void *>(attn_fwd_generic_kernel),
                                     reinterpret_cast<const void *>(attn_bwd_dq_generic_kernel),
                                     reinterpret_cast<const void *>(attn_bwd_dkdv_generic_kernel)};
    for (int k = 0; k < 3; ++k)
        if (kernels[k] == kernel)
            std::call_once(once[k], [&] {
                hipCheck(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 152 * 1024));
            });
    return generic_lds_floats(D) * sizeof(float);
}

}  // namespace

void launch_attn_fwd_generic(const FwdParams &p, hipStream_t stream) {
    const int ngrp = (p.T + kGenWaves - 1) / kGenWaves;
    const size_t lds = generic_lds_bytes(reinterpret_cast<const void *>(attn_fwd_generic_kernel), p.D);
    attn_fwd_generic_kernel<<<dim3(p.B * p.H * ngrp), dim3(256), lds, stream>>>(p);
    hipCheck(hipGetLastError());
}

void launch_attn_bwd_generic(const BwdParams &p, hipStream_t stream, const hipEvent_t *ev) {
    const int ngrp = (p.T + kGenWaves - 1) / kGenWaves;
    const size_t lds = generic_lds_bytes(reinterpret_cast<const void *>(attn_bwd_dkdv_generic_kernel), p.D);
    generic_lds_bytes(reinterpret_cast<const void *>(attn_bwd_dq_generic_kernel), p.D);
    attn_bwd_dkdv_generic_kernel<<<dim3(p.B * p.H * ngrp), dim3(256), lds, stream>>>(p);
    hipCheck(hipGetLastError());
    if (ev) {
        hipCheck(hipEventRecord(ev[3], stream));
        hipCheck(hipEventRecord(ev[4], stream));
    }
    attn_bwd_dq_generic_kernel<<<dim3(p.B * p.H * ngrp), dim3(256), lds, stream>>>(p);
    hipCheck(hipGetLastError());
}

}  // namespace gptc
