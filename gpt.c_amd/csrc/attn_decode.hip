// One decode step of causal self-attention with a KV cache: the new token's
// q, k, v row (B, 1, 3C) is attended against keys 0..pos of (B, H, L, D)
// K/V caches, after its own k, v are written at position pos.
//
// gpt.c has no KV cache: its inference loop (infer_gpt.c:339-351) runs the
// whole block_size window through the model for every new token, and keeps
// only row i-1 of the logits.  Under the causal rule that row of attention's
// output depends on keys 0..i-1 only, so this kernel returns exactly the
// row the window recompute produces (attention.c / Attention.c math:
// softmax(q k^T / sqrt(D)) v), reading each cached key and value once.
//
// The work is HBM- and latency-bound (4 L D flop against 8 L D bytes per
// (b, h)).  For D == 64 with 16-byte cache rows, steps of at most
// kDecHeadKeys keys run attn_decode_head_kernel (one launch, one workgroup
// per (b, h)) and longer ones the split-key pair at the end of this file;
// the kernel first below serves the other head sizes:
// one 1024-thread workgroup (16 waves) per (b, h), with as many row loads in
// flight as the registers allow (head sizes up to 128, and a build for the
// generic head sizes up to kGenericMaxD).
//   phase 1  thread per key: t_j = (q . k_j) log2(e)/sqrt(D) into LDS;
//   phase 2  workgroup max m and sum l of p_j = exp2(t_j - m);
//   phase 3  wave per key row, lane per dim: o = sum_j p_j v_j (coalesced
//            256-byte rows, 8 rows in flight per wave), then the 16 waves'
//            partial sums are added.
#include "attn_common.hpp"
#include "attn_kernels.hpp"
#include "hip_check.hpp"

#include <mutex>

namespace gptc {

namespace {

constexpr int kDecThreads = 1024;
constexpr int kDecWaves = kDecThreads / 64;

__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
    // Wave reduction, then the wave results through LDS (a fixed order).
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kDecWaves; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
    return r;
}

}  // namespace

// DMAX: the largest head size of the build, 2 * kDPad (128) or kGenericMaxD
// (1024, the generic head sizes; more LDS per workgroup).
template <int DMAX>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(const DecParams a) {
    constexpr int kDecMaxD = DMAX;
    static_assert(DMAX <= kDecThreads, "one thread per dim loads the new row");
    extern __shared__ float dyn_lds[];  // scores: pos + 1 floats (L with a device-side position)
    __shared__ float q_s[kDecMaxD], k_s[kDecMaxD], v_s[kDecMaxD];
    __shared__ float o_s[kDecWaves][kDecMaxD];
    __shared__ float red[kDecWaves];

    // A device-side position (graph replays) is checked here, since the host
    // could not: out of [0, L) the workgroup does nothing.
    const int pos = a.pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*a.pos_dev) : a.pos;
    if (pos < 0 || pos >= a.L) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int D = a.D, n = pos + 1;

    // The new row: q, k, v of head h; k and v also go into the caches at pos.
    const float *row = a.qkv + static_cast<size_t>(b) * 3 * a.C + h * D;
    float *kc = a.k_cache + static_cast<size_t>(bh) * a.L * D;
    float *vc = a.v_cache + static_cast<size_t>(bh) * a.L * D;
    if (tid < kDecMaxD) {
        const bool ok = tid < D;
        q_s[tid] = ok ? row[tid] : 0.0f;
        const float kn = ok ? row[a.C + tid] : 0.0f, vn = ok ? row[2 * a.C + tid] : 0.0f;
        k_s[tid] = kn;
        v_s[tid] = vn;
        if (ok) {
            kc[static_cast<size_t>(pos) * D + tid] = kn;
            vc[static_cast<size_t>(pos) * D + tid] = vn;
        }
    }
    __syncthreads();

    // Phase 1: scores in log2 units.  Key pos (the last) comes from LDS, its
    // cache row having just been written by this workgroup.  full: D == 64
    // and 16-byte rows, so a key row is 16 float4 loads.
    float q[kDPad];
#pragma unroll
    for (int d = 0; d < kDPad; ++d) q[d] = q_s[d];
    float t_max = -INFINITY;
    for (int j = tid; j < n; j += kDecThreads) {
        float acc = 0.0f;
        if (j == pos) {
            if (D <= kDPad) {
#pragma unroll
                for (int d = 0; d < kDPad; ++d) acc = fmaf(q[d], k_s[d], acc);
            } else {
                for (int d = 0; d < D; ++d) acc = fmaf(q_s[d], k_s[d], acc);
            }
        } else if (a.full) {
            const f32x4 *kr = reinterpret_cast<const f32x4 *>(kc + static_cast<size_t>(j) * D);
#pragma unroll
            for (int i = 0; i < kDPad / 4; ++i) {
                const f32x4 k4 = kr[i];
                acc = fmaf(q[4 * i], k4[0], acc);
                acc = fmaf(q[4 * i + 1], k4[1], acc);
                acc = fmaf(q[4 * i + 2], k4[2], acc);
                acc = fmaf(q[4 * i + 3], k4[3], acc);
            }
        } else {
            const float *kr = kc + static_cast<size_t>(j) * D;
            for (int d = 0; d < D; ++d) acc = fmaf(q_s[d], kr[d], acc);
        }
        const float t = acc * a.scale_log2;
        dyn_lds[j] = t;
        t_max = fmaxf(t_max, t);
    }
    const float m = block_reduce(t_max, red, true);

    // Phase 2: p_j = exp2(t_j - m) in place, and their sum.
    float l_part = 0.0f;
    for (int j = tid; j < n; j += kDecThreads) {
        const float p = fast_exp2(dyn_lds[j] - m);
        dyn_lds[j] = p;
        l_part += p;
    }
    const float l = block_reduce(l_part, red, false);  // its barriers also publish the p_j

    // Phase 3: wave w takes keys w, w + 16, ...; lane = dim (and dim + 64
    // for head sizes past 64).
    constexpr int kUnroll = 8;
    for (int dim = lane; dim < kDecMaxD; dim += 64) {
        float o = 0.0f;
        if (dim < D) {
            int j = w;
            // Keys below pos come from the cache, kUnroll rows in flight per lane.
            for (; j + (kUnroll - 1) * kDecWaves < pos; j += kUnroll * kDecWaves) {
                float v[kUnroll];
#pragma unroll
                for (int u = 0; u < kUnroll; ++u) v[u] = vc[static_cast<size_t>(j + u * kDecWaves) * D + dim];
#pragma unroll
                for (int u = 0; u < kUnroll; ++u) o = fmaf(dyn_lds[j + u * kDecWaves], v[u], o);
            }
            for (; j < n; j += kDecWaves) {
                const float v = (j == pos) ? v_s[dim] : vc[static_cast<size_t>(j) * D + dim];
                o = fmaf(dyn_lds[j], v, o);
            }
        }
        o_s[w][dim] = o;
        if (D <= kDPad) break;
    }
    __syncthreads();
    if (tid < D) {
        float y = o_s[0][tid];
#pragma unroll
        for (int i = 1; i < kDecWaves; ++i) y += o_s[i][tid];
        a.out[static_cast<size_t>(b) * a.C + h * D + tid] = y / l;
    }
}

// ---- Split-key decode (D == 64, 16-byte rows) ----
//
// At B = 1 the kernel above runs one workgroup per head, and each of its
// phases waits for a dependent round trip to HBM; twelve heads leave most of
// the GPU idle.  Here the keys 0 .. pos of every (b, h) are cut into chunks
// of kDecChunk, one 256-thread workgroup each, which writes the chunk's
// partial softmax state (max m_s and sum l_s of exp2(t - m_s), unnormalised
// o_s = sum p v); a second kernel merges the chunks of each (b, h):
//   M = max m_s,  l = sum l_s exp2(m_s - M),  o = sum o_s exp2(m_s - M) / l
// (computed in one pass as a running merge).
// The workgroup holding key pos takes the new k, v from the qkv row and
// writes them into the caches at pos; the others read cache rows below pos.
__global__ __launch_bounds__(256) void attn_decode_split_kernel(const DecParams a) {
    __shared__ __attribute__((aligned(16))) float q_s[kDPad];
    __shared__ __attribute__((aligned(16))) float k_s[kDPad];
    __shared__ __attribute__((aligned(16))) float v_s[kDPad];
    __shared__ float p_s[kDecChunk];
    __shared__ float o_red[4][kDPad];
    __shared__ float red[4];

    const int pos = a.pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*a.pos_dev) : a.pos;
    if (pos < 0 || pos >= a.L) return;
    const int bh = blockIdx.x / a.splits, sp = blockIdx.x - bh * a.splits;
    const int j0 = sp * kDecChunk;
    if (j0 > pos) return;  // a chunk past the position (fixed grids of graph replays)
    const int n = min(kDecChunk, pos + 1 - j0);
    const bool has_pos = pos < j0 + kDecChunk;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = bh / a.H, h = bh - b * a.H;

    const float *row = a.qkv + static_cast<size_t>(b) * 3 * a.C + h * kDPad;
    float *kc = a.k_cache + static_cast<size_t>(bh) * a.L * kDPad;
    float *vc = a.v_cache + static_cast<size_t>(bh) * a.L * kDPad;
    // V rows of this lane (dim `lane`; wave w takes keys w, w + 4, ...), issued
    // first so that their latency overlaps the score phase.  Key pos is
    // replaced by the new v below.
    float v[kDecChunk / 4];
#pragma unroll
    for (int u = 0; u < kDecChunk / 4; ++u) {
        const int kj = w + 4 * u;
        v[u] = kj < n ? vc[static_cast<size_t>(j0 + kj) * kDPad + lane] : 0.0f;
    }
    if (tid < kDPad) {
        q_s[tid] = row[tid];
        if (has_pos) {
            const float kn = row[a.C + tid], vn = row[2 * a.C + tid];
            k_s[tid] = kn;
            v_s[tid] = vn;
            kc[static_cast<size_t>(pos) * kDPad + tid] = kn;
            vc[static_cast<size_t>(pos) * kDPad + tid] = vn;
        }
    }
    __syncthreads();

    // Scores: four threads per key, 16 dims each.
    const int kk = tid >> 2, qq = tid & 3;
    float t = -INFINITY;
    {
        float acc = 0.0f;
        if (kk < n) {
            const int j = j0 + kk;
            const float *kr = (j == pos) ? k_s : kc + static_cast<size_t>(j) * kDPad;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x4 k4 = *reinterpret_cast<const f32x4 *>(kr + 16 * qq + 4 * i);
                const f32x4 q4 = *reinterpret_cast<const f32x4 *>(q_s + 16 * qq + 4 * i);
                acc = fmaf(q4[0], k4[0], acc);
                acc = fmaf(q4[1], k4[1], acc);
                acc = fmaf(q4[2], k4[2], acc);
                acc = fmaf(q4[3], k4[3], acc);
            }
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        if (kk < n) t = acc * a.scale_log2;
    }
    float m = t;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float p = kk < n ? fast_exp2(t - m) : 0.0f;
    if (qq == 0) p_s[kk] = p;
    // The sum of p over the chunk (each key counted by its qq == 0 thread).
    float l = qq == 0 ? p : 0.0f;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
    __syncthreads();  // p_s complete; red[] read by everyone
    if (lane == 0) red[w] = l;

    // o = sum_j p_j v_j: lane = dim, wave w takes keys w, w + 4, ... (16 rows in flight).
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < kDecChunk / 4; ++u) {
        const int kj = w + 4 * u;
        if (j0 + kj == pos) v[u] = v_s[lane];
        o = fmaf(p_s[w + 4 * u], v[u], o);
    }
    o_red[w][lane] = o;
    __syncthreads();
    if (tid < kDPad) {
        float *rec = a.part + (static_cast<size_t>(bh) * a.splits + sp) * kDecPartStride;
        rec[tid] = (o_red[0][tid] + o_red[1][tid]) + (o_red[2][tid] + o_red[3][tid]);
        if (tid == 0) {
            rec[kDPad] = m;
            rec[kDPad + 1] = (red[0] + red[1]) + (red[2] + red[3]);
        }
    }
}

__global__ __launch_bounds__(64) void attn_decode_merge_kernel(const DecParams a) {
    const int pos = a.pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*a.pos_dev) : a.pos;
    if (pos < 0 || pos >= a.L) return;
    const int bh = blockIdx.x, d = threadIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int ns = pos / kDecChunk + 1;  // chunks holding keys
    const float *rec = a.part + static_cast<size_t>(bh) * a.splits * kDecPartStride;
    // One pass, merging the chunks' states in order (their loads do not wait
    // on each other; every chunk holds a key, so its m_s is finite).
    float M = -INFINITY, l = 0.0f, o = 0.0f;
#pragma unroll 8
    for (int s = 0; s < ns; ++s) {
        const float ms = rec[s * kDecPartStride + kDPad], ls = rec[s * kDecPartStride + kDPad + 1];
        const float os = rec[s * kDecPartStride + d];
        const float mn = fmaxf(M, ms);
        const float fa = fast_exp2(M - mn), fb = fast_exp2(ms - mn);
        l = fmaf(l, fa, ls * fb);
        o = fmaf(o, fa, os * fb);
        M = mn;
    }
    a.out[static_cast<size_t>(b) * a.C + h * kDPad + d] = o / l;
}

// ---- One-launch decode of a short cache (D == 64, 16-byte rows) ----
//
// For up to kDecHeadKeys keys the whole (b, h) fits one 1024-thread
// workgroup with every K and V row it needs in flight at once, so the step
// is one launch and one memory round trip (the split pair above costs two
// launches).  Key j of round r (j = 64r + 4w + lane/16) belongs to the 16
// lanes of row group lane/16 of wave w; lane g = lane % 16 holds dims
// 4g .. 4g+3 of that key's K and V rows.  Per lane: q[4g..4g+3], then the
// dot products of its keys reduced over the 16 lanes of the group (each of
// them then holds t_j), the workgroup max through LDS, p_j = exp2(t_j - m),
// o = sum p_j v_j over the lane's keys, reduced over the wave's four groups
// and the 16 waves (a fixed order), and y = o / l.  Key pos (the new token)
// is read from the qkv row and written to both caches at pos.
// R: the rounds of 64 keys that hold a key (pos / 64 + 1), a compile-time
// count so that the loads of empty rounds are not issued at all (they would
// still cost the CU's L1 bandwidth, the step's bound at B = 1).
template <int R>
__device__ __forceinline__ void decode_head_rounds(const DecParams &a, int pos, float *m_red, float *l_red,
                                                   float (*o_red)[kDPad]) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = blockIdx.x;
    const int b = bh / a.H, h = bh - b * a.H;
    const int n = pos + 1;

    const float *row = a.qkv + static_cast<size_t>(b) * 3 * a.C + h * kDPad;
    float *kc = a.k_cache + static_cast<size_t>(bh) * a.L * kDPad;
    float *vc = a.v_cache + static_cast<size_t>(bh) * a.L * kDPad;
    const f32x4 q4 = *reinterpret_cast<const f32x4 *>(row + 4 * g);
    // Every K and V row of this lane's keys, requested before any is used
    // (no branch or select between the loads, which would wait for them):
    // keys pos and beyond read the new row, whose k, v are finite; keys past
    // pos get t = -inf and p = 0 below.
    f32x4 k4[R], v4[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int j = 64 * r + 4 * w + (lane >> 4);
        const size_t cj = static_cast<size_t>(j < pos ? j : 0) * kDPad;
        const float *kr = j < pos ? kc + cj : row + a.C;
        const float *vr = j < pos ? vc + cj : row + 2 * a.C;
        k4[r] = *reinterpret_cast<const f32x4 *>(kr + 4 * g);
        v4[r] = *reinterpret_cast<const f32x4 *>(vr + 4 * g);
    }
    if (tid < 16) {
        // The new k, v into the caches at pos (read from the qkv row).
        const f32x4 kn = *reinterpret_cast<const f32x4 *>(row + a.C + 4 * tid);
        const f32x4 vn = *reinterpret_cast<const f32x4 *>(row + 2 * a.C + 4 * tid);
        *reinterpret_cast<f32x4 *>(kc + static_cast<size_t>(pos) * kDPad + 4 * tid) = kn;
        *reinterpret_cast<f32x4 *>(vc + static_cast<size_t>(pos) * kDPad + 4 * tid) = vn;
    }

    // Scores t_j (log2 units) of the lane's keys, -inf past pos.
    float t[R];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = q4[0] * k4[r][0];
        acc = fmaf(q4[1], k4[r][1], acc);
        acc = fmaf(q4[2], k4[r][2], acc);
        acc = fmaf(q4[3], k4[r][3], acc);
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, 64);
        const int j = 64 * r + 4 * w + (lane >> 4);
        t[r] = j < n ? acc * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, t[r]);
    }
    // The four row groups of the wave, then the 16 waves.
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (lane == 0) m_red[w] = mx;
    __syncthreads();
    float m = m_red[0];
#pragma unroll
    for (int i = 1; i < kDecWaves; ++i) m = fmaxf(m, m_red[i]);

    float l = 0.0f;
    f32x4 o = zero4();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float p = fast_exp2(t[r] - m);  // 0 past pos
        l += p;
        o += p * v4[r];
    }
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += __shfl_xor(o[e], off, 64);
    }
    if (lane < 16) *reinterpret_cast<f32x4 *>(&o_red[w][4 * lane]) = o;
    if (lane == 0) l_red[w] = l;
    __syncthreads();
    if (tid < kDPad) {
        float y = o_red[0][tid], ls = l_red[0];
#pragma unroll
        for (int i = 1; i < kDecWaves; ++i) {
            y += o_red[i][tid];
            ls += l_red[i];
        }
        a.out[static_cast<size_t>(b) * a.C + h * kDPad + tid] = y / ls;
    }
}

__global__ __launch_bounds__(kDecThreads) void attn_decode_head_kernel(const DecParams a) {
    static_assert(kDecHeadKeys == 8 * 64, "the switch below covers 8 rounds of 64 keys");
    __shared__ float m_red[kDecWaves];
    __shared__ float l_red[kDecWaves];
    __shared__ __attribute__((aligned(16))) float o_red[kDecWaves][kDPad];

    const int pos = a.pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*a.pos_dev) : a.pos;
    if (pos < 0 || pos >= a.L || pos >= kDecHeadKeys) return;
    switch (pos >> 6) {  // uniform
        case 0: decode_head_rounds<1>(a, pos, m_red, l_red, o_red); break;
        case 1: decode_head_rounds<2>(a, pos, m_red, l_red, o_red); break;
        case 2: decode_head_rounds<3>(a, pos, m_red, l_red, o_red); break;
        case 3: decode_head_rounds<4>(a, pos, m_red, l_red, o_red); break;
        case 4: decode_head_rounds<5>(a, pos, m_red, l_red, o_red); break;
        case 5: decode_head_rounds<6>(a, pos, m_red, l_red, o_red); break;
        case 6: decode_head_rounds<7>(a, pos, m_red, l_red, o_red); break;
        default: decode_head_rounds<8>(a, pos, m_red, l_red, o_red); break;
    }
}

void launch_attn_decode(const DecParams &p, hipStream_t stream) {
    if (p.full && dec_head_fits(p)) {
        attn_decode_head_kernel<<<dim3(p.B * p.H), dim3(kDecThreads), 0, stream>>>(p);
        hipCheck(hipGetLastError());
        return;
    }
    if (p.full && p.part != nullptr) {
        attn_decode_split_kernel<<<dim3(p.B * p.H * p.splits), dim3(256), 0, stream>>>(p);
        hipCheck(hipGetLastError());
        attn_decode_merge_kernel<<<dim3(p.B * p.H), dim3(kDPad), 0, stream>>>(p);
        hipCheck(hipGetLastError());
        return;
    }
    const size_t lds = static_cast<size_t>(p.pos_dev != nullptr ? p.L : p.pos + 1) * sizeof(float);
    if (p.D <= 2 * kDPad) {
        attn_decode_kernel<2 * kDPad><<<dim3(p.B * p.H), dim3(kDecThreads), lds, stream>>>(p);
    } else {
        static std::once_flag once;
        std::call_once(once, [] {
            hipCheck(hipFuncSetAttribute(reinterpret_cast<const void *>(attn_decode_kernel<kGenericMaxD>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kDecMaxKeys * sizeof(float)));
        });
        attn_decode_kernel<kGenericMaxD><<<dim3(p.B * p.H), dim3(kDecThreads), lds, stream>>>(p);
    }
    hipCheck(hipGetLastError());
}

}  // namespace gptc
