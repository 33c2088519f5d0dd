// Fused causal attention forward for gfx950: S = QK^T / sqrt(D), causal
// mask, online softmax and O = PV in one pass; writes O, the row
// log-sum-exp and, for the backward, the probabilities P' against the
// running maximum with that maximum m per 64-key tile (the layout is
// described in attn_kernels.hpp).  Replaces the permute / batched SGEMM / mask / softmax /
// batched SGEMM / unpermute sequence of gpt.c
// (kernels/src/cuda/Attention.cu:170-232; math of
// kernels/src/cpu/Attention.c:46-167).
//
// Four kernels.  For D == 64 with 16-byte rows (every GPT-2 shape) the
// 16-row kernel (attn_fwd16_kernel) runs on work lists, and short heads
// (T <= 128) run attn_fwd_short_kernel (T <= 64) or attn_fwd_twotile_kernel;
// the 32-row kernel first below serves the other head sizes up to 128.
//
// 32-row kernel: one workgroup = 4 waves = 128 queries of one (b, h); wave
// w owns 32 queries.  The products are formed transposed, S^T = K Q^T and
// O^T = V^T P^T, so that each lane owns ONE query (lane % 32) and the
// softmax row statistics are per-lane scalars: the running max needs one
// exchange with the other wave half per 64-key tile, the running sum none
// until the epilogue.  Q stays in registers as the B operand; 64-key K and
// V tiles are staged in LDS by the whole workgroup and prefetched into
// registers one tile ahead.
#include <type_traits>

#include "attn_common.hpp"
#include "attn_kernels.hpp"
#include "hip_check.hpp"

namespace gptc {

constexpr int kFwdBM = 128;  // queries per workgroup
constexpr int kFwdBN = 64;   // keys per LDS tile
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)

// DP: the head size the kernel is built for, 64 (D <= 64) or 128 (64 < D <=
// 128); a smaller D is zero-padded in registers.  DP = 128 keeps 64 more
// registers per lane and twice the LDS per tile: one workgroup per CU, one
// wave per SIMD.
template <bool VEC, int DP, bool PERM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 3 : 1, DP == 64 ? 3 : 1))) void
attn_fwd_kernel(const FwdParams a) {
    constexpr int LS = DP + 4;       // LDS row stride (floats)
    constexpr int NJ = DP / 8;       // reduction steps of 8 dims (4 per lane half)
    constexpr int NDB = DP / 32;     // 32-dim blocks of the output
    constexpr int TPR = DP / 4;      // tile-load threads per row (a float4 each)
    constexpr int RPP = 256 / TPR;   // tile rows per load pass
    constexpr int NLD = kFwdBN / RPP;  // load passes per 64-key tile
    __shared__ __attribute__((aligned(16))) float k_lds[kFwdBN * LS];
    __shared__ __attribute__((aligned(16))) float v_lds[kFwdBN * LS];

    const int tid = threadIdx.x;
    // The wave index is made visibly uniform (an SGPR): branches on it are then
    // scalar branches instead of exec-masked divergent regions around MFMAs.
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, hf = lane >> 5, l32 = lane & 31;

    // Query blocks in the XCD- and CU-aware order of grid_order.hpp.
    int blk, bh;
    grid_position(a.order, a.nqb, a.bh_pad, blk, bh);
    if (bh >= a.B * a.H) return;
    const int qb = a.nqb - 1 - blk;
    const int b = bh / a.H, h = bh - b * a.H;
    const int T = a.T, D = a.D;

    const int q_blk0 = qb * kFwdBM;
    const int qw0 = q_blk0 + 32 * w;
    const int my_q = qw0 + l32;

    const float *Qh = a.q.p + b * a.q.sb + h * a.q.sh;
    const float *Kh = a.k.p + b * a.k.sb + h * a.k.sh;
    const float *Vh = a.v.p + b * a.v.sb + h * a.v.sh;

    // Q row of this lane's query, dims 8j + 4hf + c, as B operands.
    f32x4 qr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        qr[j] = (my_q < T) ? load4<VEC>(Qh + my_q * a.q.st, 8 * j + 4 * hf, D) : zero4();
    if (PERM && my_q < T) {
        float *dst = a.qp + (static_cast<uint32_t>(bh) * T + my_q) * D;
#pragma unroll
        for (int j = 0; j < NJ; ++j) store4<VEC>(dst, 8 * j + 4 * hf, D, qr[j]);
    }

    const int kv_end = min(T, q_blk0 + kFwdBM);
    const int n_tiles = (kv_end + kFwdBN - 1) / kFwdBN;

    // Cooperative tile load: thread covers rows tid / TPR + RPP i, dims 4 (tid % TPR).
    const int ld_row = tid / TPR, ld_col = 4 * (tid % TPR);
    f32x4 kpre[NLD], vpre[NLD];
    auto prefetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int key = kt * kFwdBN + ld_row + RPP * i;
            kpre[i] = (key < T) ? load4<VEC>(Kh + key * a.k.st, ld_col, D) : zero4();
            vpre[i] = (key < T) ? load4<VEC>(Vh + key * a.v.st, ld_col, D) : zero4();
        }
    };
    prefetch(0);

    const float c2 = a.scale_log2;
    float m_run = -INFINITY;  // running max of s * c2 for this lane's query
    float l_run = 0.0f;       // this half-wave's share of the running sum
    f32x16 acc_o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc_o[db] = zero16();

    for (int kt = 0; kt < n_tiles; ++kt) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int row = ld_row + RPP * i;
            *reinterpret_cast<f32x4 *>(&k_lds[row * LS + ld_col]) = kpre[i];
            *reinterpret_cast<f32x4 *>(&v_lds[row * LS + ld_col]) = vpre[i];
        }
        if (PERM && kt * kFwdBN >= q_blk0) {
            // Keys of this workgroup's own block: emit the permuted copies.
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const int key = kt * kFwdBN + ld_row + RPP * i;
                if (key < T) {
                    const uint32_t off = (static_cast<uint32_t>(bh) * T + key) * D;
                    store4<VEC>(a.kp + off, ld_col, D, kpre[i]);
                    store4<VEC>(a.vp + off, ld_col, D, vpre[i]);
                }
            }
        }
        __syncthreads();
        if (kt + 1 < n_tiles) prefetch(kt + 1);

        const int k0 = kt * kFwdBN;
        if (k0 > qw0 + 31 || qw0 >= T) continue;  // wave-uniform: tile entirely masked

        // S^T (keys x queries) for two 32-key blocks.
        f32x16 s[2] = {zero16(), zero16()};
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const f32x4 ka = *reinterpret_cast<const f32x4 *>(&k_lds[l32 * LS + 8 * j + 4 * hf]);
            const f32x4 kb = *reinterpret_cast<const f32x4 *>(&k_lds[(32 + l32) * LS + 8 * j + 4 * hf]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                s[0] = mfma32(ka[c], qr[j][c], s[0]);
                s[1] = mfma32(kb[c], qr[j][c], s[1]);
            }
        }

        if (k0 + kFwdBN - 1 > qw0) {  // tile crosses this wave's diagonal
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 32 * kb + 8 * (r >> 2) + 4 * hf + (r & 3);
                    if (key > my_q) s[kb][r] = -INFINITY;
                }
        }

        // Row max of this tile: 4 independent chains, then the other wave half.
        float mx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) mx[i] = fmaxf(s[i >> 1][(i & 1) * 8], s[i >> 1][(i & 1) * 8 + 1]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 2; r < 8; ++r) mx[i] = fmaxf(mx[i], s[i >> 1][(i & 1) * 8 + r]);
        float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
        mt = fmaxf(mt, other_half(mt)) * c2;

        // Lazy rescaling: the running max only moves when some row's max grows
        // by more than 2^kRescaleLog2 (or on the first tile).  In between, the
        // exponents are taken against a stale max, so p <= 2^kRescaleLog2,
        // which fp32 holds exactly as well; the final y = acc / l is the same.
        if (__builtin_amdgcn_ballot_w64(mt > m_run + kRescaleLog2) != 0) {
            const float m_new = fmaxf(m_run, mt);
            const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
            const float alpha = fast_exp2(m_run - m_use);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc_o[db][r] *= alpha;
            m_run = m_new;
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(fmaf(s[kb][r], c2, -m_use));
                s[kb][r] = p;
                ls[r & 3] += p;
            }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);

        // Hand P' = p and m_use to the backward: this lane's query row of the
        // packed blocks (qt, 2kt) and (qt, 2kt + 1), keys 8g + 4hf .. 8g + 4hf + 3.
        // kt <= qt here, so both blocks exist; masked keys hold exact zeros.
        {
            float *pblk = a.pp + ds_block_offset(bh, a.nqt, qw0 >> 6, 2 * kt);  // uniform
            const uint32_t prow = ((qw0 & 32) + l32) * 32 + 4 * hf;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 v = {s[kb][4 * g], s[kb][4 * g + 1], s[kb][4 * g + 2], s[kb][4 * g + 3]};
                    stream_store(reinterpret_cast<f32x4 *>(pblk + kb * kDsBlock + prow + 8 * g), v);
                }
            if (hf == 0 && my_q < T) a.pm[(static_cast<uint32_t>(bh) * a.nqt + kt) * T + my_q] = m_use;
        }

        // O^T (dims x queries) += V^T P^T; P^T register 4g+c is the B operand.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int row = 32 * kb + 8 * g + 4 * hf + c;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
                        acc_o[db] = mfma32(v_lds[row * LS + 32 * db + l32], s[kb][4 * g + c], acc_o[db]);
                }
    }

    if (qw0 >= T) return;
    const float l_tot = l_run + other_half(l_run);
    if (my_q >= T) return;
    const float inv = 1.0f / l_tot;
    float *orow = a.o.p + b * a.o.sb + my_q * a.o.st + h * a.o.sh;
    float *o2row = a.o2 ? a.o2 + b * a.o.sb + my_q * a.o.st + h * a.o.sh : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 val;
#pragma unroll
            for (int c = 0; c < 4; ++c) val[c] = acc_o[db][4 * g + c] * inv;
            const int dim = 32 * db + 8 * g + 4 * hf;
            store4<VEC>(orow, dim, D, val);
            if (o2row) store4<VEC>(o2row, dim, D, val);
        }
    if (hf == 0) a.lse[static_cast<uint32_t>(bh) * T + my_q] = (m_run + log2f(l_tot)) * kLn2;
}

// ---- Per-tile math of the 16-row forwards ----
//
// One wave, 16 queries (lane (g, i16): query i16, keys 4g .. 4g+3 of each
// 16-key block), one 64-key tile staged in LDS (rows of kLdsStride floats):
// NKB of its 16-key blocks are visible (DIAG: the tile holding the block's
// own keys, where block NKB - 1 is masked per key).
//
// Scores: S^T = K Q^T on 16 x 16 x 4 (Q^T in registers, qr[c][e] = Q[my_q]
// [16c + 4g + e]), the tile's row maximum (log2 units), the online softmax
// with lazy rescaling (the running maximum moves only when a row maximum
// grows by more than 2^kRescaleLog2), P' = exp2(S c2 - m_use) into sc and its
// row sums into l_run.  Returns m_use (0 while the row is all masked).
// The K operands come from k_op(kb, c): K[16kb + i16][16g + 4c .. +3] of the
// tile (an LDS read, or registers the caller loaded).
template <int NKB, bool DIAG, typename KOp>
__device__ __forceinline__ float fwd16_scores_op(KOp k_op, const f32x4 (&qr)[4], int g, int i16, float c2,
                                                 float &m_run, float &l_run, f32x4 (&acc)[4], f32x4 (&sc)[4]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sc[kb] = zero4();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        f32x4 ka[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) ka[kb] = k_op(kb, c);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) sc[kb] = mfma16(ka[kb][e], qr[c][e], sc[kb]);
    }
    if (DIAG) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r > i16) sc[NKB - 1][r] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) mx = fmaxf(mx, fmaxf(fmaxf(sc[kb][0], sc[kb][1]), fmaxf(sc[kb][2], sc[kb][3])));
    const float mt = max4_rows(mx) * c2;

    if (__builtin_amdgcn_ballot_w64(mt > m_run + kRescaleLog2) != 0) {
        const float m_new = fmaxf(m_run, mt);
        const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
        m_run = m_new;
    }
    const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
    float ls[2] = {0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float p = fast_exp2(fmaf(sc[kb][r], c2, -m_use));
            sc[kb][r] = p;
            ls[r & 1] += p;
        }
    l_run += ls[0] + ls[1];
    return m_use;
}

// LDS tiles of the 16-row forwards (64 keys x 64 dims each, no padding):
//   K: the 16-byte chunk d / 4 of key k sits at chunk (d / 4) ^ (k % 16) of
//     row k.  Lane group g of score step c reads dims 16c + 4g .. +3 of key
//     i16 (the Q operands use the same dims), i.e. chunk (4c + g) ^ i16;
//     a tile store (lanes 0..15 one row, one chunk each) writes one row's
//     16 chunks in permuted order;
//   V: row-major: lane (g, i16) reads row 4g + r at dims 4 i16, 256
//     contiguous bytes per group, the groups 1 KB apart.
// Measured with SQ_LDS_BANK_CONFLICT on gfx950 (an access-pattern probe of
// each read and store): these four accesses show no bank conflicts.  The
// rows of 68 floats used before, with dims 16g + 4c for lane group g,
// conflicted on both reads (half of the forward's LDS-active cycles), and
// so did K rows of 68 or 76 floats with dims 16c + 4g, and the XOR layout
// with dims 16g + 4c.
constexpr int kKStride = kDPad;
constexpr int kVStride = kDPad;
__device__ __forceinline__ int ktile_at(int key, int dim) {
    return key * kKStride + ((((dim >> 2) ^ (key & 15)) << 2) | (dim & 3));
}
__device__ __forceinline__ int vtile_at(int key, int dim) { return key * kVStride + dim; }

template <int NKB, bool DIAG>
__device__ __forceinline__ float fwd16_scores(const float *k_t, const f32x4 (&qr)[4], int g, int i16, float c2,
                                              float &m_run, float &l_run, f32x4 (&acc)[4], f32x4 (&sc)[4]) {
    return fwd16_scores_op<NKB, DIAG>(
        [&](int kb, int c) { return *reinterpret_cast<const f32x4 *>(&k_t[ktile_at(16 * kb + i16, 16 * c + 4 * g)]); },
        qr, g, i16, c2, m_run, l_run, acc, sc);
}

// O^T += V^T P^T: step (kb, r) reduces keys 16kb + 4g' + r; lane i16's A
// operands for the four dim blocks are V[key][4 i16 .. 4 i16 + 3] (one
// 16-byte LDS read), and acc[db][r] = O[my_q][16g + 4r + db].
// The V operands come from v_op(kb, r): V[16kb + 4g + r][4 i16 .. +3].
template <int NKB, typename VOp>
__device__ __forceinline__ void fwd16_pv_op(VOp v_op, const f32x4 (&sc)[4], f32x4 (&acc)[4]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f32x4 va = v_op(kb, r);
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = mfma16(va[db], sc[kb][r], acc[db]);
        }
}

template <int NKB>
__device__ __forceinline__ void fwd16_pv(const float *v_t, const f32x4 (&sc)[4], int g, int i16, f32x4 (&acc)[4]) {
    fwd16_pv_op<NKB>(
        [&](int kb, int r) { return *reinterpret_cast<const f32x4 *>(&v_t[vtile_at(16 * kb + 4 * g + r, 4 * i16)]); },
        sc, acc);
}

// ---- The 16-row forward (D == 64, buffer-resource loads) ----
//
// One workgroup = 4 waves runs the 64-query blocks of its work list
// (block_sched.hpp) one after the other; block j of head bh reduces key
// tiles 0 .. j.  The lists give every CU the same work (at B=8, H=12,
// T=1024: blocks j and 15-j of one head per workgroup, all 768 workgroups
// resident at once).  The key tiles of consecutive steps are prefetched
// into registers one step ahead, across block and head boundaries.
// Wave w owns queries 16w .. 16w+15 of the block; lane (g = lane/16,
// i = lane%16) owns query i of them and, of every 16-key block, keys
// 4g .. 4g+3 (the 16 x 16 x 4 accumulator layout of attn_common.hpp).  The
// products are formed transposed as in the kernel above: S^T = K Q^T with
// Q^T in registers, O^T = V^T P^T with P^T straight from the S accumulators.
// Output row m of O^T block db is dim 4m + db, so that one 16-byte LDS read
// of a V row gives a lane the A operands of all four blocks.  P' and m go
// out in the same packed layout, so the backward is unchanged.
//
// DEEP (short sequences, where each workgroup runs one block of at most a
// few tiles and latency dominates): tiles are prefetched two steps ahead,
// so that a two-tile block issues all of its loads before its first wait.
constexpr int kF16Rows = 64;  // queries per block of the 16-row kernel (4 waves x 16)

template <bool PERM, bool DEEP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DEEP ? 2 : 3, DEEP ? 2 : 3))) void
attn_fwd16_kernel(const FwdParams a) {
    __shared__ __attribute__((aligned(16))) float k_lds[kFwdBN * kKStride];
    __shared__ __attribute__((aligned(16))) float v_lds[kFwdBN * kVStride];
    // The qkv bias of the current step's head (q | k | v, 64 floats each).
    __shared__ __attribute__((aligned(16))) float bias_lds[3 * kDPad];

    // The pool's item for the prefetch cursor's next block (see below).
    __shared__ int pool_lds;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, g = lane >> 4, i16 = lane & 15;
    // The pool (block_sched.hpp): blocks that no list holds, taken one at a
    // time by the workgroups whose lists are done.
    const bool use_pool = !DEEP && !PERM && a.sched.pool_n > 0;
    // Thread 0 counts the workgroup done; the last one resets the counters.
    auto pool_done = [&]() {
        if (use_pool && tid == 0) {
            const int d = __hip_atomic_fetch_add(a.sched.counters + 64, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == static_cast<int>(gridDim.x) - 1) {
                __hip_atomic_store(a.sched.counters, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(a.sched.counters + 64, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    };
    const int it_end = a.sched.wg_start[blockIdx.x + 1];
    int it = a.sched.wg_start[blockIdx.x];
    if (it >= it_end) {
        pool_done();
        return;
    }
    const int T = a.T, nqt = a.nqt;

    // Cooperative tile load: thread covers rows (tid>>4) + 16i, dims 4*(tid&15).
    // Rows past T read as zeros (buffer resources over the head's T rows).
    const int ld_row = tid >> 4, ld_col = 4 * (tid & 15);
    // The qkv Linear's bias is added here (compact layout only: never with PERM).
    const bool biased = !PERM && a.kb != nullptr;
    f32x4 kpre[4], vpre[4];
    f32x4 kpre2[4], vpre2[4];  // DEEP: the step after the prefetched one
    // Threads 0..47 carry one float4 of the q | k | v bias of the head of the
    // tile in kpre (bpre) and in kpre2 (bpre2, DEEP): loaded with the tile,
    // written to bias_lds at the start of the step that stores the tile, and
    // added there (K, V) and to the block's Q rows (qr) after the step's
    // second barrier.
    const bool bias_lane = biased && tid < 3 * kDPad / 4;
    const float *bias_src = tid < kDPad / 4 ? a.qb : tid < kDPad / 2 ? a.kb : a.vb;
    const int bias_dim = 4 * (tid & 15);
    f32x4 bpre = zero4(), bpre2 = zero4();
    auto load_tile = [&](int hbh, int kt, f32x4(&kd)[4], f32x4(&vd)[4], f32x4 &bd) {
        const int hb = hbh / a.H, hh = hbh - hb * a.H;
        const auto k_rows = head_rows(a.k.p + hb * a.k.sb + hh * a.k.sh, T, a.k.st);
        const auto v_rows = head_rows(a.v.p + hb * a.v.sb + hh * a.v.sh, T, a.v.st);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = kt * kFwdBN + ld_row + 16 * i;
            kd[i] = buffer_load4(k_rows, key * a.k.st + ld_col);
            vd[i] = buffer_load4(v_rows, key * a.v.st + ld_col);
        }
        if (bias_lane) bd = *reinterpret_cast<const f32x4 *>(bias_src + hh * kDPad + bias_dim);
    };
    // The step after (sit, skt) of block sj: the next tile of the block, or
    // tile 0 of the next block of the list, or of the pool's block pool_item
    // once the list is done (sit == it_end).  False at the end.
    int pool_item = -1;  // uniform: the pool block published for the prefetch cursor
    auto advance = [&](int &sit, int &skt, int &sbh, int &sj) {
        if (skt < sj) {
            ++skt;
            return true;
        }
        if (sit + 1 < it_end) {
            ++sit;
            const int item = load_uniform_int(uniform(a.sched.items + sit));
            sbh = sched_bh(item);
            sj = sched_j(item);
            skt = 0;
            return true;
        }
        sit = it_end;
        if (pool_item < 0) return false;
        sbh = sched_bh(pool_item);
        sj = sched_j(pool_item);
        skt = 0;
        return true;
    };
    // The pool index for the block after the prefetch cursor's is taken one
    // step ahead, when that cursor reaches the last tile of the last block it
    // has: thread 0's atomic (`grab`), published through pool_lds before the
    // next step's first barrier and read between its two barriers, so the
    // cursor has it when it moves on after the second.
    // Wave 0 takes the index as a whole so that no branch here is divergent
    // (a lane-0 branch made the compiler keep the cursors in vector
    // registers, with spills): lane 0 adds 1 to counters[0], lanes 1..63 add
    // 0 to counters[1..63], so the 64 device-scope atomics fall in one cache
    // line (all 64 on counters[0] cost about 2 us per forward at C2).
    bool grab = false;  // uniform
    int grab_idx = 0;   // wave 0's (lane 0's result)
    auto take_pool_index = [&](int sit, int skt, int sj) {
        grab = use_pool && skt == sj && sit + 1 >= it_end;
        if (grab && w == 0)
            grab_idx = __hip_atomic_fetch_add(a.sched.counters + lane, lane == 0 ? 1 : 0, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    };

    // Steps (key tiles) of this workgroup's list, for the wave priority below.
    int total_steps = 0;
    for (int x = it; x < it_end; ++x) total_steps += sched_j(a.sched.items[x]) + 1;
    int done_steps = 0;
    // Current step (it, kt) of block jq of head bh.
    int kt = 0, bh = sched_bh(a.sched.items[it]), jq = sched_j(a.sched.items[it]);
    bool first_block = true;
    int b = bh / a.H, h = bh - b * a.H;
    const float c2 = a.scale_log2;
    f32x4 qr[4];  // Q[my_q][16c + 4g + e] in qr[c][e]: the B operand of step 4c + e
    auto load_q = [&]() {
        const auto q_rows = head_rows(a.q.p + b * a.q.sb + h * a.q.sh, T, a.q.st);
        const int q = jq * kF16Rows + 16 * w + i16;
#pragma unroll
        for (int c = 0; c < 4; ++c) qr[c] = buffer_load4(q_rows, static_cast<uint32_t>(q) * a.q.st + 16 * c + 4 * g);
    };
    load_q();
    load_tile(bh, 0, kpre, vpre, bpre);
    // Prefetch cursor: the step whose tile sits in kpre2 (DEEP) or is loaded
    // next; without DEEP the current step follows it.
    int pit = it, pkt = 0, pbh = bh, pj = jq;
    bool pre_ok = advance(pit, pkt, pbh, pj);
    if (DEEP && pre_ok) load_tile(pbh, pkt, kpre2, vpre2, bpre2);
    if (pre_ok) take_pool_index(pit, pkt, pj);

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc[4];  // O^T: acc[db][r] = O[my_q][16g + 4r + db] before the 1/l scaling
    int my_q = 0;

    // One key tile for this wave: NKB 16-key blocks of it are visible to the
    // wave's queries (DIAG: the tile holding the block's own keys, where block
    // NKB - 1 is masked per key and blocks NKB .. 3 are all masked).
    auto tile = [&](auto nkb_c, auto diag_c) {
        constexpr int NKB = decltype(nkb_c)::value;
        constexpr bool DIAG = decltype(diag_c)::value;
        f32x4 sc[4];
        const float m_use = fwd16_scores<NKB, DIAG>(k_lds, qr, g, i16, c2, m_run, l_run, acc, sc);

        // P' rows of block (jq, key blocks 2kt and 2kt + 1), zeros past the
        // diagonal; m of this tile (not for short heads, whose backward
        // recomputes P: pp == nullptr).
        if (a.pp != nullptr) {
            float *ptile = a.pp + ds_block_offset(bh, nqt, jq, 2 * kt);  // uniform
            const uint32_t prow = (16 * w + i16) * 32 + 4 * g;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                stream_store(reinterpret_cast<f32x4 *>(ptile + (kb >> 1) * kDsBlock + prow + 16 * (kb & 1)),
                             kb < NKB ? sc[kb] : zero4());
            if (g == 0 && my_q < T) a.pm[(static_cast<uint32_t>(bh) * nqt + kt) * T + my_q] = m_use;
        }
        fwd16_pv<NKB>(v_lds, sc, g, i16, acc);
    };

    for (;;) {
        my_q = jq * kF16Rows + 16 * w + i16;
        if (kt == 0) {
            // A new block: fresh statistics (its Q rows are loaded already
            // for the first block, here for the others).
            if (!first_block) load_q();
            first_block = false;
            if (PERM && my_q < T) {
                float *dst = a.qp + (static_cast<uint32_t>(bh) * T + my_q) * kDPad + 4 * g;
#pragma unroll
                for (int c = 0; c < 4; ++c) *reinterpret_cast<f32x4 *>(dst + 16 * c) = qr[c];
            }
            m_run = -INFINITY;
            l_run = 0.0f;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = zero4();
        }

        // Wave priority from the share of the list still to run (4 levels):
        // the SIMDs otherwise issue from the oldest waves first, so the first
        // workgroup of a CU runs ahead and the last runs alone at the end;
        // workgroups that fall behind now win the MFMA pipe and catch up
        // (C2 forward 133.8 -> 131.0 us, C5 139.8 -> 137.0 us).  The levels
        // change when 40 %, 20 % and 7 % of the list remain: within a level
        // the oldest workgroup still runs first, so the last levels are the
        // short ones (the three workgroups of a CU then end closer together;
        // C2 127.0 against 128.2 us with quarters).
        if (!DEEP) {
            const int rem100 = 100 * (total_steps - done_steps);  // wave-uniform
            if (rem100 > 40 * total_steps)
                __builtin_amdgcn_s_setprio(3);
            else if (rem100 > 20 * total_steps)
                __builtin_amdgcn_s_setprio(2);
            else if (rem100 > 7 * total_steps)
                __builtin_amdgcn_s_setprio(1);
            else
                __builtin_amdgcn_s_setprio(0);
            ++done_steps;
        }
        // The bias of this step's head; the previous step's readers of
        // bias_lds are past its second barrier.  Likewise the pool index
        // taken during the previous step (its readers too).
        if (bias_lane) *reinterpret_cast<f32x4 *>(&bias_lds[4 * tid]) = bpre;
        if (grab && w == 0) {
            const int r = __builtin_amdgcn_readfirstlane(grab_idx);
            if (lane == 0)
                pool_lds = r < a.sched.pool_n
                               ? ((a.sched.pool_bh0 + r % a.sched.pool_bh) << kSchedJBits) |
                                     (a.sched.pool_j0 - 1 - r / a.sched.pool_bh)
                               : -1;
        }
        __syncthreads();
        if (grab) pool_item = __builtin_amdgcn_readfirstlane(pool_lds);
        if (biased) {
            // Rows past T read as zeros and then hold the bias: they only
            // occur in a block's diagonal tile, beyond the diagonal of every
            // query < T (masked), and rows of queries past T are not written.
            const f32x4 kb4 = *reinterpret_cast<const f32x4 *>(&bias_lds[kDPad + ld_col]);
            const f32x4 vb4 = *reinterpret_cast<const f32x4 *>(&bias_lds[2 * kDPad + ld_col]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kpre[i] += kb4;
                vpre[i] += vb4;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<f32x4 *>(&k_lds[ktile_at(ld_row + 16 * i, ld_col)]) = kpre[i];
            *reinterpret_cast<f32x4 *>(&v_lds[vtile_at(ld_row + 16 * i, ld_col)]) = vpre[i];
        }
        const bool diag = kt == jq;  // the block's own keys: the last tile of the block
        if (PERM && diag) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = kt * kFwdBN + ld_row + 16 * i;
                if (key < T) {
                    const uint32_t off = (static_cast<uint32_t>(bh) * T + key) * kDPad + ld_col;
                    *reinterpret_cast<f32x4 *>(a.kp + off) = kpre[i];
                    *reinterpret_cast<f32x4 *>(a.vp + off) = vpre[i];
                }
            }
        }
        __syncthreads();
        // Refill the prefetch registers with the next step's tile.  DEEP: it
        // is in flight already (kpre2); it moves up after this step's tile,
        // so that this tile's compute does not wait for its loads.
        const bool has_next = pre_ok;
        const int n_kt = pkt, n_bh = pbh, n_j = pj;  // without DEEP: the next step
        if (!DEEP && pre_ok) {
            load_tile(pbh, pkt, kpre, vpre, bpre);
            pre_ok = advance(pit, pkt, pbh, pj);
            grab = false;
            if (pre_ok) take_pool_index(pit, pkt, pj);
        }
        if (biased && kt == 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c) qr[c] += *reinterpret_cast<const f32x4 *>(&bias_lds[16 * c + 4 * g]);
        }

        if (!diag) {
            tile(IntC<4>{}, std::false_type{});
        } else {
            switch (w) {  // wave-uniform
                case 0: tile(IntC<1>{}, std::true_type{}); break;
                case 1: tile(IntC<2>{}, std::true_type{}); break;
                case 2: tile(IntC<3>{}, std::true_type{}); break;
                default: tile(IntC<4>{}, std::true_type{}); break;
            }
            // End of the block: y = O / l and the log-sum-exp.
            const float lt = sum4_rows(l_run);
            if (my_q < T) {
                const float inv = 1.0f / lt;
                float *orow = a.o.p + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g;
                float *o2row = a.o2 ? a.o2 + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g : nullptr;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const f32x4 val = {acc[0][r] * inv, acc[1][r] * inv, acc[2][r] * inv, acc[3][r] * inv};
                    *reinterpret_cast<f32x4 *>(orow + 4 * r) = val;
                    if (o2row) *reinterpret_cast<f32x4 *>(o2row + 4 * r) = val;
                }
                if (g == 0) a.lse[static_cast<uint32_t>(bh) * T + my_q] = (m_run + log2f(lt)) * kLn2;
            }
        }
        if (DEEP && pre_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kpre[i] = kpre2[i];
                vpre[i] = vpre2[i];
            }
            bpre = bpre2;
            pre_ok = advance(pit, pkt, pbh, pj);
            if (pre_ok) load_tile(pbh, pkt, kpre2, vpre2, bpre2);
        }
        if (DEEP) {
            if (!advance(it, kt, bh, jq)) break;
        } else {
            if (!has_next) break;
            kt = n_kt;
            bh = n_bh;
            jq = n_j;
        }
        b = bh / a.H;
        h = bh - b * a.H;
    }
    pool_done();
}

// ---- Short heads (T <= 128, D == 64, compact layout) ----
//
// One workgroup per 64-query block (at most two key tiles), the blocks with
// two tiles first; the (head, block) pair comes from blockIdx alone, so the
// first loads issue without waiting for a work list.  Q, every key tile of
// the block and the bias go out at once; both K/V tiles are staged behind
// one barrier, and the waves then run the tiles back to back (the same
// per-tile math as the kernel above).  The backward of short heads
// recomputes P, so no P' or m is stored.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_fwd_short_kernel(const FwdParams a) {
    constexpr int KTILE = kFwdBN * kKStride, VTILE = kFwdBN * kVStride;
    __shared__ __attribute__((aligned(16))) float k_lds[kShortHeadTiles * KTILE];
    __shared__ __attribute__((aligned(16))) float v_lds[kShortHeadTiles * VTILE];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, g = lane >> 4, i16 = lane & 15;
    const int BH = a.B * a.H, T = a.T;
    const int r = static_cast<int>(blockIdx.x) / BH;
    const int bh = static_cast<int>(blockIdx.x) - r * BH;
    const int jq = a.nqt - 1 - r;  // grid = BH * nqt, so 0 <= jq < nqt
    const int b = bh / a.H, h = bh - b * a.H;
    const int my_q = jq * kF16Rows + 16 * w + i16;

    // Rows past T read as zeros (buffer resources over the head's T rows).
    const auto q_rows = head_rows(a.q.p + b * a.q.sb + h * a.q.sh, T, a.q.st);
    const auto k_rows = head_rows(a.k.p + b * a.k.sb + h * a.k.sh, T, a.k.st);
    const auto v_rows = head_rows(a.v.p + b * a.v.sb + h * a.v.sh, T, a.v.st);
    f32x4 qr[4];  // Q[my_q][16c + 4g + e] in qr[c][e]
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] = buffer_load4(q_rows, static_cast<uint32_t>(my_q) * a.q.st + 16 * c + 4 * g);
    const int ld_row = tid >> 4, ld_col = 4 * (tid & 15);
    f32x4 kpre[kShortHeadTiles][4], vpre[kShortHeadTiles][4];
#pragma unroll
    for (int kt = 0; kt < kShortHeadTiles; ++kt)
        if (kt <= jq) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t key = kt * kFwdBN + ld_row + 16 * i;
                kpre[kt][i] = buffer_load4(k_rows, key * a.k.st + ld_col);
                vpre[kt][i] = buffer_load4(v_rows, key * a.v.st + ld_col);
            }
        }
    // The qkv Linear's bias, read by every thread for its own columns.  Key
    // rows past T then hold the bias: they only occur past the diagonal of
    // every query < T (masked), and rows of queries past T are not written.
    const bool biased = a.kb != nullptr;
    f32x4 kb4 = zero4(), vb4 = zero4(), qb4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) qb4[c] = zero4();
    if (biased) {
        kb4 = *reinterpret_cast<const f32x4 *>(a.kb + h * kDPad + ld_col);
        vb4 = *reinterpret_cast<const f32x4 *>(a.vb + h * kDPad + ld_col);
#pragma unroll
        for (int c = 0; c < 4; ++c) qb4[c] = *reinterpret_cast<const f32x4 *>(a.qb + h * kDPad + 16 * c + 4 * g);
    }
#pragma unroll
    for (int kt = 0; kt < kShortHeadTiles; ++kt)
        if (kt <= jq) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *reinterpret_cast<f32x4 *>(&k_lds[kt * KTILE + ktile_at(ld_row + 16 * i, ld_col)]) = kpre[kt][i] + kb4;
                *reinterpret_cast<f32x4 *>(&v_lds[kt * VTILE + vtile_at(ld_row + 16 * i, ld_col)]) = vpre[kt][i] + vb4;
            }
        }
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] += qb4[c];
    __syncthreads();

    const float c2 = a.scale_log2;
    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = zero4();
    f32x4 sc[4];
    if (jq > 0) {  // a full tile before the diagonal one (kShortHeadTiles == 2)
        fwd16_scores<4, false>(k_lds, qr, g, i16, c2, m_run, l_run, acc, sc);
        fwd16_pv<4>(v_lds, sc, g, i16, acc);
    }
    const float *k_d = k_lds + jq * KTILE, *v_d = v_lds + jq * VTILE;
    switch (w) {  // wave-uniform: the 16-key blocks of the diagonal tile this wave sees
        case 0: fwd16_scores<1, true>(k_d, qr, g, i16, c2, m_run, l_run, acc, sc); fwd16_pv<1>(v_d, sc, g, i16, acc); break;
        case 1: fwd16_scores<2, true>(k_d, qr, g, i16, c2, m_run, l_run, acc, sc); fwd16_pv<2>(v_d, sc, g, i16, acc); break;
        case 2: fwd16_scores<3, true>(k_d, qr, g, i16, c2, m_run, l_run, acc, sc); fwd16_pv<3>(v_d, sc, g, i16, acc); break;
        default: fwd16_scores<4, true>(k_d, qr, g, i16, c2, m_run, l_run, acc, sc); fwd16_pv<4>(v_d, sc, g, i16, acc); break;
    }

    // y = O / l and the log-sum-exp.
    const float lt = sum4_rows(l_run);
    if (my_q < T) {
        const float inv = 1.0f / lt;
        float *orow = a.o.p + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g;
        float *o2row = a.o2 ? a.o2 + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g : nullptr;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const f32x4 val = {acc[0][rr] * inv, acc[1][rr] * inv, acc[2][rr] * inv, acc[3][rr] * inv};
            *reinterpret_cast<f32x4 *>(orow + 4 * rr) = val;
            if (o2row) *reinterpret_cast<f32x4 *>(o2row + 4 * rr) = val;
        }
        if (g == 0) a.lse[static_cast<uint32_t>(bh) * T + my_q] = (m_run + log2f(lt)) * kLn2;
    }
}

// ---- Two-tile heads (64 < T <= 128, D == 64, compact layout) ----
//
// A head of two 64-query blocks is 36 units of MFMA work, a unit being one
// 16-query slab against one 16-key block: slab (j, s) (queries 64j + 16s ..
// 64j + 16s + 15) sees key blocks 0 .. 4j + s, the last of them its
// diagonal, so the second block's slabs carry 5 .. 8 units and the first
// block's 1 .. 4.  Every slab is cut into pieces of at most 2 consecutive key
// blocks, one piece per wave: 20 pieces, five workgroups per head, and no
// wave carries more than 2 units (64 MFMAs), so that a SIMD of a CU holding
// two workgroups carries at most 4.  A wave loads the K and V rows of its
// piece straight into the registers it uses them from (no staging through
// LDS, no barrier before the compute), and the pieces of a slab (all in one
// workgroup) merge their partial softmax states (running max, sums, O)
// through LDS after the workgroup's one barrier, in a fixed order, on the
// wave holding the slab's diagonal block.
//   role 0: slab (1,3) [blocks 0-1 | 2-3 | 4-5 | 6-7]
//   role 1: slab (1,2) [0-1 | 2-3 | 4-5 | 6]
//   role 2: slabs (1,1) [0-1 | 2-3 | 4-5] and (0,0) [0]
//   role 3: slabs (1,0) [0-1 | 2-3 | 4] and (0,1) [0-1]
//   role 4: slabs (0,3) [0-1 | 2-3] and (0,2) [0-1 | 2]
struct SlabState {
    float m_run, l_run;
    f32x4 acc[4];
};

constexpr int kTwoTileRoles = 5;  // workgroups per head

// BIAS: the qkv bias is added to the loaded rows (a.qb, a.kb, a.vb set); a
// separate build, so that the other keeps no registers for it.
template <bool BIAS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_fwd_twotile_kernel(const FwdParams a) {
    __shared__ __attribute__((aligned(16))) f32x4 part_lds[3][5][64];  // [partial][acc0..3, {m, l}][lane]

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, g = lane >> 4, i16 = lane & 15;
    const int BH = a.B * a.H, T = a.T;
    const int role = static_cast<int>(blockIdx.x) / BH;  // grid = kTwoTileRoles * BH
    const int bh = static_cast<int>(blockIdx.x) - role * BH;
    const int b = bh / a.H, h = bh - b * a.H;

    const auto q_rows = head_rows(a.q.p + b * a.q.sb + h * a.q.sh, T, a.q.st);
    const auto k_rows = head_rows(a.k.p + b * a.k.sb + h * a.k.sh, T, a.k.st);
    const auto v_rows = head_rows(a.v.p + b * a.v.sb + h * a.v.sh, T, a.v.st);
    // This wave's slab (block j, slab s).
    const int job = 4 * role + w;  // wave-uniform
    constexpr int kJobSlab[20][2] = {{1, 3}, {1, 3}, {1, 3}, {1, 3}, {1, 2}, {1, 2}, {1, 2}, {1, 2}, {1, 1}, {1, 1},
                                     {1, 1}, {0, 0}, {1, 0}, {1, 0}, {1, 0}, {0, 1}, {0, 3}, {0, 3}, {0, 2}, {0, 2}};
    const int sj = kJobSlab[job][0], ss = kJobSlab[job][1];
    // The qkv bias: key rows past T then hold the bias; they are masked for
    // every query < T, and rows of queries past T are not written.
    constexpr bool biased = BIAS;
    // The Q rows and bias are requested here and added in piece(), after
    // the K and V requests, so that no wait comes before those are issued.
    f32x4 qr[4], qb4[4];
    {
        const int q = sj * kF16Rows + 16 * ss + i16;
#pragma unroll
        for (int c = 0; c < 4; ++c) qr[c] = buffer_load4(q_rows, static_cast<uint32_t>(q) * a.q.st + 16 * c + 4 * g);
        if (biased) {
#pragma unroll
            for (int c = 0; c < 4; ++c) qb4[c] = *reinterpret_cast<const f32x4 *>(a.qb + h * kDPad + 16 * c + 4 * g);
        }
    }

    const float c2 = a.scale_log2;
    SlabState st;
    st.m_run = -INFINITY;
    st.l_run = 0.0f;
#pragma unroll
    for (int db = 0; db < 4; ++db) st.acc[db] = zero4();
    f32x4 sc[4];
    // Key blocks KB0 .. KB0 + NKB - 1 of the wave's slab (DIAG: the last is the
    // slab's diagonal block, masked per key), their K and V rows loaded here:
    // kr[kb][c] = K[16(KB0 + kb) + i16][16c + 4g ..], vr[kb][r] = V[16(KB0 + kb) + 4g + r][4 i16 ..].
    // Step (c, e) of the scores reduces dim 16c + 4g + e on lane group g (Q
    // likewise): any one-to-one map of the dims gives the same products, and
    // this one makes each K load 64 contiguous bytes of a row per lane group.
    auto piece = [&](auto kb0_c, auto nkb_c, auto diag_c) {
        constexpr int KB0 = decltype(kb0_c)::value, NKB = decltype(nkb_c)::value;
        constexpr bool DIAG = decltype(diag_c)::value;
        f32x4 kr[NKB][4], vr[NKB][4];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t kk = 16 * (KB0 + kb) + i16, vk = 16 * (KB0 + kb) + 4 * g + c;
                kr[kb][c] = buffer_load4(k_rows, kk * a.k.st + 16 * c + 4 * g);
                vr[kb][c] = buffer_load4(v_rows, vk * a.v.st + 4 * i16);
            }
        if (biased) {
            const f32x4 vb4 = *reinterpret_cast<const f32x4 *>(a.vb + h * kDPad + 4 * i16);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                qr[c] += qb4[c];
                const f32x4 kb4 = *reinterpret_cast<const f32x4 *>(a.kb + h * kDPad + 16 * c + 4 * g);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    kr[kb][c] += kb4;
                    vr[kb][c] += vb4;
                }
            }
        }
        fwd16_scores_op<NKB, DIAG>([&](int kb, int c) { return kr[kb][c]; }, qr, g, i16, c2, st.m_run, st.l_run,
                                   st.acc, sc);
        fwd16_pv_op<NKB>([&](int kb, int r) { return vr[kb][r]; }, sc, st.acc);
    };
    auto finish = [&]() {
        const int my_q = sj * kF16Rows + 16 * ss + i16;
        const float lt = sum4_rows(st.l_run);
        if (my_q < T) {
            const float inv = 1.0f / lt;
            float *orow = a.o.p + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g;
            float *o2row = a.o2 ? a.o2 + b * a.o.sb + my_q * a.o.st + h * a.o.sh + 16 * g : nullptr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const f32x4 val = {st.acc[0][r] * inv, st.acc[1][r] * inv, st.acc[2][r] * inv, st.acc[3][r] * inv};
                *reinterpret_cast<f32x4 *>(orow + 4 * r) = val;
                if (o2row) *reinterpret_cast<f32x4 *>(o2row + 4 * r) = val;
            }
            if (g == 0) a.lse[static_cast<uint32_t>(bh) * T + my_q] = (st.m_run + log2f(lt)) * kLn2;
        }
    };
    auto put_partial = [&](int slot) {
#pragma unroll
        for (int db = 0; db < 4; ++db) part_lds[slot][db][lane] = st.acc[db];
        part_lds[slot][4][lane] = f32x4{st.m_run, st.l_run, 0.0f, 0.0f};
    };
    // The state merged with partial `slot`: both running maxima are finite
    // (every piece holds at least one key each of its queries sees).
    auto merge = [&](int slot) {
        const f32x4 ml = part_lds[slot][4][lane];
        const float m = fmaxf(st.m_run, ml[0]);
        const float fa = fast_exp2(st.m_run - m), fb = fast_exp2(ml[0] - m);
        st.l_run = st.l_run * fa + ml[1] * fb;
#pragma unroll
        for (int db = 0; db < 4; ++db) st.acc[db] = st.acc[db] * fa + part_lds[slot][db][lane] * fb;
        st.m_run = m;
    };

    // Compute phase: at most 2 units per wave.
    using F = std::false_type;
    using D = std::true_type;
    switch (job) {
        case 0: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(0); break;
        case 1: piece(IntC<2>{}, IntC<2>{}, F{}); put_partial(1); break;
        case 2: piece(IntC<4>{}, IntC<2>{}, F{}); put_partial(2); break;
        case 3: piece(IntC<6>{}, IntC<2>{}, D{}); break;
        case 4: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(0); break;
        case 5: piece(IntC<2>{}, IntC<2>{}, F{}); put_partial(1); break;
        case 6: piece(IntC<4>{}, IntC<2>{}, F{}); put_partial(2); break;
        case 7: piece(IntC<6>{}, IntC<1>{}, D{}); break;
        case 8: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(0); break;
        case 9: piece(IntC<2>{}, IntC<2>{}, F{}); put_partial(1); break;
        case 10: piece(IntC<4>{}, IntC<2>{}, D{}); break;
        case 11: piece(IntC<0>{}, IntC<1>{}, D{}); finish(); break;
        case 12: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(0); break;
        case 13: piece(IntC<2>{}, IntC<2>{}, F{}); put_partial(1); break;
        case 14: piece(IntC<4>{}, IntC<1>{}, D{}); break;
        case 15: piece(IntC<0>{}, IntC<2>{}, D{}); finish(); break;
        case 16: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(0); break;
        case 17: piece(IntC<2>{}, IntC<2>{}, D{}); break;
        case 18: piece(IntC<0>{}, IntC<2>{}, F{}); put_partial(1); break;
        default: piece(IntC<2>{}, IntC<1>{}, D{}); break;
    }
    __syncthreads();
    // Merge phase: the diagonal piece of a split slab takes in the others.
    switch (job) {
        case 3:
        case 7: merge(0); merge(1); merge(2); finish(); break;
        case 10:
        case 14: merge(0); merge(1); finish(); break;
        case 17: merge(0); finish(); break;
        case 19: merge(1); finish(); break;
        default: break;
    }
}

void launch_attn_fwd(const FwdParams &p_in, hipStream_t stream, const hipEvent_t *ev) {
    FwdParams p = p_in;
    const bool perm = p.qp != nullptr;
    if (p.D > 2 * kDPad) {
        if (ev) hipCheck(hipEventRecord(ev[0], stream));
        launch_attn_fwd_generic(p, stream);
        if (ev) hipCheck(hipEventRecord(ev[1], stream));
        return;
    }
    if (p.full) {
        // Short heads leave P' to the backward; in the compact layout they
        // run one workgroup per block, in the reference layout the DEEP
        // variant of the work-list kernel (which also writes the caches).
        const bool deep = p.nqt <= kShortHeadTiles;
        if (deep) p.pp = p.pm = nullptr;
        if (deep && !perm) {
            if (ev) hipCheck(hipEventRecord(ev[0], stream));
            if (p.nqt == 2)
                if (p.kb != nullptr)
                    attn_fwd_twotile_kernel<true><<<dim3(kTwoTileRoles * p.B * p.H), dim3(256), 0, stream>>>(p);
                else
                    attn_fwd_twotile_kernel<false><<<dim3(kTwoTileRoles * p.B * p.H), dim3(256), 0, stream>>>(p);
            else
                attn_fwd_short_kernel<<<dim3(p.B * p.H * p.nqt), dim3(256), 0, stream>>>(p);
            hipCheck(hipGetLastError());
            if (ev) hipCheck(hipEventRecord(ev[1], stream));
            return;
        }
        const void *kern = deep ? (perm ? reinterpret_cast<const void *>(attn_fwd16_kernel<true, true>)
                                        : reinterpret_cast<const void *>(attn_fwd16_kernel<false, true>))
                                : (perm ? reinterpret_cast<const void *>(attn_fwd16_kernel<true, false>)
                                        : reinterpret_cast<const void *>(attn_fwd16_kernel<false, false>));
        int num_wg = 0;
        // The pool serves the compact layout's kernel only (the DEEP and PERM
        // variants keep whole lists).
        p.sched = device_block_schedule(p.B * p.H, p.nqt, kern, stream, &num_wg, 0, !deep && !perm);
        const dim3 grid(num_wg), block(256);
        if (ev) hipCheck(hipEventRecord(ev[0], stream));
        if (deep && perm)
            attn_fwd16_kernel<true, true><<<grid, block, 0, stream>>>(p);
        else if (deep)
            attn_fwd16_kernel<false, true><<<grid, block, 0, stream>>>(p);
        else if (perm)
            attn_fwd16_kernel<true, false><<<grid, block, 0, stream>>>(p);
        else
            attn_fwd16_kernel<false, false><<<grid, block, 0, stream>>>(p);
        hipCheck(hipGetLastError());
        if (ev) hipCheck(hipEventRecord(ev[1], stream));
        return;
    }
    // The 32-row kernel: other head sizes and unaligned rows (the 16-row
    // kernel above serves D == 64 with 16-byte rows).
    auto pick = [&](auto dp_c) {
        constexpr int DP = decltype(dp_c)::value;
        if (p.vec && perm) return reinterpret_cast<const void *>(attn_fwd_kernel<true, DP, true>);
        if (p.vec) return reinterpret_cast<const void *>(attn_fwd_kernel<true, DP, false>);
        if (perm) return reinterpret_cast<const void *>(attn_fwd_kernel<false, DP, true>);
        return reinterpret_cast<const void *>(attn_fwd_kernel<false, DP, false>);
    };
    const bool wide = p.D > kDPad;
    const void *kern = wide ? pick(IntC<2 * kDPad>{}) : pick(IntC<kDPad>{});
    p.order = choose_grid_order(p.nqb, p.bh_pad, kern);
    const dim3 grid(p.nqb * p.bh_pad), block(256);
    if (ev) hipCheck(hipEventRecord(ev[0], stream));
    void *args[] = {&p};
    hipCheck(hipLaunchKernel(kern, grid, block, args, 0, stream));
    hipCheck(hipGetLastError());
    if (ev) hipCheck(hipEventRecord(ev[1], stream));
}

}  // namespace gptc
