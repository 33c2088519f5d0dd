// Fused causal attention backward for gfx950.  Like gpt.c's backward it
// starts from the probabilities the forward kept (here the packed causal
// blocks of P' with their per-tile maxima, rescaled by the saved
// log-sum-exp; gpt.c keeps the full (B, H, T, T) P).  Replaces gpt.c's
// unpermute / 4 batched SGEMMs / softmax backward / permute sequence
// (kernels/src/cuda/Attention.cu:235-324; math of
// kernels/src/cpu/Attention.c:169-301):
//     dP = dO V^T,  dV = P^T dO,  dS = P o (dP - rowsum(dP o P)),
//     dQ = dS K / sqrt(D),  dK = dS^T Q / sqrt(D),
// using rowsum(dP o P) = rowsum(dO o O) =: delta.  These are the four
// contractions of the reference; none is recomputed.
//
// Three kernels, bit-for-bit deterministic: every output element is written
// once, except the dK, dV rows of a key block split in two (grids that leave
// CUs idle, bwd_split_plan), which receive exactly two atomic adds into
// rows zeroed by the delta kernel (a + b == b + a in fp32):
//   attn_bwd_delta_kernel  delta = rowsum(dO o O); streams dO and O once.
//   attn_bwd_dkdv_dma_kernel  (D == 64 with the stored P') key-parallel:
//                          per 32-key wave (V resident in registers), over
//                          the query tiles: P from P', dP, dS,
//                          dV += P^T dO, dK += dS^T Q.  dS overwrites P'
//                          in place, in the exact register layout the dq
//                          kernel consumes it in.
//   attn_bwd_dkdv_kernel   the same for other head sizes, and with P
//                          recomputed from the LSE (short heads, the
//                          LSE-only state).
//   attn_bwd_dq16_kernel   query-parallel, D == 64: dQ += dS K, 16 queries
//                          per wave, work lists of 64-query blocks
//                          (block_sched.hpp).
//   attn_bwd_dq16_recomp_kernel  the same with S and dP recomputed, for an
//                          LSE-only state with no room for dS.
//   attn_bwd_dq_kernel     query-parallel, other D: dQ^T += K^T dS^T.
// P' and dS are written once and read once, through non-temporal accesses
// (stream_load / stream_store).
// The accumulator of the score product is directly the operand of the
// gradient products (see the layout note in attn_common.hpp).
#include <algorithm>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "attn_common.hpp"
#include "attn_kernels.hpp"
#include "hip_check.hpp"

namespace gptc {

constexpr int kBwdBK = 128;  // keys per dk/dv workgroup (32 per wave)
constexpr int kBwdBQ = 64;   // queries per LDS tile in the dk/dv kernel
constexpr int kBwdBM = 128;  // queries per dq workgroup (32 per wave)
constexpr int kBwdBN = 64;   // keys per LDS tile in the dq kernel

// ---- delta = rowsum(dO o O): 16 lanes per (b, t, h) row, 16 rows per workgroup ----
template <bool VEC>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const BwdParams a) {
    const int l16 = threadIdx.x & 15;
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);  // (b*T + t)*H + h: memory order of (B, T, C)
    const int rows = a.B * a.T * a.H;
    float sum = 0.0f;
    int b = 0, t = 0, h = 0;
    if (row < rows) {
        h = row % a.H;
        const int bt = row / a.H;
        t = bt % a.T;
        b = bt / a.T;
        const float *o = a.o.p + b * a.o.sb + t * a.o.st + h * a.o.sh;
        const float *g = a.dout.p + b * a.dout.sb + t * a.dout.st + h * a.dout.sh;
        if (VEC) {
            for (int d = 4 * l16; d < a.D; d += 64) {
                const f32x4 x = load4<true>(o, d, a.D), y = load4<true>(g, d, a.D);
                sum += x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
            }
        } else {
            for (int d = l16; d < a.D; d += 16) sum = fmaf(o[d], g[d], sum);
        }
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 16);
    if (row < rows && l16 == 0) a.delta[(static_cast<uint32_t>(b) * a.H + h) * a.T + t] = sum;
    // dK, dV rows of the split key blocks start at zero (D == 64, 16-byte rows).
    if (VEC && row < rows && t < a.nsplit * kBwdBK) {
        *reinterpret_cast<f32x4 *>(a.dk.p + b * a.dk.sb + t * a.dk.st + h * a.dk.sh + 4 * l16) = zero4();
        *reinterpret_cast<f32x4 *>(a.dv.p + b * a.dv.sb + t * a.dv.st + h * a.dv.sh + 4 * l16) = zero4();
    }
}

// ---- dK, dV (and the dS tiles): head sizes other than 64, and RECOMP ----
// FULL: D == kDPad, 16-byte rows and 31-bit head sizes; the tile loads then
// go through bounds-checked buffer resources (no branches, no row tests).
// FULL is built with RECOMP only: D == 64 with the stored P' runs
// attn_bwd_dkdv_dma_kernel.
// RECOMP (short heads, whose forward stored no P'): P is recomputed as
// exp2(S log2(e)/sqrt(D) - LSE log2(e)) with S = Q K^T formed like dP (Q rows
// from LDS as A operands, this lane's K row in registers as B operands) and
// the causal mask applied per element; one workgroup per head at T <= 128,
// so the kernel may use the registers of one wave per SIMD.
//
// DP: the head size the kernel is built for, 64 (D <= 64, the only choice
// with FULL) or 128 (64 < D <= 128: one wave per SIMD, 64 more registers
// per lane for V and as many for each of dK and dV).
template <bool VEC, bool FULL, bool RECOMP, int DP = kDPad>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RECOMP || DP > kDPad ? 1 : 2,
                                                                     RECOMP || DP > kDPad ? 1 : 2))) void
attn_bwd_dkdv_kernel(const BwdParams a) {
    static_assert(!FULL || DP == kDPad, "FULL kernels are built for D == 64");
    static_assert(!FULL || RECOMP, "D == 64 with the stored P' runs attn_bwd_dkdv_dma_kernel");
    constexpr int LS = DP + 4;         // LDS row stride (floats)
    constexpr int NJ = DP / 8;         // reduction steps of 8 dims (4 per lane half)
    constexpr int NDB = DP / 32;       // 32-dim blocks of dK and dV
    constexpr int TPR = DP / 4;        // tile-load threads per row (a float4 each)
    constexpr int RPP = 256 / TPR;     // tile rows per load pass
    constexpr int NLD = kBwdBQ / RPP;  // load passes per 64-query tile
    __shared__ __attribute__((aligned(16))) float q_lds[kBwdBQ * LS];
    __shared__ __attribute__((aligned(16))) float do_lds[kBwdBQ * LS];
    // Per-query statistics of the tile, one entry per thread: [0, 128) the
    // factors f of P = P' * f for the workgroup's two 64-key tiles
    // ([key tile][query]; RECOMP: [0, 64) LSE log2(e), +inf past T),
    // [128, 192) delta, [192, 256) unused.
    __shared__ __attribute__((aligned(16))) float stat_lds[256];
    const float *dl_lds = stat_lds + 2 * kBwdBQ;
    // The q bias of the head (FULL kernels with the qkv bias folded in),
    // added to the Q tile as it is stored; then the db column sums.
    __shared__ __attribute__((aligned(16))) float qb_lds[kDPad];
    __shared__ float red_lds[4][2 * kDPad];

    const int tid = threadIdx.x;
    // The wave index is made visibly uniform (an SGPR): branches on it are then
    // scalar branches instead of exec-masked divergent regions around MFMAs.
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
    const int bh = blockIdx.x % a.bh_pad;
    if (bh >= a.B * a.H) return;
    const int kb_idx = static_cast<int>(blockIdx.x / a.bh_pad);
    const int b = bh / a.H, h = bh - b * a.H;
    const int T = a.T, D = a.D;

    const int k_blk0 = kb_idx * kBwdBK;
    const int kw0 = k_blk0 + 32 * w;
    const int my_k = kw0 + l32;
    const bool k_ok = my_k < T;

    const float *Qh = a.q.p + b * a.q.sb + h * a.q.sh;
    const float *Vh = a.v.p + b * a.v.sb + h * a.v.sh;
    const float *dOh = a.dout.p + b * a.dout.sb + h * a.dout.sh;
    const float *lse_h = a.lse + static_cast<uint32_t>(bh) * T;
    const float *dl_h = a.delta + static_cast<uint32_t>(bh) * T;
    const float *pm_h = a.pm + static_cast<uint32_t>(bh) * a.nqt * T;

    // V row of this lane's key, dims 8j + 4hf + c: B operand of dP = dO V^T.
    f32x4 vr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) vr[j] = k_ok ? load4<VEC>(Vh + my_k * a.v.st, 8 * j + 4 * hf, D) : zero4();
    // RECOMP: the K row of this lane's key, dims 8j + 4hf + c: B operand of S = Q K^T.
    f32x4 kr[RECOMP ? NJ : 1];
    if (RECOMP) {
        const float *Kh = a.k.p + b * a.k.sb + h * a.k.sh;
#pragma unroll
        for (int j = 0; j < NJ; ++j) kr[j] = k_ok ? load4<VEC>(Kh + my_k * a.k.st, 8 * j + 4 * hf, D) : zero4();
    }
    // The qkv bias (FULL only): added to this key's V (and K) row here, to
    // the Q tiles through qb_lds.  Keys past T keep a zero row.
    const bool biased = FULL && a.qb != nullptr;
    f32x4 vbias[NJ], kbias[RECOMP ? NJ : 1];
    f32x4 qb4 = zero4();
    if (biased) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            vbias[j] = *reinterpret_cast<const f32x4 *>(a.vb + h * kDPad + 8 * j + 4 * hf);
            if (RECOMP) kbias[j] = *reinterpret_cast<const f32x4 *>(a.kb + h * kDPad + 8 * j + 4 * hf);
        }
        if (tid < kDPad / 4) qb4 = *reinterpret_cast<const f32x4 *>(a.qb + h * kDPad + 4 * tid);
    }
    // Let these loads land here: a loop-invariant register with a load still
    // counted as outstanding makes every use in the loop wait for all loads.
    __builtin_amdgcn_s_waitcnt(0);
    if (biased) {
        if (k_ok) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                vr[j] += vbias[j];
                if (RECOMP) kr[j] += kbias[j];
            }
        }
        if (tid < kDPad / 4) *reinterpret_cast<f32x4 *>(&qb_lds[4 * tid]) = qb4;
    }

    // Query tiles [qt0, n_qt): all from the diagonal on.
    const int n_qt = a.nqt;
    const int qt0 = k_blk0 / kBwdBQ, q_end = n_qt;
    const int ld_row = tid / TPR, ld_col = 4 * (tid % TPR);
    const auto q_rows = head_rows(Qh, T, a.q.st);
    const auto do_rows = head_rows(dOh, T, a.dout.st);
    f32x4 qpre[NLD], dpre[NLD];
    float st0 = 0.0f, st1 = 0.0f;
    bool st_ok = false;
    auto prefetch = [&](int qt) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int q = qt * kBwdBQ + ld_row + RPP * i;
            if (FULL) {
                qpre[i] = buffer_load4(q_rows, static_cast<uint32_t>(q) * a.q.st + ld_col);
                dpre[i] = buffer_load4(do_rows, static_cast<uint32_t>(q) * a.dout.st + ld_col);
            } else {
                qpre[i] = (q < T) ? load4<VEC>(Qh + q * a.q.st, ld_col, D) : zero4();
                dpre[i] = (q < T) ? load4<VEC>(dOh + q * a.dout.st, ld_col, D) : zero4();
            }
        }
        // Threads 0..127: m and lse of query (tid & 63) for key tile 2kb + tid/64;
        // threads 128..191: delta.  Loads from clamped, always valid addresses;
        // rows past T (and a key tile past T) get f = 0 and delta = 0 when the
        // values are written to LDS.  Arithmetic or selects on them here would
        // make the wave wait for all its outstanding loads at once.
        const int q = qt * kBwdBQ + (tid & (kBwdBQ - 1));
        const int qc = min(q, T - 1);
        const bool is_m = tid < 2 * kBwdBQ;
        const int kt = 2 * kb_idx + ((tid >> 6) & 1);
        st_ok = q < T && (!is_m || kt < n_qt);
        st0 = RECOMP ? dl_h[qc] : *(is_m ? pm_h + min(kt, n_qt - 1) * T + qc : dl_h + qc);
        st1 = lse_h[qc];
    };
    if (qt0 < q_end) prefetch(qt0);

    // P' of one 32-query half, loaded one half ahead of its use: register r
    // holds query 8(r/4) + 4hf + r%4 of the half, key my_k (the accumulator
    // layout of a queries x keys product).  A half is needed when some of
    // its queries see some of this wave's keys and it starts before T.  The
    // forward wrote every row of such a half (finite values; rows at or past
    // T get f = 0), so the loads need no row check.
    float pbuf[16];
    auto half_needed = [&](int qt, int qb) {
        const int qh0 = qt * kBwdBQ + 32 * qb;
        return qh0 + 31 >= kw0 && kw0 < T && qh0 < T;
    };
    // This wave's half of block (qt, kw0/32): a uniform base (SGPRs) plus a
    // lane offset, so that every row of the half is an immediate offset.
    const uint32_t lane_off = 4 * hf * 32 + l32;
    auto half_base = [&](int qt, int qb) {
        return a.ds + uniform(static_cast<uint32_t>(ds_block_offset(bh - a.ds_bh0, n_qt, qt, kw0 >> 5)) + 32 * qb * 32);
    };
    auto load_p = [&](int qt, int qb) {
        if (RECOMP || !half_needed(qt, qb)) return;
        const float *hb = half_base(qt, qb);
#pragma unroll
        for (int r = 0; r < 16; ++r) pbuf[r] = stream_load(hb + lane_off + (8 * (r >> 2) + (r & 3)) * 32);
    };
    if (qt0 < q_end) load_p(qt0, 0);

    f32x16 acc_dk[NDB], acc_dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc_dk[db] = acc_dv[db] = zero16();

    for (int qt = qt0; qt < q_end; ++qt) {
        __syncthreads();
        if (biased) {
            // Q rows past T hold the bias too: their dO rows are zero and
            // their P is 0 (f = 0, or the +inf LSE of RECOMP), so they add nothing.
            const f32x4 qb = *reinterpret_cast<const f32x4 *>(&qb_lds[ld_col]);
#pragma unroll
            for (int i = 0; i < NLD; ++i) qpre[i] += qb;
        }
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int row = ld_row + RPP * i;
            *reinterpret_cast<f32x4 *>(&q_lds[row * LS + ld_col]) = qpre[i];
            *reinterpret_cast<f32x4 *>(&do_lds[row * LS + ld_col]) = dpre[i];
        }
        // Unconditional, so that no exec-masked branch sits between the loads
        // and their uses (branches make the wait counts conservative).
        if (RECOMP) {
            stat_lds[tid] = tid < kBwdBQ ? (st_ok ? st1 * kLog2e : INFINITY) : (st_ok ? st0 : 0.0f);
        } else {
            const float f = fast_exp2(st0 - st1 * kLog2e);
            stat_lds[tid] = st_ok ? (tid < 2 * kBwdBQ ? f : st0) : 0.0f;
        }
        __syncthreads();

        const float *f_w = stat_lds + (w >> 1) * kBwdBQ;  // this wave's key tile
        // The tile's two 32-query halves one after the other: one P and one dP
        // block live at a time, which keeps the wave within the register budget
        // of two waves per SIMD.
        for (int qb = 0; qb < 2; ++qb) {
            const bool need = half_needed(qt, qb);
            f32x16 s, dp = zero16();
            if (need) {
                // dP (queries x keys) for this 32-query half.
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const f32x4 da = *reinterpret_cast<const f32x4 *>(
                        &do_lds[(32 * qb + l32) * LS + 8 * j + 4 * hf]);
#pragma unroll
                    for (int c = 0; c < 4; ++c) dp = mfma32(da[c], vr[j][c], dp);
                }
                if (RECOMP) {
                    // S (queries x keys) for this half, then P with the causal mask.
                    s = zero16();
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const f32x4 qa = *reinterpret_cast<const f32x4 *>(
                            &q_lds[(32 * qb + l32) * LS + 8 * j + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) s = mfma32(qa[c], kr[j][c], s);
                    }
                    const float c2 = a.scale * kLog2e;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&stat_lds[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const int q = qt * kBwdBQ + 32 * qb + 8 * g + 4 * hf + c;
                            const float p = fast_exp2(fmaf(s[4 * g + c], c2, -l4[c]));
                            s[4 * g + c] = my_k > q ? 0.0f : p;  // P
                        }
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 f4 = *reinterpret_cast<const f32x4 *>(&f_w[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) s[4 * g + c] = pbuf[4 * g + c] * f4[c];  // P
                    }
                }
            }
            // The next half's P' (its registers are free now).
            if (qb == 0) {
                load_p(qt, 1);
                // Issued after this half's P' is consumed, so that waiting for
                // that P' never waits for these loads.
                if (qt + 1 < q_end) prefetch(qt + 1);
            } else if (qt + 1 < q_end) {
                load_p(qt + 1, 0);
            }
            if (!need) continue;

#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&dl_lds[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                for (int c = 0; c < 4; ++c) dp[4 * g + c] = s[4 * g + c] * (dp[4 * g + c] - d4[c]);  // dS
            }

            // dS replaces P' in place: block (qt, key block kw0/32), [64 queries][32 keys]
            // (none with the LSE-only state, whose dq kernel recomputes it).
            if (!RECOMP || a.ds != nullptr) {
                float *hb = half_base(qt, qb);
#pragma unroll
                for (int r = 0; r < 16; ++r) stream_store(hb + lane_off + (8 * (r >> 2) + (r & 3)) * 32, dp[r]);
            }

            // dV += P^T dO and dK += dS^T Q (keys x dims).
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int row = 32 * qb + 8 * g + 4 * hf + c;
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        acc_dv[db] = mfma32(s[4 * g + c], do_lds[row * LS + 32 * db + l32], acc_dv[db]);
                        acc_dk[db] = mfma32(dp[4 * g + c], q_lds[row * LS + 32 * db + l32], acc_dk[db]);
                    }
                }
        }
    }

    // Accumulator layout (keys x dims): lane -> dim 32*db + l32,
    // register r -> key kw0 + 8(r/4) + 4hf + r%4.
    float *dKh = a.dk.p + b * a.dk.sb + h * a.dk.sh;
    float *dVh = a.dv.p + b * a.dv.sb + h * a.dv.sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
        const int dim = 32 * db + l32;
        if (dim >= D) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kw0 + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (key < T) {
                dKh[key * a.dk.st + dim] = acc_dk[db][r] * a.scale;
                dVh[key * a.dv.st + dim] = acc_dv[db][r];
            }
        }
    }
    if (FULL && a.db != nullptr) {
        // db of the k and v parts: column sums of this workgroup's 128 dK and
        // dV rows (keys < T), in a fixed order: registers, lane halves, waves.
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            float sk = 0.0f, sv = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const bool ok = kw0 + 8 * (r >> 2) + 4 * hf + (r & 3) < T;
                sk += ok ? acc_dk[db][r] : 0.0f;
                sv += ok ? acc_dv[db][r] : 0.0f;
            }
            sk += other_half(sk);
            sv += other_half(sv);
            if (hf == 0) {
                red_lds[w][32 * db + l32] = sk * a.scale;
                red_lds[w][kDPad + 32 * db + l32] = sv;
            }
        }
        __syncthreads();
        if (tid < 2 * kDPad) {
            const float s = (red_lds[0][tid] + red_lds[1][tid]) + (red_lds[2][tid] + red_lds[3][tid]);
            // Row (b, key block or its part 1) of the (B*(nkb + nsplit)) x 2C
            // partials: dk part, then dv part.
            const int col = (tid < kDPad ? 0 : a.C) + h * kDPad + (tid & (kDPad - 1));
            a.dbkv_part[(static_cast<size_t>(b) * a.nkb + kb_idx) * 2 * a.C + col] = s;
        }
    }
}

// ---- dK, dV of D == 64 heads with the stored P' (the long-head path) ----
// The same per-wave work as attn_bwd_dkdv_kernel<true, true, false> on one
// 128-key block (wave w: keys 32w .. 32w+31 of it), run over work lists
// (block_sched.hpp): each workgroup takes its items (query tiles [qa, qe) of
// key block kb of head bh) one after the other, as one sequence of steps
// (one step = one 64-query tile of one item).
//
// The Q and dO tiles are double-buffered in LDS and filled by buffer loads
// that write LDS directly (64 floats per instruction; rows past T read as
// zeros through the buffer resource).  The tile of the next step (the next
// item's first one at the end of an item) is requested right after the
// barrier that opens a step, so one barrier per step both publishes the next
// tile and frees the previous one, and the tile loads take no registers and
// no LDS store instructions.  The statistics and the P' rows of the next step
// are loaded during this one likewise.
//
// dO is stored by rows (one row per instruction): dP = dO V^T reads a lane's
// query row as float4s.  Q feeds only dK += dS^T Q, whose B operand gives a
// lane one dim of 4 consecutive queries per 4 MFMAs, so Q is stored as
// [query / 4][dim][query % 4]: one 16-byte read per lane and 4 MFMAs.  Each
// load instruction gathers 16 dims of 4 consecutive rows (4 pieces of 64
// bytes) into 64 consecutive LDS words.
//
// The loads are __builtin_amdgcn_raw_ptr_buffer_load_lds: the compiler sets
// M0 (the LDS address of the instruction's 64 words) and counts them.  The
// wait for a tile is an explicit s_waitcnt vmcnt(0) right before the barrier
// that publishes it; every LDS read of that buffer comes after the barrier.
//
// At the end of an item its dK, dV rows are stored (added, for the two items
// of a key block kb < nsplit), then the next item's V rows are loaded.
//
// BIAS: the v bias joins the V rows as they are loaded; the q bias is added
// to the Q operand of dK += dS^T Q as it is read (the same sum as adding it
// to the stored tile: rows past T then hold the bias, with dS = 0 there).
//
// RECOMP (the LSE-only state: the forward stored no P'): P is recomputed as
// exp2(S log2(e)/sqrt(D) - LSE log2(e)) with S = Q K^T formed like dP (Q
// rows from LDS as A operands, this lane's K row in registers as B
// operands), and dS goes to a.ds, a scratch of the packed blocks of heads
// [ds_bh0, ...) that the dq16 kernel reads next.  The Q tile is then stored
// by rows, like dO (S reads a lane's query row as float4s; dK's B operand
// becomes one word per MFMA, as dV's), and the statistics are the LSE (log2
// units, +inf past T) and delta.
template <bool BIAS, bool RECOMP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_bwd_dkdv_dma_kernel(const BwdParams a) {
    constexpr int LS = kDPad + 4;      // LDS row stride (floats)
    constexpr int NJ = kDPad / 8;      // reduction steps of 8 dims (4 per lane half)
    constexpr int kTile = kBwdBQ * LS;      // floats per dO tile (rows)
    constexpr int kQTile = RECOMP ? kTile : kBwdBQ * kDPad;  // floats per Q tile (rows, or [q / 4][dim][q % 4])
    __shared__ __attribute__((aligned(16))) float q_lds[2 * kQTile];
    __shared__ __attribute__((aligned(16))) float do_lds[2 * kTile];
    // Per buffer, one entry per thread: [0, 128) the factors f of P = P' * f
    // for the workgroup's two 64-key tiles ([key tile][query]; RECOMP: [0, 64)
    // LSE log2(e), +inf past T), [128, 192) delta, [192, 256) unused.
    __shared__ __attribute__((aligned(16))) float stat_lds[2 * 256];
    __shared__ float red_lds[4][2 * kDPad];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
    const int it_end = a.ksched.wg_start[blockIdx.x + 1];
    const int it0 = a.ksched.wg_start[blockIdx.x];
    if (it0 >= it_end) return;
    const int T = a.T, n_qt = a.nqt;

    // A step: tile qt of item it = (bh, kb, qa, qe).  All fields are uniform.
    struct Step {
        int it, bh, kb, qa, qt, qe;
    };
    auto item_step = [&](int i) {
        const int *e = a.ksched.items + 4 * i;
        return Step{i, e[0], e[1], e[2], e[2], e[3]};
    };
    // The step after s: the next tile of its item, or the next item's first.
    auto advance = [&](Step &s) {
        if (s.qt + 1 < s.qe) {
            ++s.qt;
            return true;
        }
        if (s.it + 1 >= it_end) return false;
        s = item_step(s.it + 1);
        return true;
    };
    auto head_of = [&](int bh, int &b, int &h) {
        b = bh / a.H;
        h = bh - b * a.H;
    };

    // V row of this lane's key, dims 8j + 4hf + c: B operand of dP = dO V^T
    // (RECOMP: the K row too, B operand of S = Q K^T).  BIAS: the v (and k)
    // bias joins it (keys past T keep a zero row); qbias holds the q bias of
    // this lane's two dims.
    f32x4 vr[NJ];
    f32x4 kr[RECOMP ? NJ : 1];
    float qbias[2] = {0.0f, 0.0f};
    // RECOMP with BIAS: S = (Q + qb) K'^T = Q K'^T + qb . K' (K' = K + kb):
    // the q bias adds qbk = qb . K'[my_k] to every score of this lane's key.
    float qbk = 0.0f;
    auto load_v = [&](const Step &s) {
        int b, h;
        head_of(s.bh, b, h);
        const int my_k = s.kb * kBwdBK + 32 * w + l32;
        const bool k_ok = my_k < T;
        const float *Vh = a.v.p + b * a.v.sb + h * a.v.sh;
#pragma unroll
        for (int j = 0; j < NJ; ++j) vr[j] = k_ok ? load4<true>(Vh + my_k * a.v.st, 8 * j + 4 * hf, kDPad) : zero4();
        if (RECOMP) {
            const float *Kh = a.k.p + b * a.k.sb + h * a.k.sh;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                kr[j] = k_ok ? load4<true>(Kh + my_k * a.k.st, 8 * j + 4 * hf, kDPad) : zero4();
        }
        if (BIAS) {
            if (k_ok) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    vr[j] += *reinterpret_cast<const f32x4 *>(a.vb + h * kDPad + 8 * j + 4 * hf);
                    if (RECOMP) kr[j] += *reinterpret_cast<const f32x4 *>(a.kb + h * kDPad + 8 * j + 4 * hf);
                }
            }
            if (RECOMP) {
                float part = 0.0f;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const f32x4 q4 = *reinterpret_cast<const f32x4 *>(a.qb + h * kDPad + 8 * j + 4 * hf);
#pragma unroll
                    for (int c = 0; c < 4; ++c) part = fmaf(q4[c], kr[j][c], part);
                }
                qbk = part + other_half(part);
            }
            qbias[0] = a.qb[h * kDPad + l32];
            qbias[1] = a.qb[h * kDPad + 32 + l32];
        }
    };

    // Rows 16w .. 16w+15 of the step's tile into LDS buffer buf (mq, md: the
    // LDS byte address an instruction's 64 words start at).  dO: row q0 + i,
    // lane -> dim.  Q: instruction i takes rows q0 + 4(i/4) + (lane % 4), dims
    // 16(i % 4) + lane / 4, i.e. group q4 = 4w + i/4 of the tile, words
    // [64(i % 4), 64(i % 4) + 64) of the group's 256.
    const uint32_t vl = 4u * lane;
    const uint32_t vq = 4u * ((lane & 3) * a.q.st + (lane >> 2));
    const uint32_t lds_q = uniform(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                               (__attribute__((address_space(3))) float *)q_lds)) +
                           16u * w * (RECOMP ? LS : kDPad) * 4u);
    const uint32_t lds_do = uniform(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                                (__attribute__((address_space(3))) float *)do_lds)) + 16u * w * LS * 4u);
    auto load_tile = [&](const Step &s, int buf) {
        int b, h;
        head_of(s.bh, b, h);
        const auto q_rows = head_rows(a.q.p + b * a.q.sb + h * a.q.sh, T, a.q.st);
        const auto do_rows = head_rows(a.dout.p + b * a.dout.sb + h * a.dout.sh, T, a.dout.st);
        const uint32_t q0 = static_cast<uint32_t>(s.qt * kBwdBQ + 16 * w);
        const uint32_t mq = lds_q + buf * (kQTile * 4u), md = lds_do + buf * (kTile * 4u);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t q = q0 + i;
            const uint32_t gq = q0 + 4 * (i >> 2);
            if (RECOMP)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(q_rows, lds_ptr(mq + i * LS * 4u), 4, q * a.q.st * 4u + vl, 0,
                                                         0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(q_rows,
                                                         lds_ptr(mq + (i >> 2) * (4u * kDPad * 4u) + (i & 3) * 256u),
                                                         4, gq * a.q.st * 4u + (i & 3) * 64u + vq, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(do_rows, lds_ptr(md + i * LS * 4u), 4,
                                                     q * a.dout.st * 4u + vl, 0, 0, 0);
        }
    };
    // The statistics of a step, loaded one step ahead (see attn_bwd_dkdv_kernel).
    float st0 = 0.0f, st1 = 0.0f;
    bool st_ok = false;
    auto load_stats = [&](const Step &s) {
        const uint32_t bh = static_cast<uint32_t>(s.bh);
        const int q = s.qt * kBwdBQ + (tid & (kBwdBQ - 1));
        const int qc = min(q, T - 1);
        if (RECOMP) {
            st_ok = q < T;
            st0 = a.delta[bh * T + qc];
        } else {
            const bool is_m = tid < 2 * kBwdBQ;
            const int kt = 2 * s.kb + ((tid >> 6) & 1);
            st_ok = q < T && (!is_m || kt < n_qt);
            st0 = *(is_m ? a.pm + bh * n_qt * T + min(kt, n_qt - 1) * T + qc : a.delta + bh * T + qc);
        }
        st1 = a.lse[bh * T + qc];
    };

    float pbuf[16];
    auto half_needed = [&](const Step &s, int qb) {
        const int qh0 = s.qt * kBwdBQ + 32 * qb, kw0 = s.kb * kBwdBK + 32 * w;
        return qh0 + 31 >= kw0 && kw0 < T && qh0 < T;
    };
    const uint32_t lane_off = 4 * hf * 32 + l32;
    auto half_base = [&](const Step &s, int qb) {
        const int kw0 = s.kb * kBwdBK + 32 * w;
        return a.ds + uniform(static_cast<uint32_t>(ds_block_offset(s.bh - a.ds_bh0, n_qt, s.qt, kw0 >> 5)) +
                              32 * qb * 32);
    };
    auto load_p = [&](const Step &s, int qb) {
        if (RECOMP || !half_needed(s, qb)) return;
        const float *hb = half_base(s, qb);
#pragma unroll
        for (int r = 0; r < 16; ++r) pbuf[r] = stream_load(hb + lane_off + (8 * (r >> 2) + (r & 3)) * 32);
    };

    f32x16 acc_dk[2], acc_dv[2];
#pragma unroll
    for (int db = 0; db < 2; ++db) acc_dk[db] = acc_dv[db] = zero16();

    // Accumulator layout (keys x dims): lane -> dim 32*db + l32,
    // register r -> key kw0 + 8(r/4) + 4hf + r%4.
    auto finish_item = [&](const Step &s) {
        int b, h;
        head_of(s.bh, b, h);
        const int kw0 = s.kb * kBwdBK + 32 * w;
        const bool split = s.kb < a.nsplit;
        float *dKh = a.dk.p + b * a.dk.sb + h * a.dk.sh;
        float *dVh = a.dv.p + b * a.dv.sb + h * a.dv.sh;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const int dim = 32 * db + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kw0 + 8 * (r >> 2) + 4 * hf + (r & 3);
                if (key < T) {
                    if (split) {
                        unsafeAtomicAdd(&dKh[key * a.dk.st + dim], acc_dk[db][r] * a.scale);
                        unsafeAtomicAdd(&dVh[key * a.dv.st + dim], acc_dv[db][r]);
                    } else {
                        dKh[key * a.dk.st + dim] = acc_dk[db][r] * a.scale;
                        dVh[key * a.dv.st + dim] = acc_dv[db][r];
                    }
                }
            }
        }
        if (a.db != nullptr) {
            // db of the k and v parts, as in attn_bwd_dkdv_kernel.  red_lds is
            // free: its last readers passed at least one step barrier since.
#pragma unroll
            for (int db = 0; db < 2; ++db) {
                float sk = 0.0f, sv = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const bool ok = kw0 + 8 * (r >> 2) + 4 * hf + (r & 3) < T;
                    sk += ok ? acc_dk[db][r] : 0.0f;
                    sv += ok ? acc_dv[db][r] : 0.0f;
                }
                sk += other_half(sk);
                sv += other_half(sv);
                if (hf == 0) {
                    red_lds[w][32 * db + l32] = sk * a.scale;
                    red_lds[w][kDPad + 32 * db + l32] = sv;
                }
            }
            __syncthreads();
            if (tid < 2 * kDPad) {
                const float sum = (red_lds[0][tid] + red_lds[1][tid]) + (red_lds[2][tid] + red_lds[3][tid]);
                const int col = (tid < kDPad ? 0 : a.C) + h * kDPad + (tid & (kDPad - 1));
                const int prow = split && s.qa != 2 * s.kb ? a.nkb + s.kb : s.kb;
                a.dbkv_part[(static_cast<size_t>(b) * (a.nkb + a.nsplit) + prow) * 2 * a.C + col] = sum;
            }
        }
    };

    Step cur = item_step(it0);
    load_v(cur);
    load_tile(cur, 0);
    load_stats(cur);
    load_p(cur, 0);
    int total_steps = 0, done_steps = 0;
    for (int i = it0; i < it_end; ++i) total_steps += a.ksched.items[4 * i + 3] - a.ksched.items[4 * i + 2];

    for (int buf = 0;; buf ^= 1) {
        // Wave priority from the steps of the list still to run, one level
        // per 3 (4 levels): the SIMDs otherwise issue from the oldest waves
        // first, so the CU's first workgroup runs ahead and the other one
        // runs alone at the end; the workgroup with more left to do now wins
        // the MFMA pipe, whatever the two lists' lengths.  (A level per
        // quarter of the workgroup's own list ended two equal lists of a CU
        // 16 us apart at C2; this is 1 us faster there and at C5.)
        switch ((total_steps - done_steps) / 3) {  // wave-uniform
            case 0: __builtin_amdgcn_s_setprio(0); break;
            case 1: __builtin_amdgcn_s_setprio(1); break;
            case 2: __builtin_amdgcn_s_setprio(2); break;
            default: __builtin_amdgcn_s_setprio(3); break;
        }
        ++done_steps;
        if (RECOMP) {
            stat_lds[buf * 256 + tid] = tid < kBwdBQ ? (st_ok ? st1 * kLog2e : INFINITY) : (st_ok ? st0 : 0.0f);
        } else {
            const float f = fast_exp2(st0 - st1 * kLog2e);
            stat_lds[buf * 256 + tid] = st_ok ? (tid < 2 * kBwdBQ ? f : st0) : 0.0f;
        }
        // This wave's loads of this step's tile have landed; after the barrier
        // every wave's have, and the other buffer (the previous step's) is no
        // longer read.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        Step nxt = cur;
        const bool more = advance(nxt);
        if (more) load_tile(nxt, buf ^ 1);

        const float *qs = q_lds + buf * kQTile, *dos = do_lds + buf * kTile;
        const float *f_w = stat_lds + buf * 256 + (w >> 1) * kBwdBQ;
        const float *dl_w = stat_lds + buf * 256 + 2 * kBwdBQ;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const bool need = half_needed(cur, qb);
            f32x16 s, dp = zero16();
            if (need) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const f32x4 da = *reinterpret_cast<const f32x4 *>(&dos[(32 * qb + l32) * LS + 8 * j + 4 * hf]);
#pragma unroll
                    for (int c = 0; c < 4; ++c) dp = mfma32(da[c], vr[j][c], dp);
                }
                if (RECOMP) {
                    // S (queries x keys), then P with the causal mask (keys
                    // past T see only queries below T: masked too).
                    s = zero16();
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const f32x4 qa = *reinterpret_cast<const f32x4 *>(&qs[(32 * qb + l32) * LS + 8 * j + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) s = mfma32(qa[c], kr[j][c], s);
                    }
                    const float c2 = a.scale * kLog2e;
                    const int my_k = cur.kb * kBwdBK + 32 * w + l32;
                    const float *lse_w = stat_lds + buf * 256;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&lse_w[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const int q = cur.qt * kBwdBQ + 32 * qb + 8 * g + 4 * hf + c;
                            const float sv = BIAS ? s[4 * g + c] + qbk : s[4 * g + c];
                            const float pv = fast_exp2(fmaf(sv, c2, -l4[c]));
                            s[4 * g + c] = my_k > q ? 0.0f : pv;  // P
                        }
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 f4 = *reinterpret_cast<const f32x4 *>(&f_w[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                        for (int c = 0; c < 4; ++c) s[4 * g + c] = pbuf[4 * g + c] * f4[c];  // P
                    }
                }
            }
            if (qb == 0) {
                load_p(cur, 1);
                if (more) load_stats(nxt);
            } else if (more) {
                load_p(nxt, 0);
            }
            if (!need) continue;

#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&dl_w[32 * qb + 8 * g + 4 * hf]);
#pragma unroll
                for (int c = 0; c < 4; ++c) dp[4 * g + c] = s[4 * g + c] * (dp[4 * g + c] - d4[c]);  // dS
            }
            {
                float *hb = half_base(cur, qb);
#pragma unroll
                for (int r = 0; r < 16; ++r) stream_store(hb + lane_off + (8 * (r >> 2) + (r & 3)) * 32, dp[r]);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                // Q rows 32qb + 8g + 4hf + c, c = 0..3, dim 32db + l32.
                f32x4 q4[2];
                if (!RECOMP) {
#pragma unroll
                    for (int db = 0; db < 2; ++db)
                        q4[db] = *reinterpret_cast<const f32x4 *>(&qs[(8 * qb + 2 * g + hf) * (4 * kDPad) +
                                                                       (32 * db + l32) * 4]);
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int row = 32 * qb + 8 * g + 4 * hf + c;
#pragma unroll
                    for (int db = 0; db < 2; ++db) {
                        const float qv = RECOMP ? qs[row * LS + 32 * db + l32] : q4[db][c];
                        acc_dv[db] = mfma32(s[4 * g + c], dos[row * LS + 32 * db + l32], acc_dv[db]);
                        acc_dk[db] = mfma32(dp[4 * g + c], BIAS ? qv + qbias[db] : qv, acc_dk[db]);
                    }
                }
            }
        }

        if (!more || nxt.it != cur.it) {
            finish_item(cur);
            if (!more) break;
            load_v(nxt);
#pragma unroll
            for (int db = 0; db < 2; ++db) acc_dk[db] = acc_dv[db] = zero16();
        }
        cur = nxt;
    }
}

// ---- dQ = dS K / sqrt(D) from the stored dS tiles (head sizes other than 64) ----
// DP: the head size the kernel is built for, 64 or 128 (as for dk/dv).
template <bool VEC, int DP>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const BwdParams a) {
    constexpr int LS = DP + 4;         // LDS row stride (floats)
    constexpr int NDB = DP / 32;       // 32-dim blocks of dQ
    constexpr int TPR = DP / 4;        // tile-load threads per row (a float4 each)
    constexpr int RPP = 256 / TPR;     // tile rows per load pass
    constexpr int NLD = kBwdBN / RPP;  // load passes per 64-key tile
    __shared__ __attribute__((aligned(16))) float k_lds[kBwdBN * LS];

    const int tid = threadIdx.x;
    // The wave index is made visibly uniform (an SGPR): branches on it are then
    // scalar branches instead of exec-masked divergent regions around MFMAs.
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
    // Query blocks in the XCD- and CU-aware order of grid_order.hpp.
    int blk, bh;
    grid_position(a.dq_order, a.nqb, a.bh_pad, blk, bh);
    if (bh >= a.B * a.H) return;
    const int qb = a.nqb - 1 - blk;
    const int b = bh / a.H, h = bh - b * a.H;
    const int T = a.T, D = a.D;

    const int q_blk0 = qb * kBwdBM;
    const int qw0 = q_blk0 + 32 * w;
    const int my_q = qw0 + l32;
    const bool wave_on = qw0 < T;

    const float *Kh = a.k.p + b * a.k.sb + h * a.k.sh;
    // This lane's dS row (query my_q) inside its 64-query tile: key block kb32
    // starts kb32 * 2048 floats after the (uniform) tile base; keys
    // 8g + 4hf + c come as float4 g.
    const int qt = qw0 >> 6;
    const float *ds_tile = a.ds + ds_block_offset(bh, a.nqt, qt, 0);
    const uint32_t row_off = ((qw0 & 32) + l32) * 32 + 4 * hf;

    const int kv_end = min(T, q_blk0 + kBwdBM);
    const int n_tiles = (kv_end + kBwdBN - 1) / kBwdBN;
    const int ld_row = tid / TPR, ld_col = 4 * (tid % TPR);
    f32x4 kpre[NLD];
    f32x4 dsn[2][4];
    auto prefetch = [&](int kt) {
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int key = kt * kBwdBN + ld_row + RPP * i;
            kpre[i] = (key < T) ? load4<VEC>(Kh + key * a.k.st, ld_col, D) : zero4();
        }
        // Key blocks past this wave's diagonal (all of dS zero there) or wholly
        // past T are never written by the dk/dv kernel: read nothing from them.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int kb32 = 2 * kt + kb;
            const bool ok = wave_on && 32 * kb32 <= qw0 && 32 * kb32 < T;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                dsn[kb][g] = ok ? stream_load(reinterpret_cast<const f32x4 *>(ds_tile + kb32 * kDsBlock + row_off + 8 * g))
                                : zero4();
        }
    };
    prefetch(0);

    f32x16 acc_dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc_dq[db] = zero16();
    for (int kt = 0; kt < n_tiles; ++kt) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            *reinterpret_cast<f32x4 *>(&k_lds[(ld_row + RPP * i) * LS + ld_col]) = kpre[i];
        __syncthreads();
        f32x4 dsc[2][4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g = 0; g < 4; ++g) dsc[kb][g] = dsn[kb][g];
        if (kt + 1 < n_tiles) prefetch(kt + 1);

        if (!wave_on || kt * kBwdBN > qw0 + 31) continue;
        // dQ^T (dims x queries) += K^T dS^T
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int row = 32 * kb + 8 * g + 4 * hf + c;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
                        acc_dq[db] = mfma32(k_lds[row * LS + 32 * db + l32], dsc[kb][g][c], acc_dq[db]);
                }
    }

    if (my_q >= T) return;
    float *dqrow = a.dq.p + b * a.dq.sb + my_q * a.dq.st + h * a.dq.sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 val;
#pragma unroll
            for (int c = 0; c < 4; ++c) val[c] = acc_dq[db][4 * g + c] * a.scale;
            store4<VEC>(dqrow, 32 * db + 8 * g + 4 * hf, D, val);
        }
}

// ---- dQ, 16-row form (D == kDPad, 16-byte rows, 31-bit head sizes) ----
// WG = 4 waves x 16 queries = one 64-query block of one (b, h) at a time,
// running the blocks of its work list (block_sched.hpp: at B=8, H=12,
// T=1024 blocks j and 15-j of one head, so every WG reduces nqt+1 key
// tiles and the grid is resident at once with equal work per WG).
// v_mfma_f32_16x16x4_f32 on dQ[q][d] += sum_k dS[q][k] K[k][d]:
//   A = dS (lane l: query l%16, k-slot l/16), B = K (k-slot l/16, column l%16).
// Step (t, c) of a 64-key tile puts key 16t + 4j + c in k-slot j, so the A
// operands of a lane for c = 0..3 are one float4 of its dS row and its B
// operands one float4 of the K tile, which LDS holds as
//     k_lds[(key / 4) * 256 + 4 * (16 * (d % 4) + d / 4) + key % 4]
// (16 lanes read 256 contiguous bytes).  Column n of dim block db is dim
// 4n + db: a lane ends with dims 4n .. 4n+3 of its rows, one float4 store each.
// dS is read only where the wave's queries see the keys: on the block's own
// tile, 16-key slices t <= w (the rest of that tile is zero).
constexpr int kDq16KStride = 256;  // floats per group of 4 keys in k_lds

__global__ __launch_bounds__(256) void attn_bwd_dq16_kernel(const BwdParams a) {
    __shared__ __attribute__((aligned(16))) float k_lds[16 * kDq16KStride];
    __shared__ float red_lds[4][kDPad];  // db column sums of the block's dQ rows, per wave

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, j = lane >> 4, n = lane & 15;
    const int it_end = a.sched.wg_start[blockIdx.x + 1];
    int it = a.sched.wg_start[blockIdx.x];
    if (it >= it_end) return;
    const int T = a.T, nqt = a.nqt;

    // The step after (sit, skt) of block sj: the next tile of the block, or
    // tile 0 of the next block of the list.  False at the end of the list.
    auto advance = [&](int &sit, int &skt, int &sbh, int &sj) {
        if (skt < sj) {
            ++skt;
            return true;
        }
        if (++sit >= it_end) return false;
        const int item = load_uniform_int(a.sched.items + sit);
        sbh = sched_bh(item);
        sj = sched_j(item);
        skt = 0;
        return true;
    };

    // Cooperative K tile load: thread (kg, c4) reads keys 4kg .. 4kg+3, dims
    // 4c4 .. 4c4+3 (rows past T read as zeros).
    const int kg = tid >> 4, c4 = tid & 15;
    const bool biased = a.kb != nullptr;  // the qkv bias is added to the K tile here
    f32x4 kpre[4];
    f32x4 kbias = zero4();  // bias of dims 4c4 .. 4c4+3 for the head of the tile in kpre
    auto prefetch_k = [&](int hbh, int kt) {
        const int hb = hbh / a.H, hh = hbh - hb * a.H;
        const auto k_rows = head_rows(a.k.p + hb * a.k.sb + hh * a.k.sh, T, a.k.st);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t key = kt * kBwdBQ + 4 * kg + c;
            kpre[c] = buffer_load4(k_rows, key * a.k.st + 4 * c4);
        }
        if (biased) kbias = *reinterpret_cast<const f32x4 *>(a.kb + hh * kDPad + 4 * c4);
    };
    // dS of the wave's 16 rows for tile kt of block jq: slice t (keys
    // 16t .. 16t+15) lies in block 2kt + t/2, columns 16(t%2) ...
    f32x4 dsn[4];
    auto prefetch_ds = [&](int hbh, int jq, int kt) {
        if (jq * kBwdBQ + 16 * w >= T) return;  // rows wholly past T: nothing to reduce
        const int nt = kt == jq ? w + 1 : 4;
        const float *base = a.ds + uniform(static_cast<uint32_t>(ds_block_offset(hbh - a.ds_bh0, nqt, jq, 2 * kt)));
        const uint32_t off = (16 * w + n) * 32 + 4 * j;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (t < nt) dsn[t] = stream_load(reinterpret_cast<const f32x4 *>(base + (t >> 1) * kDsBlock + off + 16 * (t & 1)));
    };

    int kt = 0, bh = sched_bh(a.sched.items[it]), jq = sched_j(a.sched.items[it]);
    prefetch_k(bh, 0);
    prefetch_ds(bh, jq, 0);
    int pit = it, pkt = 0, pbh = bh, pj = jq;  // the step whose loads are issued next
    bool pre_ok = advance(pit, pkt, pbh, pj);

    f32x4 acc[4];  // acc[db][r] = dQ[q0 + 4j + r][4n + db] before the 1/sqrt(D) scaling
    f32x4 dsc[4];
    auto tile = [&](auto nt_c) {
        constexpr int NT = decltype(nt_c)::value;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const f32x4 kb = *reinterpret_cast<const f32x4 *>(&k_lds[(4 * t + j) * kDq16KStride + 4 * (16 * db + n)]);
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[db] = mfma16(dsc[t][c], kb[c], acc[db]);
            }
    };

    for (;;) {
        const int q0 = jq * kBwdBQ + 16 * w;
        if (kt == 0) {
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = zero4();
        }

        __syncthreads();
        if (biased) {
            // K rows past T hold the bias too: the dS this kernel reads for
            // them is zero (the dk/dv kernel writes zeros for keys past T in
            // every 32-key block that holds a key below T).
#pragma unroll
            for (int c = 0; c < 4; ++c) kpre[c] += kbias;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f32x4 v = {kpre[0][e], kpre[1][e], kpre[2][e], kpre[3][e]};
            *reinterpret_cast<f32x4 *>(&k_lds[kg * kDq16KStride + 4 * (16 * e + c4)]) = v;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) dsc[t] = dsn[t];
        __syncthreads();
        if (pre_ok) {
            prefetch_k(pbh, pkt);
            prefetch_ds(pbh, pj, pkt);
            pre_ok = advance(pit, pkt, pbh, pj);
        }

        if (q0 < T) {  // wave-uniform
            if (kt != jq) {
                tile(IntC<4>{});
            } else {
                switch (w) {  // wave-uniform
                    case 0: tile(IntC<1>{}); break;
                    case 1: tile(IntC<2>{}); break;
                    case 2: tile(IntC<3>{}); break;
                    default: tile(IntC<4>{}); break;
                }
                // End of the block: dQ rows q0 + 4j + r.
                const int b = bh / a.H, h = bh - b * a.H;
                float *dQh = a.dq.p + b * a.dq.sb + h * a.dq.sh + 4 * n;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = q0 + 4 * j + r;
                    if (q < T) {
                        const f32x4 val = {acc[0][r] * a.scale, acc[1][r] * a.scale, acc[2][r] * a.scale,
                                           acc[3][r] * a.scale};
                        *reinterpret_cast<f32x4 *>(dQh + q * a.dq.st) = val;
                    }
                }
            }
        }
        if (a.db != nullptr && kt == jq) {
            // db of the q part: column sums of the block's 64 dQ rows (rows
            // < T) in a fixed order: registers, the 4 row groups j, waves.
            // Every wave takes part (waves wholly past T add zeros).
            f32x4 cs = zero4();
            if (q0 < T) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (q0 + 4 * j + r < T) cs += f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                cs[e] += __shfl_xor(cs[e], 16, 64);
                cs[e] += __shfl_xor(cs[e], 32, 64);
            }
            if (j == 0) *reinterpret_cast<f32x4 *>(&red_lds[w][4 * n]) = cs * a.scale;
            __syncthreads();
            if (tid < kDPad) {
                const int b = bh / a.H, h = bh - b * a.H;
                // red_lds[w][4n + e] holds dim 4n + e (acc[e] is dim 4n + e).
                const float s = (red_lds[0][tid] + red_lds[1][tid]) + (red_lds[2][tid] + red_lds[3][tid]);
                a.dbq_part[(static_cast<size_t>(b) * nqt + jq) * a.C + h * kDPad + tid] = s;
            }
        }
        if (!advance(it, kt, bh, jq)) break;
    }
}

// ---- dQ recomputing P and dP (the LSE-only backward, D == 64) ----
//
// For a forward that stored no P' (its state would not fit, or the caller
// capped it): the dk/dv kernel recomputes P and writes no dS, and this
// kernel forms dQ from the saved statistics alone.  It runs the forward's
// work lists (block_sched.hpp) with its tile layout: a workgroup is 4 waves
// x 16 queries of a 64-query block, K and V tiles of 64 keys are staged in
// LDS (prefetched one step ahead), and lane (g, i16) owns query i16 of the
// wave and keys 4g .. 4g+3 of each 16-key block.  Per tile:
//   S^T = K Q^T and dP^T = V dO^T (Q and dO rows in registers as B operands),
//   P = exp2(S log2(e)/sqrt(D) - LSE log2(e)), zero above the diagonal,
//   dS = P o (dP - delta),  dQ^T += K^T dS^T  (K rows as A operands, dS^T
//   straight from the accumulators, as O^T += V^T P^T in the forward).
// Three contractions per tile where the dq16 kernel reads dS and does one.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_bwd_dq16_recomp_kernel(const BwdParams a) {
    constexpr int LS = kLdsStride;
    __shared__ __attribute__((aligned(16))) float k_lds[kBwdBQ * LS];
    __shared__ __attribute__((aligned(16))) float v_lds[kBwdBQ * LS];
    __shared__ float red_lds[4][kDPad];  // db column sums of the block's dQ rows, per wave

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, g = lane >> 4, i16 = lane & 15;
    const int it_end = a.sched.wg_start[blockIdx.x + 1];
    int it = a.sched.wg_start[blockIdx.x];
    const int it_first = it;  // a register: re-reading the table would wait for every load in flight
    if (it >= it_end) return;
    const int T = a.T;
    const float c2 = a.scale * kLog2e;

    auto advance = [&](int &sit, int &skt, int &sbh, int &sj) {
        if (skt < sj) {
            ++skt;
            return true;
        }
        if (++sit >= it_end) return false;
        const int item = load_uniform_int(a.sched.items + sit);
        sbh = sched_bh(item);
        sj = sched_j(item);
        skt = 0;
        return true;
    };

    // Cooperative K/V tile load: thread covers rows (tid >> 4) + 16i, dims
    // 4 (tid & 15); rows past T read as zeros.  With the qkv bias folded in,
    // each thread adds the k and v bias of its dims as it stores the tile.
    const int ld_row = tid >> 4, ld_col = 4 * (tid & 15);
    const bool biased = a.kb != nullptr;
    f32x4 kpre[4], vpre[4], kb4 = zero4(), vb4 = zero4();
    auto load_tile = [&](int hbh, int kt) {
        const int hb = hbh / a.H, hh = hbh - hb * a.H;
        const auto k_rows = head_rows(a.k.p + hb * a.k.sb + hh * a.k.sh, T, a.k.st);
        const auto v_rows = head_rows(a.v.p + hb * a.v.sb + hh * a.v.sh, T, a.v.st);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t key = kt * kBwdBQ + ld_row + 16 * i;
            kpre[i] = buffer_load4(k_rows, key * a.k.st + ld_col);
            vpre[i] = buffer_load4(v_rows, key * a.v.st + ld_col);
        }
        if (biased) {
            kb4 = *reinterpret_cast<const f32x4 *>(a.kb + hh * kDPad + ld_col);
            vb4 = *reinterpret_cast<const f32x4 *>(a.vb + hh * kDPad + ld_col);
        }
    };

    int kt = 0, bh = sched_bh(a.sched.items[it]), jq = sched_j(a.sched.items[it]);
    // The wave's rows of the current block: Q (with its bias) and dO as B
    // operands (qr[c][e] = Q[my_q][16g + 4c + e]), and the query's LSE log2(e)
    // and delta (rows past T read a clamped row and are never stored).
    f32x4 qr[4], dor[4];
    float lse2 = 0.0f, dl = 0.0f;
    int my_q = 0;
    auto load_rows = [&]() {
        const int b = bh / a.H, h = bh - b * a.H;
        my_q = jq * kBwdBQ + 16 * w + i16;
        const auto q_rows = head_rows(a.q.p + b * a.q.sb + h * a.q.sh, T, a.q.st);
        const auto d_rows = head_rows(a.dout.p + b * a.dout.sb + h * a.dout.sh, T, a.dout.st);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            qr[c] = buffer_load4(q_rows, static_cast<uint32_t>(my_q) * a.q.st + 16 * g + 4 * c);
            dor[c] = buffer_load4(d_rows, static_cast<uint32_t>(my_q) * a.dout.st + 16 * g + 4 * c);
            if (biased) qr[c] += *reinterpret_cast<const f32x4 *>(a.qb + h * kDPad + 16 * g + 4 * c);
        }
        const int qc = min(my_q, T - 1);
        lse2 = a.lse[static_cast<uint32_t>(bh) * T + qc] * kLog2e;
        dl = a.delta[static_cast<uint32_t>(bh) * T + qc];
    };
    load_rows();
    load_tile(bh, 0);
    int pit = it, pkt = 0, pbh = bh, pj = jq;  // the step whose tile is loaded next
    bool pre_ok = advance(pit, pkt, pbh, pj);

    f32x4 acc[4];  // dQ^T: acc[db][r] = dQ[my_q][16g + 4r + db] before the 1/sqrt(D) scaling
    // One key tile: NKB 16-key blocks visible to the wave's queries (DIAG:
    // the block's own tile, block NKB - 1 masked per key).
    auto tile = [&](auto nkb_c, auto diag_c) {
        constexpr int NKB = decltype(nkb_c)::value;
        constexpr bool DIAG = decltype(diag_c)::value;
        f32x4 sc[4], dp[4];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sc[kb] = dp[kb] = zero4();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f32x4 ka[NKB], va[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                ka[kb] = *reinterpret_cast<const f32x4 *>(&k_lds[(16 * kb + i16) * LS + 16 * g + 4 * c]);
                va[kb] = *reinterpret_cast<const f32x4 *>(&v_lds[(16 * kb + i16) * LS + 16 * g + 4 * c]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    sc[kb] = mfma16(ka[kb][e], qr[c][e], sc[kb]);
                    dp[kb] = mfma16(va[kb][e], dor[c][e], dp[kb]);
                }
        }
        // dS in place of S: sc[kb][r] is key 16kb + 4g + r of the tile.
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float p = fast_exp2(fmaf(sc[kb][r], c2, -lse2));
                if (DIAG && kb == NKB - 1 && 4 * g + r > i16) p = 0.0f;
                sc[kb][r] = p * (dp[kb][r] - dl);
            }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const f32x4 ka = *reinterpret_cast<const f32x4 *>(&k_lds[(16 * kb + 4 * g + r) * LS + 4 * i16]);
#pragma unroll
                for (int db = 0; db < 4; ++db) acc[db] = mfma16(ka[db], sc[kb][r], acc[db]);
            }
    };

    for (;;) {
        if (kt == 0) {
            if (it != it_first) load_rows();
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = zero4();
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = ld_row + 16 * i;
            *reinterpret_cast<f32x4 *>(&k_lds[row * LS + ld_col]) = kpre[i] + kb4;
            *reinterpret_cast<f32x4 *>(&v_lds[row * LS + ld_col]) = vpre[i] + vb4;
        }
        __syncthreads();
        if (pre_ok) {
            load_tile(pbh, pkt);
            pre_ok = advance(pit, pkt, pbh, pj);
        }

        const bool diag = kt == jq;
        const int q0 = jq * kBwdBQ + 16 * w;
        if (q0 < T) {  // wave-uniform
            if (!diag) {
                tile(IntC<4>{}, std::false_type{});
            } else {
                switch (w) {  // wave-uniform
                    case 0: tile(IntC<1>{}, std::true_type{}); break;
                    case 1: tile(IntC<2>{}, std::true_type{}); break;
                    case 2: tile(IntC<3>{}, std::true_type{}); break;
                    default: tile(IntC<4>{}, std::true_type{}); break;
                }
                if (my_q < T) {
                    const int b = bh / a.H, h = bh - b * a.H;
                    float *row = a.dq.p + b * a.dq.sb + my_q * a.dq.st + h * a.dq.sh + 16 * g;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        *reinterpret_cast<f32x4 *>(row + 4 * r) =
                            f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]} * a.scale;
                }
            }
        }
        if (a.db != nullptr && diag) {
            // db of the q part: column sums of the block's 64 dQ rows (rows
            // < T) in a fixed order: the 16 queries of a wave (lanes of one
            // g), then the 4 waves.  Lane (g, i16) holds dims 16g + 4r + db.
            f32x4 cs[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool ok = q0 < T && my_q < T;
                cs[r] = ok ? f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]} : zero4();
#pragma unroll
                for (int off = 1; off < 16; off <<= 1)
#pragma unroll
                    for (int e = 0; e < 4; ++e) cs[r][e] += __shfl_xor(cs[r][e], off, 64);
            }
            if (i16 == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) *reinterpret_cast<f32x4 *>(&red_lds[w][16 * g + 4 * r]) = cs[r] * a.scale;
            }
            __syncthreads();
            if (tid < kDPad) {
                const int b = bh / a.H, h = bh - b * a.H;
                const float s = (red_lds[0][tid] + red_lds[1][tid]) + (red_lds[2][tid] + red_lds[3][tid]);
                a.dbq_part[(static_cast<size_t>(b) * a.nqt + jq) * a.C + h * kDPad + tid] = s;
            }
        }
        if (!advance(it, kt, bh, jq)) break;
    }
}

int bwd_split_plan(BwdParams &p, hipStream_t stream) {
    p.nsplit = 0;
    p.k_wg = 0;
    p.ksched = KeySched{nullptr, nullptr};
    if (!p.full || p.nqt <= kShortHeadTiles || p.ds == nullptr) return 0;  // the recomputing dk/dv runs whole blocks
    // The LSE-only scratch in chunks of heads: no split blocks (their db
    // partial rows would differ between chunks); the lists are built per
    // chunk by launch_attn_bwd.
    if (p.lse_only && p.ds_heads < p.B * p.H) return 0;
    // Both instances of a kernel keep two workgroups per CU; the lists are
    // built for the residency of the one without the bias.
    const void *kernel = p.lse_only ? reinterpret_cast<const void *>(attn_bwd_dkdv_dma_kernel<false, true>)
                                    : reinterpret_cast<const void *>(attn_bwd_dkdv_dma_kernel<false, false>);
    p.ksched = device_key_schedule(p.B * p.H, p.nqt, kernel, stream, &p.k_wg, &p.nsplit);
    return p.nsplit;
}

size_t bwd_ds_floats(int B, int H, int T) {
    const size_t nqt = (T + kBwdBQ - 1) / kBwdBQ;
    return static_cast<size_t>(B) * H * nqt * (nqt + 1) * kDsBlock;
}

void launch_attn_bwd(const BwdParams &p_in, hipStream_t stream, const hipEvent_t *ev) {
    BwdParams p = p_in;
    const bool wide = p.D > kDPad;  // 64 < D <= 128: the DP = 128 kernels
    // The 32-row dq kernel for head sizes other than 64, and its grid order
    // (the 16-row one runs work lists).
    const void *dq_kern = nullptr;
    if (!p.full) {
        if (wide)
            dq_kern = p.vec ? reinterpret_cast<const void *>(attn_bwd_dq_kernel<true, 2 * kDPad>)
                            : reinterpret_cast<const void *>(attn_bwd_dq_kernel<false, 2 * kDPad>);
        else
            dq_kern = p.vec ? reinterpret_cast<const void *>(attn_bwd_dq_kernel<true, kDPad>)
                            : reinterpret_cast<const void *>(attn_bwd_dq_kernel<false, kDPad>);
        p.dq_order = choose_grid_order(p.nqb, p.bh_pad, dq_kern);
    }
    const dim3 block(256);
    const int rows = p.B * p.T * p.H;
    const dim3 grid_d((rows + 15) / 16), grid_k(p.nkb * p.bh_pad), grid_q(p.nqb * p.bh_pad);
    if (ev) hipCheck(hipEventRecord(ev[0], stream));
    if (p.vec)
        attn_bwd_delta_kernel<true><<<grid_d, block, 0, stream>>>(p);
    else
        attn_bwd_delta_kernel<false><<<grid_d, block, 0, stream>>>(p);
    hipCheck(hipGetLastError());
    if (ev) {
        hipCheck(hipEventRecord(ev[1], stream));
        hipCheck(hipEventRecord(ev[2], stream));
    }
    if (p.D > 2 * kDPad) {
        launch_attn_bwd_generic(p, stream, ev);
        if (ev) hipCheck(hipEventRecord(ev[5], stream));
        return;
    }
    if (p.full && p.lse_only && p.ds != nullptr && p.nqt > kShortHeadTiles) {
        // The LSE-only state with a dS scratch: per chunk of heads, dK/dV
        // recomputing P (dS into the scratch), then dQ from that dS.  With
        // more than one chunk the events bracket the whole loop as dk/dv.
        const int BH = p.B * p.H;
        const bool chunked = p.ds_heads < BH;
        const void *kern = reinterpret_cast<const void *>(attn_bwd_dkdv_dma_kernel<false, true>);
        for (int bh0 = 0; bh0 < BH; bh0 += p.ds_heads) {
            const int nbh = std::min(p.ds_heads, BH - bh0);
            BwdParams c = p;
            c.ds_bh0 = bh0;
            if (chunked) {
                int ns = 0;
                c.ksched = device_key_schedule(nbh, p.nqt, kern, stream, &c.k_wg, &ns, bh0, 0);
                c.nsplit = 0;
            }
            if (c.qb != nullptr)
                attn_bwd_dkdv_dma_kernel<true, true><<<dim3(c.k_wg), block, 0, stream>>>(c);
            else
                attn_bwd_dkdv_dma_kernel<false, true><<<dim3(c.k_wg), block, 0, stream>>>(c);
            hipCheck(hipGetLastError());
            if (ev && bh0 == 0 && !chunked) {
                hipCheck(hipEventRecord(ev[3], stream));
                hipCheck(hipEventRecord(ev[4], stream));
            }
            int num_wg = 0;
            c.sched = device_block_schedule(nbh, p.nqt, reinterpret_cast<const void *>(attn_bwd_dq16_kernel), stream,
                                            &num_wg, bh0);
            attn_bwd_dq16_kernel<<<dim3(num_wg), block, 0, stream>>>(c);
            hipCheck(hipGetLastError());
        }
        if (ev && chunked) {
            hipCheck(hipEventRecord(ev[3], stream));
            hipCheck(hipEventRecord(ev[4], stream));
        }
        if (ev) hipCheck(hipEventRecord(ev[5], stream));
        return;
    }
    if (p.full && (p.nqt <= kShortHeadTiles || p.ds == nullptr))
        attn_bwd_dkdv_kernel<true, true, true><<<grid_k, block, 0, stream>>>(p);
    else if (p.full && p.qb != nullptr)
        attn_bwd_dkdv_dma_kernel<true, false><<<dim3(p.k_wg), block, 0, stream>>>(p);
    else if (p.full)
        attn_bwd_dkdv_dma_kernel<false, false><<<dim3(p.k_wg), block, 0, stream>>>(p);
    else if (wide && p.vec)
        attn_bwd_dkdv_kernel<true, false, false, 2 * kDPad><<<grid_k, block, 0, stream>>>(p);
    else if (wide)
        attn_bwd_dkdv_kernel<false, false, false, 2 * kDPad><<<grid_k, block, 0, stream>>>(p);
    else if (p.vec)
        attn_bwd_dkdv_kernel<true, false, false><<<grid_k, block, 0, stream>>>(p);
    else
        attn_bwd_dkdv_kernel<false, false, false><<<grid_k, block, 0, stream>>>(p);
    hipCheck(hipGetLastError());
    if (ev) {
        hipCheck(hipEventRecord(ev[3], stream));
        hipCheck(hipEventRecord(ev[4], stream));
    }
    if (p.full && p.ds == nullptr) {
        int num_wg = 0;
        p.sched = device_block_schedule(p.B * p.H, p.nqt,
                                        reinterpret_cast<const void *>(attn_bwd_dq16_recomp_kernel), stream, &num_wg);
        attn_bwd_dq16_recomp_kernel<<<dim3(num_wg), block, 0, stream>>>(p);
    } else if (p.full) {
        int num_wg = 0;
        p.sched = device_block_schedule(p.B * p.H, p.nqt, reinterpret_cast<const void *>(attn_bwd_dq16_kernel),
                                        stream, &num_wg);
        attn_bwd_dq16_kernel<<<dim3(num_wg), block, 0, stream>>>(p);
    }
    else {
        void *args[] = {&p};
        hipCheck(hipLaunchKernel(dq_kern, grid_q, block, args, 0, stream));
    }
    hipCheck(hipGetLastError());
    if (ev) hipCheck(hipEventRecord(ev[5], stream));
}

}  // namespace gptc
