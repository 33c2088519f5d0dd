// Host-visible launch parameters of the attention kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include "attn_common.hpp"
#include "block_sched.hpp"
#include "grid_order.hpp"

namespace gptc {

// The forward hands the backward the softmax probabilities it computed, so
// that the backward needs no S = QK^T recomputation.  It stores them as
//     P'[q][k] = exp2(S[q][k] * log2(e)/sqrt(D) - m[q][kt])
// where m[q][kt] is the running row maximum (log2 units) that the forward
// used for 64-key tile kt; the backward recovers
//     P[q][k] = P'[q][k] * exp2(m[q][kt] - lse[q] * log2(e)).
// P' and, in the backward, dS (which overwrites P' in place) share one packed
// layout: per (b, h), for each 64-query tile qt the 32-key blocks
// kb32 = 0 .. 2qt+1 (all that the causal rule leaves non-zero) follow one
// another; block (qt, kb32) is a row-major [64 queries][32 keys] array.
constexpr int kDsBlock = 64 * 32;

__host__ __device__ inline size_t ds_block_offset(int bh, int nqt, int qt, int kb32) {
    return (static_cast<size_t>(bh) * nqt * (nqt + 1) + static_cast<size_t>(qt) * (qt + 1) + kb32) * kDsBlock;
}

// Short heads: at most this many 64-key tiles (T <= 128).  Their forward
// (D = 64) is latency-bound: it prefetches two tiles ahead and does not
// store P' or m; their dk/dv kernel recomputes P = exp2(S log2(e)/sqrt(D)
// - LSE log2(e)) from Q, K and the saved LSE instead.  The dS blocks keep
// their place in the state either way.
constexpr int kShortHeadTiles = 2;

// Floats of the packed P' / dS blocks for a (B, H, T) problem.
size_t bwd_ds_floats(int B, int H, int T);

struct FwdParams {
    HeadView q, k, v;     // inputs
    HeadViewW o;          // y (B, T, C)
    float *o2;            // optional copy of y, same strides as o (nullptr: none)
    float *lse;           // (B, H, T) natural-log row log-sum-exp
    float *qp, *kp, *vp;  // optional permuted copies (B, H, T, D) (nullptr: none)
    float *pp;            // P' blocks, bwd_ds_floats(B, H, T) floats
    float *pm;            // m, (B, H, nqt, T): m of query q for key tile kt at (bh*nqt + kt)*T + q
    int B, H, T, D;
    float scale_log2;     // log2(e) / sqrt(D)
    int nqb;              // ceil(T / 128)
    int nqt;              // ceil(T / 64)
    int bh_pad;           // B*H rounded up to a multiple of 8
    bool vec;             // D % 4 == 0 and every row 16-byte aligned
    bool full;            // vec, D == kDPad and every head's rows span < 2^31 bytes
    GridOrder order;      // grid order of the 32-row kernel (set by launch_attn_fwd)
    BlockSched sched;     // work lists of the 16-row kernel (set by launch_attn_fwd)
    // Bias of the qkv Linear, added to q, k, v as they are loaded (16-row
    // kernel only; nullptr: the input already holds x W^T + b).  Head h's
    // entries are qb[h*D + d], kb[h*D + d], vb[h*D + d].
    const float *qb, *kb, *vb;
};

struct BwdParams {
    HeadView q, k, v;     // saved inputs
    HeadView o;           // saved y
    HeadView dout;        // upstream gradient dy (B, T, C)
    const float *lse;     // (B, H, T)
    const float *pm;      // m saved by the forward, (B, H, nqt, T)
    float *delta;         // (B, H, T) rowsum(dy * y), written by the delta kernel
    float *ds;            // in: P' from the forward; out: dS (same packed blocks)
    HeadViewW dq, dk, dv; // slices of dqkv (B, T, 3C)
    int B, H, T, D;
    float scale;          // 1 / sqrt(D)
    int nqb;              // ceil(T / 128) query blocks (dq kernel)
    int nkb;              // ceil(T / 128) key blocks (dk/dv kernel)
    int nqt;              // ceil(T / 64) query tiles of the P' / dS blocks
    int bh_pad;
    bool vec;
    bool full;            // vec, D == kDPad and every head's rows span < 2^31 bytes
    GridOrder dq_order;   // grid order of the 32-row dq kernel (set by launch_attn_bwd)
    BlockSched sched;     // work lists of the 16-row dq kernel (set by launch_attn_bwd)
    // The qkv Linear's bias folded into the loads (as in FwdParams; D = 64
    // kernels only), and its gradient: per-workgroup column sums of the dq
    // rows ((B*nqt) x C, one row per 64-query block) and of the dk | dv rows
    // ((B*nkb) x 2C, one row per 128-key block), reduced in a fixed order into
    // db (3C, accumulated) by the last kernel.  db == nullptr: none of this.
    const float *qb, *kb, *vb;
    float *dbq_part, *dbkv_part, *db;
    int C;
    // Work lists of the D = 64 dk/dv kernel with the stored P' (block_sched.hpp):
    // key blocks kb < nsplit are cut by query range into two items, which add
    // their dK, dV parts into rows that the delta kernel zeroed (two addends:
    // the sum is the same in either order).  The db partials then hold
    // B * (nkb + nsplit) rows (the item that does not start on the diagonal
    // writes row nkb + kb).
    int nsplit;
    KeySched ksched;
    int k_wg;  // workgroups of the work-list launch
    // The LSE-only state (the forward kept no P'): with ds set, it is a
    // scratch of the packed blocks of ds_heads heads at a time, which the
    // recomputing dk/dv kernel fills with dS and the dq16 kernel reads; the
    // heads run in chunks [ds_bh0, ds_bh0 + ds_heads) (ds_bh0 set per chunk
    // by launch_attn_bwd).  ds == nullptr: both gradient kernels recompute P.
    bool lse_only;
    int ds_heads;
    int ds_bh0;
};

// Sets p.nsplit, p.ksched and p.k_wg for the D = 64 dk/dv kernel of p's
// shape on the current device (building and uploading the work lists on
// `stream` on first use; nsplit = 0 for the other kernels) and returns nsplit.
int bwd_split_plan(BwdParams &p, hipStream_t stream);

// One KV-cache decode step (attn_decode.hip).
struct DecParams {
    const float *qkv;     // (B, 1, 3C): the new token's q | k | v
    float *k_cache;       // (B, H, L, D); row pos is written
    float *v_cache;       // (B, H, L, D); row pos is written
    float *out;           // (B, 1, C)
    int B, H, C, D, L;
    int pos;              // position of the new token; keys 0 .. pos are attended
    const int *pos_dev;   // if set, the position is read from device memory instead
                          // (graph replays); the score buffer is then sized for L keys
    float scale_log2;     // log2(e) / sqrt(D)
    bool full;            // D == kDPad and 16-byte aligned cache rows
    float *part;          // if set (and full): split-key partials, B*H*splits*kDecPartStride floats
    int splits;           // key chunks of kDecChunk per (b, h) (split path)
};

constexpr int kDecMaxKeys = 8192;  // pos + 1 limit (the scores live in LDS)
constexpr int kDecChunk = 64;      // keys per workgroup of the split-key decode
constexpr int kDecPartStride = 68; // floats per partial: o[64], m, l, 2 unused

constexpr int kDecHeadKeys = 512;  // keys the one-launch decode (one workgroup per (b, h)) takes

// Whether a decode step runs the one-launch kernel: D == 64 with 16-byte
// rows, and at most kDecHeadKeys keys (pos + 1, or the cache length L when
// the position is read on the device).  Longer steps run the split pair.
inline bool dec_head_fits(const DecParams &p) {
    return p.full && (p.pos_dev != nullptr ? p.L : p.pos + 1) <= kDecHeadKeys;
}

// Floats of the partials buffer of the split-key decode for B sequences of
// H heads attending up to n_keys keys.
inline size_t dec_part_floats(int B, int H, int n_keys) {
    return static_cast<size_t>(B) * H * ((n_keys + kDecChunk - 1) / kDecChunk) * kDecPartStride;
}

void launch_attn_decode(const DecParams &p, hipStream_t stream);

// ev: optional events recorded on `stream` around each kernel launch
// (forward: ev[0], ev[1]; backward: ev[0..1] around the delta kernel,
// ev[2..3] around the dk/dv kernel, ev[4..5] around the dq kernel).
// nullptr: no events.
void launch_attn_fwd(const FwdParams &p, hipStream_t stream, const hipEvent_t *ev);
void launch_attn_bwd(const BwdParams &p, hipStream_t stream, const hipEvent_t *ev);

// Head sizes past 2 * kDPad, up to kGenericMaxD: plain-FMA kernels
// (attn_generic.hip) with the LSE-only state.  The backward launcher runs
// the dk/dv and dq kernels (the delta kernel is launch_attn_bwd's) and
// records ev[3], ev[4] between them.
constexpr int kGenericMaxD = 1024;
void launch_attn_fwd_generic(const FwdParams &p, hipStream_t stream);
void launch_attn_bwd_generic(const BwdParams &p, hipStream_t stream, const hipEvent_t *ev);

}  // namespace gptc
