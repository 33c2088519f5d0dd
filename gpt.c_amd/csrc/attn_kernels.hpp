// Host-visible launch parameters of the attention kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include "attn_common.hpp"

namespace gptc {

struct FwdParams {
    HeadView q, k, v;     // inputs
    HeadViewW o;          // y (B, T, C)
    float *o2;            // optional copy of y, same strides as o (nullptr: none)
    float *lse;           // (B, H, T) natural-log row log-sum-exp
    float *qp, *kp, *vp;  // optional permuted copies (B, H, T, D) (nullptr: none)
    int B, H, T, D;
    float scale_log2;     // log2(e) / sqrt(D)
    int nqb;              // ceil(T / 128)
    int bh_pad;           // B*H rounded up to a multiple of 8
    bool vec;             // D % 4 == 0 and every row 16-byte aligned
};

struct BwdParams {
    HeadView q, k, v;     // saved inputs
    HeadView o;           // saved y
    HeadView dout;        // upstream gradient dy (B, T, C)
    const float *lse;     // (B, H, T)
    float *delta;         // (B, H, T) rowsum(dy * y), written by the dq kernel
    HeadViewW dq, dk, dv; // slices of dqkv (B, T, 3C)
    int B, H, T, D;
    float scale_log2;     // log2(e) / sqrt(D)
    float scale;          // 1 / sqrt(D)
    int nqb;              // ceil(T / 128) query blocks (dq kernel)
    int nkb;              // ceil(T / 128) key blocks (dk/dv kernel)
    int bh_pad;
    bool vec;
};

// ev: optional events recorded on `stream` around each kernel launch
// (forward: ev[0], ev[1]; backward: ev[0..1] around the dq kernel and
// ev[2..3] around the dk/dv kernel).  nullptr: no events.
void launch_attn_fwd(const FwdParams &p, hipStream_t stream, const hipEvent_t *ev);
void launch_attn_bwd(const BwdParams &p, hipStream_t stream, const hipEvent_t *ev);

}  // namespace gptc
