// C-ABI entry points of the causal attention path: shape and layout checks
// on the host, then the fused HIP kernels on the library stream.
// Replaces kernels/src/cuda/Attention.cu:170-324 behind the signatures of
// kernels/src/cuda/Attention.h:9-22 (called by
// kernels/src/core/Attention.c:40-41,75-76).
#include <cmath>
#include <cstdint>
#include "attn_kernels.hpp"
#include "gpu_kernels.h"
#include "hip_check.hpp"
#include "utils.h"

namespace {

using gptc::BwdParams;
using gptc::FwdParams;
using gptc::HeadView;
using gptc::HeadViewW;

struct Dims {
    int B, T, C, H, D;
};

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int bh_padded(int bh) { return (bh + 7) / 8 * 8; }

void check_head_size(const Dims &d) {
    CHECK_ERROR(d.H <= 0 || d.C % d.H != 0, "Expected C = %d to be divisible by n_heads = %d.", d.C, d.H);
    CHECK_ERROR(d.D < 1 || d.D > gptc::kDPad,
                "Head size %d is not supported by the GPU attention kernels (1 <= n_embd / n_heads <= %d).", d.D,
                gptc::kDPad);
}

// Views of q, k, v inside a (B, T, 3C) qkv tensor.
void qkv_views(const float *x, const Dims &d, HeadView &q, HeadView &k, HeadView &v) {
    const uint32_t sb = static_cast<uint32_t>(d.T) * 3 * d.C, st = 3 * d.C, sh = d.D;
    q = HeadView{x, sb, st, sh};
    k = HeadView{x + d.C, sb, st, sh};
    v = HeadView{x + 2 * d.C, sb, st, sh};
}

// View of one (B, H, T, D) tensor.
HeadView bhtd_view(const float *p, const Dims &d) {
    return HeadView{p, static_cast<uint32_t>(d.H) * d.T * d.D, static_cast<uint32_t>(d.D),
                    static_cast<uint32_t>(d.T) * d.D};
}

// View of a (B, T, C) tensor split into heads.
template <typename V, typename P>
V btc_view(P p, const Dims &d) {
    return V{p, static_cast<uint32_t>(d.T) * d.C, static_cast<uint32_t>(d.C), static_cast<uint32_t>(d.D)};
}

bool is_bhtd(const tensor_t *t, const Dims &d) {
    return t->ndims == 4 && t->shape[0] == d.B && t->shape[1] == d.H && t->shape[2] == d.T && t->shape[3] == d.D;
}

// Floats of the compact state kept in cache[3] by the reference cache
// layout: y copy (B*T*C), log-sum-exp (B*H*T), delta scratch (B*H*T).
int64_t packed_state_len(const Dims &d) {
    return static_cast<int64_t>(d.B) * d.T * d.C + 2LL * d.B * d.H * d.T;
}

// Events registered by gptc_set_kernel_events: [0,1] around the forward
// kernel, then [2,3] delta, [4,5] dk/dv and [6,7] dq of the backward.
constexpr int kNumEvents = 8;
hipEvent_t g_events[kNumEvents];
bool g_have_events = false;

}  // namespace

extern "C" void gptc_set_kernel_events(void **events, int n) {
    if (events == NULL) {
        g_have_events = false;
        return;
    }
    CHECK_ERROR(n != kNumEvents,
                "Expected %d events (start and end of forward, delta, dk/dv and dq kernels), but got %d.",
                kNumEvents, n);
    for (int i = 0; i < kNumEvents; i++) g_events[i] = static_cast<hipEvent_t>(events[i]);
    g_have_events = true;
}

extern "C" void attention_forward_cuda_kernel(const tensor_t *input, const tensor_t *mask, const int n_heads,
                                              tensor_t **cache, tensor_t *output) {
    CHECK_ERROR(input == NULL || mask == NULL || output == NULL || cache == NULL,
                "Expected input, mask, cache and output to be non-NULL.");
    for (int i = 0; i < 4; i++) CHECK_ERROR(cache[i] == NULL, "Expected cache[%d] to be allocated.", i);
    CHECK_ERROR(input->ndims != 3, "Expected input of shape (B, T, 3C), but got %d dims.", input->ndims);
    CHECK_ERROR(input->shape[2] % 3 != 0, "Expected the last dim of input to be 3C, but got %d.", input->shape[2]);

    Dims d;
    d.B = input->shape[0];
    d.T = input->shape[1];
    d.C = input->shape[2] / 3;
    d.H = n_heads;
    CHECK_ERROR(d.H <= 0, "Expected n_heads > 0, but got %d.", d.H);
    d.D = d.C / d.H;
    check_head_size(d);

    CHECK_ERROR(mask->ndims < 2, "Expected a 2-D (block, block) mask, but got %d dims.", mask->ndims);
    const int mrows = mask->shape[mask->ndims - 2], mcols = mask->shape[mask->ndims - 1];
    CHECK_ERROR(mrows < d.T || mcols < d.T, "Sequence length T = %d exceeds the mask (block size %d x %d).", d.T,
                mrows, mcols);
    CHECK_ERROR(output->length != d.B * d.T * d.C, "Expected output of %d elements, but got %d.", d.B * d.T * d.C,
                output->length);
    if (d.B == 0 || d.T == 0 || d.C == 0) return;

    FwdParams p{};
    qkv_views(input->t, d, p.q, p.k, p.v);
    p.o = btc_view<HeadViewW>(output->t, d);
    const int64_t bht = static_cast<int64_t>(d.B) * d.H * d.T;

    if (cache[0] == input || cache[0]->t == input->t) {
        // Compact layout: the layer keeps the input itself.
        CHECK_ERROR(cache[1]->length != output->length, "Expected cache[1] of %d elements (copy of the output).",
                    output->length);
        CHECK_ERROR(cache[2]->length < bht || cache[3]->length < bht,
                    "Expected cache[2] and cache[3] of at least B*H*T = %lld elements.", (long long)bht);
        p.o2 = cache[1]->t;
        p.lse = cache[2]->t;
        p.qp = p.kp = p.vp = nullptr;
    } else {
        // Reference layout (gpt.c attention.c:105-120): permuted q, k, v go to
        // cache[0..2]; cache[3] is re-pointed to the compact state.
        for (int i = 0; i < 3; i++)
            CHECK_ERROR(!is_bhtd(cache[i], d), "Expected cache[%d] of shape (B, H, T, D) = (%d, %d, %d, %d).", i, d.B,
                        d.H, d.T, d.D);
        const int64_t need = packed_state_len(d);
        if (cache[3]->length != need || cache[3]->ndims != 1) {
            free_cuda(cache[3]->t);
            cache[3]->t = static_cast<float *>(alloc_cuda(static_cast<size_t>(need) * sizeof(float)));
            cache[3]->ndims = 1;
            cache[3]->length = static_cast<int>(need);
            for (int i = 0; i < 8; i++) cache[3]->shape[i] = 0;
            cache[3]->shape[0] = static_cast<int>(need);
        }
        p.o2 = cache[3]->t;
        p.lse = cache[3]->t + static_cast<int64_t>(d.B) * d.T * d.C;
        p.qp = cache[0]->t;
        p.kp = cache[1]->t;
        p.vp = cache[2]->t;
    }

    p.B = d.B;
    p.H = d.H;
    p.T = d.T;
    p.D = d.D;
    p.scale_log2 = gptc::kLog2e / std::sqrt(static_cast<float>(d.D));
    p.nqb = (d.T + 127) / 128;
    p.bh_pad = bh_padded(d.B * d.H);
    p.vec = (d.D % 4 == 0) && aligned16(input->t) && aligned16(output->t) && aligned16(p.o2) &&
            (!p.qp || (aligned16(p.qp) && aligned16(p.kp) && aligned16(p.vp)));
    gptc::launch_attn_fwd(p, gptc_stream_checked(), g_have_events ? g_events : nullptr);
}

extern "C" void attention_backward_cuda_kernel(const tensor_t *global_grad, tensor_t **cache, const int n_heads,
                                               tensor_t *dout) {
    CHECK_ERROR(global_grad == NULL || cache == NULL || dout == NULL,
                "Expected global_grad, cache and dout to be non-NULL.");
    for (int i = 0; i < 4; i++)
        CHECK_ERROR(cache[i] == NULL, "Expected cache[%d] to be allocated (was forward called?).", i);
    CHECK_ERROR(global_grad->ndims != 3, "Expected global_grad of shape (B, T, C), but got %d dims.",
                global_grad->ndims);

    Dims d;
    d.B = global_grad->shape[0];
    d.T = global_grad->shape[1];
    d.C = global_grad->shape[2];
    d.H = n_heads;
    CHECK_ERROR(d.H <= 0, "Expected n_heads > 0, but got %d.", d.H);
    d.D = d.C / d.H;
    check_head_size(d);
    CHECK_ERROR(dout->length != 3 * d.B * d.T * d.C, "Expected dout of shape (B, T, 3C) = %d elements, but got %d.",
                3 * d.B * d.T * d.C, dout->length);
    if (d.B == 0 || d.T == 0 || d.C == 0) return;

    BwdParams p{};
    const int64_t btc = static_cast<int64_t>(d.B) * d.T * d.C;
    const int64_t bht = static_cast<int64_t>(d.B) * d.H * d.T;
    const tensor_t *c0 = cache[0];
    const float *state = nullptr;
    if (c0->ndims == 3 && c0->shape[0] == d.B && c0->shape[1] == d.T && c0->shape[2] == 3 * d.C) {
        CHECK_ERROR(cache[1]->length != btc, "Expected cache[1] of B*T*C = %lld elements.", (long long)btc);
        CHECK_ERROR(cache[2]->length < bht || cache[3]->length < bht,
                    "Expected cache[2] and cache[3] of at least B*H*T = %lld elements.", (long long)bht);
        qkv_views(c0->t, d, p.q, p.k, p.v);
        p.o = btc_view<HeadView>(static_cast<const float *>(cache[1]->t), d);
        p.lse = cache[2]->t;
        p.delta = cache[3]->t;
        state = cache[1]->t;
    } else {
        for (int i = 0; i < 3; i++)
            CHECK_ERROR(!is_bhtd(cache[i], d), "Expected cache[%d] of shape (B, H, T, D) = (%d, %d, %d, %d).", i, d.B,
                        d.H, d.T, d.D);
        CHECK_ERROR(cache[3]->ndims != 1 || cache[3]->length != packed_state_len(d),
                    "cache[3] does not hold the state written by attention_forward_cuda_kernel for this shape.");
        p.q = bhtd_view(cache[0]->t, d);
        p.k = bhtd_view(cache[1]->t, d);
        p.v = bhtd_view(cache[2]->t, d);
        p.o = btc_view<HeadView>(static_cast<const float *>(cache[3]->t), d);
        p.lse = cache[3]->t + btc;
        p.delta = cache[3]->t + btc + bht;
        state = cache[3]->t;
    }
    p.dout = btc_view<HeadView>(static_cast<const float *>(global_grad->t), d);
    const uint32_t sb3 = static_cast<uint32_t>(d.T) * 3 * d.C, st3 = 3 * d.C;
    p.dq = HeadViewW{dout->t, sb3, st3, static_cast<uint32_t>(d.D)};
    p.dk = HeadViewW{dout->t + d.C, sb3, st3, static_cast<uint32_t>(d.D)};
    p.dv = HeadViewW{dout->t + 2 * d.C, sb3, st3, static_cast<uint32_t>(d.D)};

    p.B = d.B;
    p.H = d.H;
    p.T = d.T;
    p.D = d.D;
    p.scale = 1.0f / std::sqrt(static_cast<float>(d.D));
    p.scale_log2 = gptc::kLog2e * p.scale;
    p.nqb = (d.T + 127) / 128;
    p.nkb = (d.T + 127) / 128;
    p.nqt = (d.T + 63) / 64;
    p.bh_pad = bh_padded(d.B * d.H);
    p.vec = (d.D % 4 == 0) && aligned16(p.q.p) && aligned16(p.k.p) && aligned16(p.v.p) && aligned16(state) &&
            aligned16(global_grad->t) && aligned16(dout->t);

    // dS scratch: stream-ordered, released right after the kernels that use it.
    const size_t ds_floats = gptc::bwd_ds_floats(d.B, d.H, d.T);
    p.ds = static_cast<float *>(alloc_cuda(ds_floats * sizeof(float)));
    gptc::launch_attn_bwd(p, gptc_stream_checked(), g_have_events ? g_events + 2 : nullptr);
    free_cuda(p.ds);
}
