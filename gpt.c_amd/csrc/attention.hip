// C-ABI entry points of the causal attention path: shape and layout checks
// on the host, then the fused HIP kernels on the library stream.
// Replaces kernels/src/cuda/Attention.cu:170-324 behind the signatures of
// kernels/src/cuda/Attention.h:9-22 (called by
// kernels/src/core/Attention.c:40-41,75-76).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <initializer_list>
#include <mutex>
#include <vector>
#include <tuple>
#include <set>
#include "attn_kernels.hpp"
#include "ops_common.hpp"
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

// The buffer-resource tile loads (FULL kernels) need D == kDPad and the rows
// of one head, row stride st floats, to span fewer than 2^31 bytes.
bool full_tiles(const Dims &d, std::initializer_list<uint32_t> strides) {
    if (d.D != gptc::kDPad) return false;
    for (uint32_t st : strides)
        if ((static_cast<int64_t>(d.T - 1) * st + gptc::kDPad) * 4 >= (1LL << 31)) return false;
    return true;
}

// Head sizes 1 .. 128 run the MFMA kernels, 129 .. kGenericMaxD the generic
// ones (plain FMAs, the LSE-only state); larger ones are refused.
bool generic_head(const Dims &d) { return d.D > 2 * gptc::kDPad; }

void check_head_size(const Dims &d) {
    CHECK_ERROR(d.H <= 0 || d.C % d.H != 0, "Expected C = %d to be divisible by n_heads = %d.", d.C, d.H);
    CHECK_ERROR(d.D < 1 || d.D > gptc::kGenericMaxD,
                "Head size %d is not supported by the GPU attention kernels (1 <= n_embd / n_heads <= %d).", d.D,
                gptc::kGenericMaxD);
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

int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }

// Float offsets of the state that cache[3] carries from forward to backward,
// each part 256-byte aligned:
//   [y copy (B*T*C) | log-sum-exp (B*H*T)]   reference cache layout only
//   delta (B*H*T)                            written by the backward
//   m (B*H*nqt*T)                            per-tile row maxima of P'
//   db partials (B*nqt*C + B*2nkb*2C)       column sums of the dq | dk, dv
//                                            rows (qkv bias folded in only)
//   P' / dS blocks (bwd_ds_floats)           P' from forward, dS in backward
// The LSE-only state (lse_only) has no m and no P' / dS blocks: its
// backward recomputes P from the log-sum-exp in both gradient kernels.
struct StateLayout {
    int64_t y, lse, delta, m, dbq, dbkv, p, total;
};

StateLayout state_layout(const Dims &d, bool reference_layout, bool lse_only) {
    const int64_t btc = static_cast<int64_t>(d.B) * d.T * d.C;
    const int64_t bht = static_cast<int64_t>(d.B) * d.H * d.T;
    const int64_t nqt = (d.T + 63) / 64;
    StateLayout s{};
    int64_t off = 0;
    if (reference_layout) {
        s.y = off;
        off += align64(btc);
        s.lse = off;
        off += align64(bht);
    }
    s.delta = off;
    off += align64(bht);
    s.m = off;
    if (!lse_only) off += align64(bht * nqt);
    const int64_t nkb = (d.T + 127) / 128;
    s.dbq = off;
    off += align64(static_cast<int64_t>(d.B) * nqt * d.C);
    s.dbkv = off;  // up to 2 nkb rows per batch row: split key blocks add one each
    off += align64(static_cast<int64_t>(d.B) * 2 * nkb * 2 * d.C);
    s.p = off;
    if (!lse_only) off += static_cast<int64_t>(gptc::bwd_ds_floats(d.B, d.H, d.T));
    s.total = off;
    return s;
}

// Largest P' state (floats) a forward keeps; above it, kernels that can
// (D == 64 with 16-byte rows) keep the LSE-only state instead.  The default
// is the int length of a tensor_t, past which the state cannot exist.
std::atomic<long long> g_state_limit{INT32_MAX};

// Largest dS scratch (floats) the backward of the LSE-only state allocates
// (in whole heads: chunks of as many heads as fit run one after the other).
// The default, 2^30 floats (4 GiB), keeps the block offsets within 32 bits.
constexpr long long kScratchLimitMax = 1LL << 30;
std::atomic<long long> g_scratch_limit{kScratchLimitMax};

// The state layout a forward uses: LSE-only when the D == 64 kernels run
// (`full`) and the P' state would exceed the limit, and always for the
// generic head sizes.
StateLayout forward_state(const Dims &d, bool reference_layout, bool full, bool *lse_only) {
    *lse_only = generic_head(d) || (full && state_layout(d, reference_layout, false).total > g_state_limit.load());
    const StateLayout s = state_layout(d, reference_layout, *lse_only);
    CHECK_ERROR(s.total > INT32_MAX,
                "Attention state of %lld floats for B=%d, T=%d, H=%d exceeds the int length of a tensor_t "
                "(head sizes other than 64 keep the probability blocks).",
                (long long)s.total, d.B, d.T, d.H);
    return s;
}

// Makes `t` a 1-D device tensor of exactly n floats (the backward state),
// replacing its storage unless it already is one.
void ensure_state_tensor(tensor_t *t, int64_t n) {
    if (t->ndims == 1 && t->length == n) return;
    free_cuda(t->t);
    t->t = static_cast<float *>(alloc_cuda(static_cast<size_t>(n) * sizeof(float)));
    t->ndims = 1;
    t->length = static_cast<int>(n);
    for (int i = 0; i < 8; i++) t->shape[i] = 0;
    t->shape[0] = static_cast<int>(n);
}

// The mask.  gpt.c keeps score (i, j) where mask[i][j] == 1.0f and sets it
// to -inf elsewhere (kernels/src/cpu/Attention.c:135-142, row stride the
// mask's last dim).  The kernels apply the causal rule j <= i from indices
// and never read the mask, so a mask that is not that rule on the T x T
// block a call reads is refused.  The check reads the block once per mask
// buffer and remembers it while the buffer's allocation serial is unchanged
// (a new allocation at the same address, or a write into it through the
// library's tensor data ops, checks again); a buffer that is not an
// alloc_cuda block is checked at every call.  Writes by other kernels into
// a checked mask are not seen.
struct MaskKey {
    const float *p;
    uint64_t serial;
    int T, stride;
    bool operator<(const MaskKey &o) const {
        return std::tie(p, serial, T, stride) < std::tie(o.p, o.serial, o.T, o.stride);
    }
};
std::mutex g_mask_mu;
std::set<MaskKey> g_causal_masks;

void check_causal_mask(const tensor_t *mask, int T) {
    const int stride = mask->shape[mask->ndims - 1];
    const bool on_device = mask->device == CUDA;
    const uint64_t serial = on_device ? gptc_block_serial(mask->t) : 0;
    const MaskKey key{mask->t, serial, T, stride};
    if (serial != 0) {
        std::lock_guard<std::mutex> lk(g_mask_mu);
        if (g_causal_masks.count(key)) return;
    }
    // Rows in chunks, so that the host copy stays small at any T.
    const int chunk = std::max(1, std::min(T, (1 << 22) / T));
    std::vector<float> m(static_cast<size_t>(chunk) * T);
    for (int i0 = 0; i0 < T; i0 += chunk) {
        const int rows = std::min(chunk, T - i0);
        const float *src = mask->t + static_cast<size_t>(i0) * stride;
        if (on_device) {
            hipStream_t s = gptc_stream_checked();
            hipCheck(hipMemcpy2DAsync(m.data(), static_cast<size_t>(T) * sizeof(float), src,
                                      static_cast<size_t>(stride) * sizeof(float),
                                      static_cast<size_t>(T) * sizeof(float), rows, hipMemcpyDeviceToHost, s));
            hipCheck(hipStreamSynchronize(s));
        } else {
            for (int r = 0; r < rows; r++)
                std::copy(src + static_cast<size_t>(r) * stride, src + static_cast<size_t>(r) * stride + T,
                          m.begin() + static_cast<size_t>(r) * T);
        }
        for (int r = 0; r < rows; r++)
            for (int j = 0; j < T; j++) {
                const int i = i0 + r;
                const float v = m[static_cast<size_t>(r) * T + j];
                CHECK_ERROR((v == 1.0f) != (j <= i),
                            "The GPU attention kernels apply the causal mask (mask[i][j] == 1 exactly for j <= i); "
                            "this mask differs at (%d, %d) (value %g).",
                            i, j, (double)v);
            }
    }
    if (serial != 0) {
        std::lock_guard<std::mutex> lk(g_mask_mu);
        g_causal_masks.insert(key);
    }
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

namespace {

// The forward of both entry points.  bias: the qkv Linear's bias (3C),
// nullptr when the input already includes it.  With a bias, the compact
// layout is required; the D = 64 kernels add it as they load q, k, v, other
// head sizes get it added to the input in place first.
void forward_impl(const tensor_t *input, const tensor_t *bias, const tensor_t *mask, const int n_heads,
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
    CHECK_ERROR(mask->t == NULL && d.T > 0, "Expected the mask to hold data.");
    CHECK_ERROR(output->length != d.B * d.T * d.C, "Expected output of %d elements, but got %d.", d.B * d.T * d.C,
                output->length);
    if (d.B == 0 || d.T == 0 || d.C == 0) return;
    check_causal_mask(mask, d.T);

    FwdParams p{};
    qkv_views(input->t, d, p.q, p.k, p.v);
    p.o = btc_view<HeadViewW>(output->t, d);
    const int64_t bht = static_cast<int64_t>(d.B) * d.H * d.T;

    const bool compact = cache[0] == input || cache[0]->t == input->t;
    // Whether the D == 64 kernels run (they decide which state is kept): the
    // views' alignment, y's second copy (a buffer of its own in the compact
    // layout; in the reference layout it lies in the state, 256-byte aligned)
    // and the permuted caches of the reference layout.
    p.B = d.B;
    p.H = d.H;
    p.T = d.T;
    p.D = d.D;
    {
        const float *o2 = compact ? (cache[1]->t == output->t ? nullptr : cache[1]->t) : nullptr;
        p.vec = (d.D % 4 == 0) && aligned16(input->t) && aligned16(output->t) && aligned16(o2) &&
                (compact || (aligned16(cache[0]->t) && aligned16(cache[1]->t) && aligned16(cache[2]->t)));
        p.full = p.vec && full_tiles(d, {p.q.st, p.k.st, p.v.st});
    }
    bool lse_only = false;
    const StateLayout st = forward_state(d, !compact, p.full, &lse_only);
    if (compact) {
        // Compact layout: the layer keeps the input itself, y in cache[1]
        // (the output's own storage, or a buffer that receives a copy), the
        // log-sum-exp in cache[2] and the backward state in cache[3]
        // (re-pointed here unless it already has the state's size).
        CHECK_ERROR(cache[1]->length != output->length, "Expected cache[1] of %d elements (the output or a copy).",
                    output->length);
        CHECK_ERROR(cache[2]->length < bht, "Expected cache[2] of at least B*H*T = %lld elements.", (long long)bht);
        ensure_state_tensor(cache[3], st.total);
        p.o2 = cache[1]->t == output->t ? nullptr : cache[1]->t;
        p.lse = cache[2]->t;
        p.qp = p.kp = p.vp = nullptr;
    } else {
        // Reference layout (gpt.c attention.c:105-120): permuted q, k, v go to
        // cache[0..2]; cache[3] is re-pointed from the (B, H, T, T) P to the
        // compact state, which includes y and the log-sum-exp.
        for (int i = 0; i < 3; i++)
            CHECK_ERROR(!is_bhtd(cache[i], d), "Expected cache[%d] of shape (B, H, T, D) = (%d, %d, %d, %d).", i, d.B,
                        d.H, d.T, d.D);
        ensure_state_tensor(cache[3], st.total);
        p.o2 = cache[3]->t + st.y;
        p.lse = cache[3]->t + st.lse;
        p.qp = cache[0]->t;
        p.kp = cache[1]->t;
        p.vp = cache[2]->t;
    }
    p.pm = lse_only ? nullptr : cache[3]->t + st.m;
    p.pp = lse_only ? nullptr : cache[3]->t + st.p;

    p.scale_log2 = gptc::kLog2e / std::sqrt(static_cast<float>(d.D));
    p.nqb = (d.T + 127) / 128;
    p.nqt = (d.T + 63) / 64;
    p.bh_pad = bh_padded(d.B * d.H);
    if (bias != nullptr) {
        CHECK_ERROR(!compact, "The qkv bias can be folded in with the compact cache layout only.");
        CHECK_ERROR(bias->device != CUDA || bias->length != 3 * d.C, "Expected a GPU bias of 3C = %d elements.",
                    3 * d.C);
        const bool folded = p.full && aligned16(bias->t);
        if (folded) {
            p.qb = bias->t;
            p.kb = bias->t + d.C;
            p.vb = bias->t + 2 * d.C;
        } else {
            // The input is the layer's own (cache[0]): add the bias in place.
            gptc::launch_bias_add(input->t, bias->t, static_cast<int64_t>(d.B) * d.T, 3 * d.C, gptc_stream_checked());
        }
        // The backward must know whether the input still lacks the bias: the
        // state is 1-D, so its unused second shape entry records it.
        cache[3]->shape[1] = folded ? 1 : 0;
    } else if (compact) {
        cache[3]->shape[1] = 0;
    }
    gptc::launch_attn_fwd(p, gptc_stream_checked(), g_have_events ? g_events : nullptr);
}

}  // namespace

extern "C" void attention_forward_cuda_kernel(const tensor_t *input, const tensor_t *mask, const int n_heads,
                                              tensor_t **cache, tensor_t *output) {
    forward_impl(input, nullptr, mask, n_heads, cache, output);
}

extern "C" void gptc_attention_forward_qkv_bias(const tensor_t *input, const tensor_t *bias, const tensor_t *mask,
                                                const int n_heads, tensor_t **cache, tensor_t *output) {
    REQUIRE_ARG(bias);
    forward_impl(input, bias, mask, n_heads, cache, output);
}

namespace {

// The backward of both entry points: bias and db given (db += the column
// sums of dout) when the forward took the bias.
void backward_impl(const tensor_t *global_grad, tensor_t **cache, const tensor_t *bias, const int n_heads,
                   tensor_t *dout, tensor_t *db) {
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
    const float *y_saved = nullptr;
    const bool compact = c0->ndims == 3 && c0->shape[0] == d.B && c0->shape[1] == d.T && c0->shape[2] == 3 * d.C;
    // Which state the forward kept: told apart by its length (the LSE-only
    // state has no probability blocks, so it is strictly shorter).
    const StateLayout st_lse = state_layout(d, !compact, true);
    const bool lse_only = cache[3]->ndims == 1 && cache[3]->length == st_lse.total;
    const StateLayout st = lse_only ? st_lse : state_layout(d, !compact, false);
    CHECK_ERROR(cache[3]->ndims != 1 || cache[3]->length != st.total,
                "cache[3] does not hold the state written by attention_forward_cuda_kernel for this shape.");
    if (compact) {
        CHECK_ERROR(cache[1]->length != btc, "Expected cache[1] of B*T*C = %lld elements.", (long long)btc);
        CHECK_ERROR(cache[2]->length < bht, "Expected cache[2] of at least B*H*T = %lld elements.", (long long)bht);
        qkv_views(c0->t, d, p.q, p.k, p.v);
        y_saved = cache[1]->t;
        p.lse = cache[2]->t;
    } else {
        for (int i = 0; i < 3; i++)
            CHECK_ERROR(!is_bhtd(cache[i], d), "Expected cache[%d] of shape (B, H, T, D) = (%d, %d, %d, %d).", i, d.B,
                        d.H, d.T, d.D);
        p.q = bhtd_view(cache[0]->t, d);
        p.k = bhtd_view(cache[1]->t, d);
        p.v = bhtd_view(cache[2]->t, d);
        y_saved = cache[3]->t + st.y;
        p.lse = cache[3]->t + st.lse;
    }
    p.o = btc_view<HeadView>(y_saved, d);
    p.delta = cache[3]->t + st.delta;
    // The backward consumes the state: dS overwrites P' (gpt.c's CPU backward
    // likewise reuses its caches as scratch, kernels/src/cpu/Attention.c:198-201).
    // The LSE-only state has neither: the dk/dv kernel recomputes P, and dS
    // goes to a scratch of the packed blocks (below) for as many heads at a
    // time as the scratch limit allows; without room for one head, the dq
    // kernel recomputes P and dP as well.
    p.pm = lse_only ? nullptr : cache[3]->t + st.m;
    p.ds = lse_only ? nullptr : cache[3]->t + st.p;
    p.lse_only = lse_only;
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
    p.nqb = (d.T + 127) / 128;
    p.nkb = (d.T + 127) / 128;
    p.nqt = (d.T + 63) / 64;
    p.bh_pad = bh_padded(d.B * d.H);
    p.vec = (d.D % 4 == 0) && aligned16(p.q.p) && aligned16(p.k.p) && aligned16(p.v.p) && aligned16(y_saved) &&
            aligned16(global_grad->t) && aligned16(dout->t);
    p.full = p.vec && full_tiles(d, {p.q.st, p.k.st, p.dout.st});
    CHECK_ERROR(lse_only && !p.full && !generic_head(d),
                "The forward kept the log-sum-exp-only state, which only the D = 64 kernels read, but these "
                "gradient buffers need the other kernels (unaligned rows).");
    hipStream_t s = gptc_stream_checked();
    float *ds_scratch = nullptr;
    if (lse_only && p.full) {
        const int64_t bh = static_cast<int64_t>(d.B) * d.H;
        const int64_t per_head = static_cast<int64_t>(gptc::bwd_ds_floats(1, 1, d.T));
        const int64_t heads = std::min<int64_t>(bh, g_scratch_limit.load() / per_head);
        // Short heads (one recomputing workgroup per key block over all heads) take the scratch only whole.
        if (heads >= 1 && (p.nqt > gptc::kShortHeadTiles || heads == bh)) {
            ds_scratch = static_cast<float *>(alloc_cuda(static_cast<size_t>(heads * per_head) * sizeof(float)));
            p.ds = ds_scratch;
            p.ds_heads = static_cast<int>(heads);
        }
    }
    gptc::bwd_split_plan(p, s);
    bool folded = false;
    if (bias != nullptr) {
        CHECK_ERROR(!compact, "The qkv bias can be folded in with the compact cache layout only.");
        CHECK_ERROR(db == NULL || db->device != CUDA || db->length != 3 * d.C || bias->length != 3 * d.C,
                    "Expected a GPU bias and db of 3C = %d elements.", 3 * d.C);
        // Whether the forward left the bias out of the input (recorded in the
        // state's unused second shape entry).  If so and these kernels cannot
        // fold it in (a differently aligned dy or dout), add it to the input.
        const bool fwd_folded = cache[3]->shape[1] == 1;
        folded = fwd_folded && p.full;
        if (fwd_folded && !folded)
            gptc::launch_bias_add(const_cast<float *>(c0->t), bias->t, static_cast<int64_t>(d.B) * d.T, 3 * d.C, s);
        if (folded) {
            p.qb = bias->t;
            p.kb = bias->t + d.C;
            p.vb = bias->t + 2 * d.C;
            p.db = db->t;
            p.dbq_part = cache[3]->t + st.dbq;
            p.dbkv_part = cache[3]->t + st.dbkv;
            p.C = d.C;
        }
    }
    gptc::launch_attn_bwd(p, s, g_have_events ? g_events + 2 : nullptr);
    // Stream-ordered: the block returns to the allocator's cache behind the
    // kernels that use it.
    if (ds_scratch != nullptr) free_cuda(ds_scratch);
    if (bias != nullptr) {
        const int nqt = (d.T + 63) / 64, nkb = (d.T + 127) / 128;
        if (folded) {
            // db += the per-block column sums, in a fixed order.
            gptc::launch_add_column_partials(p.dbq_part, db->t, d.B * nqt, d.C, s);
            gptc::launch_add_column_partials(p.dbkv_part, db->t + d.C, d.B * (nkb + p.nsplit), 2 * d.C, s);
        } else {
            gptc::launch_column_sum_add(dout->t, db->t, d.B * d.T, 3 * d.C, s);
        }
    }
}

}  // namespace

extern "C" void attention_backward_cuda_kernel(const tensor_t *global_grad, tensor_t **cache, const int n_heads,
                                               tensor_t *dout) {
    backward_impl(global_grad, cache, nullptr, n_heads, dout, nullptr);
}

extern "C" void gptc_attention_backward_qkv_bias(const tensor_t *global_grad, tensor_t **cache, const tensor_t *bias,
                                                 const int n_heads, tensor_t *dout, tensor_t *db) {
    REQUIRE_ARG(bias);
    REQUIRE_ARG(db);
    backward_impl(global_grad, cache, bias, n_heads, dout, db);
}

extern "C" long long gptc_attention_state_floats(int B, int T, int C, int n_heads) {
    CHECK_ERROR(B < 0 || T < 0 || C < 0 || n_heads <= 0 || C % n_heads != 0,
                "Expected B, T, C >= 0 and C divisible by n_heads > 0, but got B=%d, T=%d, C=%d, n_heads=%d.", B, T,
                C, n_heads);
    const Dims d{B, T, C, n_heads, C / n_heads};
    // The state the forward keeps in the compact layout, taking head size 64
    // to run the D == 64 kernels (a forward that finds otherwise re-points
    // cache[3] to its own size).
    bool lse_only = false;
    return forward_state(d, false, d.D == gptc::kDPad, &lse_only).total;
}

extern "C" long long gptc_attention_set_state_limit(long long floats) {
    return g_state_limit.exchange(floats < 0 ? static_cast<long long>(INT32_MAX) : floats);
}

extern "C" long long gptc_attention_set_scratch_limit(long long floats) {
    return g_scratch_limit.exchange(floats < 0 || floats > kScratchLimitMax ? kScratchLimitMax : floats);
}

namespace {

// Shape checks and launch parameters of the decode step; the position comes
// from the host (pos, checked here) or from device memory (pos_dev, checked
// by the kernel, for graph replays).
gptc::DecParams decode_params(const tensor_t *qkv, tensor_t *k_cache, tensor_t *v_cache, const int pos,
                              const int *pos_dev, const int n_heads, tensor_t *output) {
    CHECK_ERROR(qkv == NULL || k_cache == NULL || v_cache == NULL || output == NULL,
                "Expected qkv, k_cache, v_cache and output to be non-NULL.");
    CHECK_ERROR(qkv->ndims != 3 || qkv->shape[1] != 1 || qkv->shape[2] % 3 != 0,
                "Expected qkv of shape (B, 1, 3C) (the new token's row), but got %d dims.", qkv->ndims);
    Dims d;
    d.B = qkv->shape[0];
    d.T = 1;
    d.C = qkv->shape[2] / 3;
    d.H = n_heads;
    CHECK_ERROR(d.H <= 0, "Expected n_heads > 0, but got %d.", d.H);
    d.D = d.C / d.H;
    check_head_size(d);
    for (const tensor_t *c : {static_cast<const tensor_t *>(k_cache), static_cast<const tensor_t *>(v_cache)})
        CHECK_ERROR(c->ndims != 4 || c->shape[0] != d.B || c->shape[1] != d.H || c->shape[3] != d.D,
                    "Expected k_cache and v_cache of shape (B, H, L, D) = (%d, %d, L, %d).", d.B, d.H, d.D);
    const int L = k_cache->shape[2];
    CHECK_ERROR(v_cache->shape[2] != L, "Expected k_cache and v_cache with the same length L, but got %d and %d.", L,
                v_cache->shape[2]);
    if (pos_dev == nullptr) {
        CHECK_ERROR(pos < 0 || pos >= L, "Expected 0 <= pos < L = %d, but got pos = %d.", L, pos);
        CHECK_ERROR(pos + 1 > gptc::kDecMaxKeys, "Decode attends at most %d keys, but pos = %d.", gptc::kDecMaxKeys,
                    pos);
    } else {
        CHECK_ERROR(L > gptc::kDecMaxKeys, "Decode with a device-side position takes caches of at most %d rows.",
                    gptc::kDecMaxKeys);
    }
    CHECK_ERROR(output->length != d.B * d.C, "Expected output of B*C = %d elements, but got %d.", d.B * d.C,
                output->length);

    gptc::DecParams p{};
    p.qkv = qkv->t;
    p.k_cache = k_cache->t;
    p.v_cache = v_cache->t;
    p.out = output->t;
    p.B = d.B;
    p.H = d.H;
    p.C = d.C;
    p.D = d.D;
    p.L = L;
    p.pos = pos;
    p.pos_dev = pos_dev;
    p.scale_log2 = gptc::kLog2e / std::sqrt(static_cast<float>(d.D));
    p.full = d.D == gptc::kDPad && aligned16(k_cache->t) && aligned16(v_cache->t);
    // Split-key kernels for D == 64: chunks of the keys 0 .. pos, or of the
    // cache length with a device-side position.
    if (p.full) p.splits = ((pos_dev == nullptr ? pos + 1 : L) + gptc::kDecChunk - 1) / gptc::kDecChunk;
    return p;
}

void decode_step(const tensor_t *qkv, tensor_t *k_cache, tensor_t *v_cache, const int pos, const int *pos_dev,
                 const int n_heads, tensor_t *output, float *part) {
    gptc::DecParams p = decode_params(qkv, k_cache, v_cache, pos, pos_dev, n_heads, output);
    if (p.B == 0 || p.C == 0) return;
    // The eager form takes the partials buffer from the stream-ordered
    // allocator; the merge kernel reads it before anything queued later can
    // reuse it.
    bool own_part = false;
    if (p.full && !gptc::dec_head_fits(p)) {
        if (part == nullptr) {
            part = static_cast<float *>(
                alloc_cuda(static_cast<size_t>(p.B) * p.H * p.splits * gptc::kDecPartStride * sizeof(float)));
            own_part = true;
        }
        p.part = part;
    }
    gptc::launch_attn_decode(p, gptc_stream_checked());
    if (own_part) free_cuda(part);
}

}  // namespace

extern "C" void attention_decode_cuda_kernel(const tensor_t *qkv, tensor_t *k_cache, tensor_t *v_cache, const int pos,
                                             const int n_heads, tensor_t *output) {
    decode_step(qkv, k_cache, v_cache, pos, nullptr, n_heads, output, nullptr);
}

// ---- Allocation-free decode step ----
// The split-key decode's partials (B*H*splits*kDecPartStride floats) live in
// a file-scope device array instead of a stream-ordered allocation, for
// callers that must not allocate (graph capture, serving loops).  Each GPU
// holds its own copy of the array until the process ends; host code reaches
// it only through the address hipGetSymbolAddress returns for the current
// device (the array's name is a host-side stand-in, not a device address).
// Steps of at most kDecHeadKeys keys run the one-launch kernel, which needs
// no partials, so only longer steps use the array.  Every call on a GPU
// reuses that GPU's array: calls that overlap on one GPU (other streams,
// other threads) race.  Nothing needs clearing between
// calls: the merge kernel reads only the partials the split kernel of the
// same call wrote.
namespace {

constexpr size_t kDecodeScratchFloats = size_t(1) << 20;  // 4 MiB per GPU
__device__ __align__(256) float scratch[kDecodeScratchFloats];

constexpr int kMaxDevices = 64;
float *g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch`, looked up once per device.
float *device_scratch() {
    int dev = 0;
    hipCheck(hipGetDevice(&dev));
    CHECK_ERROR(dev < 0 || dev >= kMaxDevices, "Device %d is beyond the %d devices the decode scratch serves.", dev,
                kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        CHECK_ERROR(rc != hipSuccess || p == nullptr, "hipGetSymbolAddress(decode scratch) failed on device %d: %s.",
                    dev, hipGetErrorString(rc));
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" void attention_decode_noalloc_cuda_kernel(const tensor_t *qkv, tensor_t *k_cache, tensor_t *v_cache,
                                                     const int pos, const int n_heads, tensor_t *output) {
    gptc::DecParams p = decode_params(qkv, k_cache, v_cache, pos, nullptr, n_heads, output);
    if (p.B == 0 || p.C == 0) return;
    if (p.full && !gptc::dec_head_fits(p)) {
        const size_t need = static_cast<size_t>(p.B) * p.H * p.splits * gptc::kDecPartStride;
        CHECK_ERROR(need > kDecodeScratchFloats,
                    "attention_decode_noalloc_cuda_kernel: B=%d, H=%d, pos=%d needs %zu floats of partials, more than "
                    "its fixed %zu-float scratch; use attention_decode_cuda_kernel.",
                    p.B, p.H, pos, need, kDecodeScratchFloats);
        p.part = device_scratch();
    }
    gptc::launch_attn_decode(p, gptc_stream_checked());
}

extern "C" long long gptc_decode_noalloc_scratch_floats(void) {
    return static_cast<long long>(kDecodeScratchFloats);
}

void gptc::attention_decode_cached(const tensor_t *qkv, tensor_t *k_cache, tensor_t *v_cache, const int pos,
                                   const int *pos_dev, const int n_heads, tensor_t *output, float *part) {
    decode_step(qkv, k_cache, v_cache, pos, pos_dev, n_heads, output, part);
}

size_t gptc::attention_decode_part_floats(const int B, const int H, const int L) {
    return gptc::dec_part_floats(B, H, L);
}
