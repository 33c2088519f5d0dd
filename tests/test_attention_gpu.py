"""GPU parity of the fused causal attention against the CPU oracle.

Every case runs the HIP kernels through the library's C-ABI (gpt.c's
Attention() layer or the attention_*_cuda_kernel entry points directly)
and compares with the oracle (the C restatement of gpt.c's OpenBLAS CPU
path) on the same seeded inputs.  Tolerance, from the BASELINE north star:
max abs err <= 1e-4 on y, dq, dk, dv and the saved log-sum-exp.
"""
import contextlib
import ctypes

import numpy as np
import pytest

import gptc

pytestmark = pytest.mark.gpu

TOL = 1e-4


def qkv_inputs(rt, B, T, C, seed_x=1337, seed_dy=1338):
    x = rt.normal((B, T, 3 * C), seed_x)
    dy = rt.normal((B, T, C), seed_dy)
    return x, dy


def run_layer(rt, x, dy, H, block=None):
    """Forward + backward through Attention() exactly as SelfAttention calls it."""
    B, T, C3 = x.shape
    C = C3 // 3
    layer = gptc.AttentionLayer(rt, C, H, block or T)
    layer.to(gptc.CUDA)
    yt = layer.forward(rt.from_numpy(x))
    y = rt.to_numpy(yt)
    lse = rt.to_numpy(layer.cache(2)).reshape(B, H, T)
    dqkv = None
    if dy is not None:
        dt = layer.backward(rt.from_numpy(dy))
        dqkv = rt.to_numpy(dt)
        rt.free(dt)
        assert all(not layer.cache(i) for i in range(4))
    rt.free(yt)
    layer.free()
    rt.sync()
    return y, lse, dqkv


def lse_fp64(q, k):
    """Natural-log row log-sum-exp (B, H, T) of the causal scores, float64."""
    B, H, T, D = q.shape
    keep = np.tril(np.ones((T, T), bool))
    out = np.empty((B, H, T))
    for b in range(B):
        s = np.matmul(q[b].astype(np.float64), k[b].astype(np.float64).transpose(0, 2, 1)) / np.sqrt(D)
        s = np.where(keep, s, -np.inf)
        m = s.max(-1)
        out[b] = m + np.log(np.exp(s - m[..., None]).sum(-1))
    return out


def check(name, got, ref, tol=TOL):
    err = float(np.abs(got.astype(np.float64) - ref).max()) if got.size else 0.0
    print(f"  {name}: max abs err {err:.3e}")
    assert np.isfinite(got).all(), name
    assert err <= tol, f"{name}: max abs err {err:.3e} > {tol}"
    return err


def compare_with_oracle(rt, oracle, B, T, C, H, backward=True, block=None):
    x, dy = qkv_inputs(rt, B, T, C)
    y, lse, dqkv = run_layer(rt, x, dy if backward else None, H, block)
    y_ref, q, k, v, att = oracle.forward(x, H)
    print(f"case B={B} T={T} C={C} H={H} D={C // H}", flush=True)
    check("y", y, y_ref)
    check("lse (every head)", lse, lse_fp64(q, k))
    if backward:
        d_ref = oracle.backward(dy, H, q, k, v, att)
        check("dq", dqkv[..., :C], d_ref[..., :C])
        check("dk", dqkv[..., C:2 * C], d_ref[..., C:2 * C])
        check("dv", dqkv[..., 2 * C:], d_ref[..., 2 * C:])


SMALL = [  # (B, T, C, H)
    (1, 1, 64, 1),
    (2, 17, 192, 3),
    (1, 64, 128, 2),
    (2, 100, 256, 4),
    (1, 129, 128, 2),      # crosses a 128-query block
    (1, 200, 64, 2),       # D = 32
    (2, 5, 6, 2),          # D = 3 (gpt.c's tests/test_self_attention.c shape class)
    (2, 16, 16, 2),        # D = 8
    (1, 70, 100, 25),      # H = 25, D = 4
    (1, 257, 48, 1),       # D = 48
    (2, 300, 48, 3),       # D = 16
    (1, 511, 768, 12),     # C4's longest window shape at B = 1
    (2, 77, 384, 4),       # D = 96 (kernels built for 128 padded dims)
    (1, 200, 768, 6),      # D = 128
    (2, 33, 260, 4),       # D = 65 (128 padded dims, ragged)
    (3, 65, 128, 2),       # two-tile head: one query in the second block
    (1, 127, 192, 3),      # two-tile head, ragged second block
]


@pytest.mark.parametrize("B,T,C,H", SMALL)
def test_small_shapes_fwd_bwd(rt, oracle, B, T, C, H):
    compare_with_oracle(rt, oracle, B, T, C, H)


def test_head_size_128_full_length(rt, oracle):
    """D = 128 over 16 key tiles (T = 1024): the 128-dim forward, dk/dv and dq kernels."""
    compare_with_oracle(rt, oracle, 1, 1024, 1024, 8)


@pytest.mark.parametrize("B,T,C,H", [
    (1, 40, 258, 2),      # D = 129: the smallest generic head size
    (2, 77, 384, 2),      # D = 192
    (1, 300, 512, 2),     # D = 256, several key chunks
    (2, 33, 1024, 2),     # D = 512 (32-key chunks)
    (1, 21, 1024, 1),     # D = 1024 (8-key chunks), the largest served
])
def test_generic_head_sizes_fwd_bwd(rt, oracle, B, T, C, H):
    """Head sizes past 128 (gpt.c accepts any D with C % H == 0,
    src/attention.c:23): the generic plain-FMA kernels with the LSE-only
    state, against the oracle at the same tolerance."""
    compare_with_oracle(rt, oracle, B, T, C, H)


def test_generic_head_size_reference_layout(rt, oracle):
    """The generic forward with gpt.c's own cache layout (permuted q, k, v
    in cache[0..2]): the caches hold exactly the permuted inputs."""
    B, T, C, H = 2, 50, 400, 2  # D = 200
    x, dy = qkv_inputs(rt, B, T, C, 61, 62)
    lib = rt.lib
    xt = rt.from_numpy(x)
    mask = rt.from_numpy(np.tril(np.ones((T, T), np.float32)))
    D = C // H
    caches = (gptc.TensorP * 4)(rt.empty((B, H, T, D)), rt.empty((B, H, T, D)), rt.empty((B, H, T, D)),
                                rt.empty((B, H, T, T)))
    yt, dout = rt.empty((B, T, C)), rt.empty((B, T, 3 * C))
    lib.attention_forward_cuda_kernel(xt, mask, H, caches, yt)
    y_ref, q, k, v, att = oracle.forward(x, H)
    check("y", rt.to_numpy(yt), y_ref)
    for i, ref in enumerate((q, k, v)):
        assert np.array_equal(rt.to_numpy(caches[i]), ref), f"cache[{i}]"
    dyt = rt.from_numpy(dy)
    lib.attention_backward_cuda_kernel(dyt, caches, H, dout)
    check("dqkv", rt.to_numpy(dout), oracle.backward(dy, H, q, k, v, att))
    for t in (xt, dyt, mask, yt, dout, *caches):
        rt.free(t)
    rt.sync()


def test_head_size_past_1024_is_refused():
    """Head sizes past the generic kernels' 1024 end the process with gpt.c's
    error report before any launch (a host-side check)."""
    import os
    import subprocess
    import sys
    import textwrap
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gpt.c_amd")
    code = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {pkg!r})
        import numpy as np
        import gptc
        lib = gptc.load()
        rt = gptc.Runtime(lib)
        rt.init()
        layer = gptc.AttentionLayer(rt, 2060, 2, 4)
        layer.to(gptc.CUDA)
        layer.forward(rt.from_numpy(np.zeros((1, 4, 3 * 2060), np.float32)))
        print('survived')
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "survived" not in r.stdout, r.stderr
    assert "Head size 1030 is not supported" in r.stderr and "[ERROR]" in r.stderr


def test_mask_block_larger_than_T(rt, oracle):
    compare_with_oracle(rt, oracle, 2, 77, 128, 2, block=1024)


def test_c1_forward_b8_t128_h12(rt, oracle):
    compare_with_oracle(rt, oracle, 8, 128, 768, 12, backward=False)


def test_c1_fwd_bwd_b8_t128_h12(rt, oracle):
    """C1's shape through the backward too: short heads (T <= 128), where the
    forward stores no P' and the dk/dv kernel recomputes P from Q, K, LSE."""
    compare_with_oracle(rt, oracle, 8, 128, 768, 12)


def test_c2_fwd_bwd_b8_t1024_h12(rt, oracle):
    compare_with_oracle(rt, oracle, 8, 1024, 768, 12)


def test_c5_fwd_bwd_b4_t1024_h25(rt, oracle):
    compare_with_oracle(rt, oracle, 4, 1024, 1600, 25)


def test_odd_block_count_wide_grid(rt, oracle):
    """T = 960: 15 query blocks of 64, so in the paired forward and dq grids
    (blocks j and 14-j per workgroup) the middle block of each head runs alone."""
    compare_with_oracle(rt, oracle, 8, 960, 768, 12)


def test_reference_cache_layout(rt, oracle):
    """gpt.c's unchanged attention.c allocates q, k, v (B,H,T,D) and att (B,H,T,T)
    caches (attention.c:105-120) and passes a zeroed dout: the entry points
    must serve that layout too, leaving the same q, k, v the CPU kernel caches."""
    reference_layout_vs_oracle(rt, oracle)


def test_reference_cache_layout_lse_only_state(rt, oracle, lse_only_state):
    """The same layout when the forward keeps only the log-sum-exp (D = 64
    shapes; the D = 3 shape keeps its probability blocks)."""
    reference_layout_vs_oracle(rt, oracle)


def reference_layout_vs_oracle(rt, oracle):
    lib = rt.lib
    for B, T, C, H in [(2, 150, 256, 4), (2, 100, 256, 4), (2, 5, 6, 2)]:
        D = C // H
        x, dy = qkv_inputs(rt, B, T, C, 7, 8)
        xt = rt.from_numpy(x)
        mask = rt.from_numpy(np.tril(np.ones((T, T), np.float32)))
        caches = (gptc.TensorP * 4)(*[rt.empty((B, H, T, D)) for _ in range(3)], rt.empty((B, H, T, T)))
        yt = rt.empty((B, T, C))
        lib.attention_forward_dispatch(xt, mask, H, caches, yt)
        y = rt.to_numpy(yt)
        rt.free(xt)  # attention.c:123 frees the input right after the call
        y_ref, q, k, v, att = oracle.forward(x, H)
        check("y", y, y_ref)
        for i, ref in enumerate((q, k, v)):
            assert np.array_equal(rt.to_numpy(caches[i]), ref), f"cache[{i}]"
        dyt = rt.from_numpy(dy)
        dout = lib.zeros((ctypes.c_int * 3)(B, T, 3 * C), 3, gptc.CUDA)
        lib.attention_backward_dispatch(dyt, caches, H, dout)
        d = rt.to_numpy(dout)
        d_ref = oracle.backward(dy, H, q, k, v, att)
        check("dqkv", d, d_ref)
        for t in (yt, dyt, dout, mask, *caches):
            rt.free(t)
        rt.sync()


def test_output_freed_before_backward(rt, oracle):
    """SelfAttention's c_proj frees y before attention's backward runs
    (gpt.c self_attention.c:78, linear.c:215).  The layer keeps y by sharing
    its storage, so the backward must still see the forward's y."""
    B, T, C, H = 2, 200, 256, 4
    x, dy = qkv_inputs(rt, B, T, C, 41, 42)
    layer = gptc.AttentionLayer(rt, C, H, T)
    layer.to(gptc.CUDA)
    yt = layer.forward(rt.from_numpy(x))
    y = rt.to_numpy(yt)
    rt.free(yt)
    # Fresh allocations of y's size must not land on the kept storage.
    junk = [rt.from_numpy(np.full((B, T, C), 7.0, np.float32)) for _ in range(3)]
    dt = layer.backward(rt.from_numpy(dy))
    y_ref, q, k, v, att = oracle.forward(x, H)
    check("y", y, y_ref)
    check("dqkv", rt.to_numpy(dt), oracle.backward(dy, H, q, k, v, att))
    for t in junk + [dt]:
        rt.free(t)
    layer.free()
    rt.sync()


def test_compact_layout_with_own_output_copy(rt, oracle):
    """The entry points with compact caches whose cache[1] is a buffer of its
    own (not the output's storage): the forward copies y there."""
    lib = rt.lib
    B, T, C, H = 2, 300, 256, 4
    x, dy = qkv_inputs(rt, B, T, C, 51, 52)
    xt = rt.from_numpy(x)
    mask = rt.from_numpy(np.tril(np.ones((T, T), np.float32)))
    n_state = lib.gptc_attention_state_floats(B, T, C, H)
    caches = (gptc.TensorP * 4)(xt, rt.empty((B, T, C)), rt.empty((B, H, T)), rt.empty((n_state,)))
    yt, dout = rt.empty((B, T, C)), rt.empty((B, T, 3 * C))
    lib.attention_forward_cuda_kernel(xt, mask, H, caches, yt)
    y = rt.to_numpy(yt)
    assert np.array_equal(rt.to_numpy(caches[1]), y)
    lib.fill_tensor_data_cuda(yt, ctypes.c_float(3.0))  # the backward must read the copy, not yt
    dyt = rt.from_numpy(dy)
    lib.attention_backward_cuda_kernel(dyt, caches, H, dout)
    y_ref, q, k, v, att = oracle.forward(x, H)
    check("y", y, y_ref)
    check("dqkv", rt.to_numpy(dout), oracle.backward(dy, H, q, k, v, att))
    for t in (dyt, mask, yt, dout, *caches):
        rt.free(t)
    rt.sync()


def test_deterministic(rt):
    x, dy = qkv_inputs(rt, 2, 300, 256, 11, 12)
    a = run_layer(rt, x, dy, 4)
    b = run_layer(rt, x, dy, 4)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


def test_forward_pool_over_repeated_launches(rt, oracle):
    """C2's forward leaves blocks 0..2 of every head to a pool that workgroups
    take from through device counters, which the last workgroup resets for
    the next launch (block_sched.hpp).  Three launches in a row, each into an
    output filled with NaN first, on other inputs each time: a block the
    pool lost would leave NaN rows, a stale counter would lose the blocks of
    the next launch.  Every launch against the oracle."""
    lib = rt.lib
    B, T, C, H = 8, 1024, 768, 12
    mask = rt.from_numpy(np.tril(np.ones((T, T), np.float32)))
    n_state = lib.gptc_attention_state_floats(B, T, C, H)
    for launch, seed in enumerate((61, 62, 63)):
        x = rt.normal((B, T, 3 * C), seed)
        xt = rt.from_numpy(x)
        yt = rt.from_numpy(np.full((B, T, C), np.nan, np.float32))
        caches = (gptc.TensorP * 4)(xt, yt, rt.empty((B, H, T)), rt.empty((n_state,)))
        lib.attention_forward_cuda_kernel(xt, mask, H, caches, yt)
        y = rt.to_numpy(yt)
        print(f"launch {launch}: seed {seed}", flush=True)
        check("y", y, oracle.forward(x, H)[0])
        for t in (xt, yt, caches[2], caches[3]):
            rt.free(t)
    rt.free(mask)
    rt.sync()


def test_split_key_blocks_b1_t1024(rt, oracle):
    """B*H = 12 heads of T = 1024 fill 96 of the GPU's dk/dv workgroup slots, so
    each key block with two or more query tiles runs as two workgroups over
    halves of its query range, adding into dK, dV rows the delta kernel zeroed:
    oracle parity, and the same bits again (two addends in either order)."""
    compare_with_oracle(rt, oracle, 1, 1024, 768, 12)
    x, dy = qkv_inputs(rt, 1, 1024, 768, 31, 32)
    a = run_layer(rt, x, dy, 12)
    b = run_layer(rt, x, dy, 12)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


def test_split_key_blocks_ragged_t(rt, oracle):
    """Split key blocks when T is not a multiple of the 64-query tile (T = 1000:
    the last key block and the last query half are partial)."""
    compare_with_oracle(rt, oracle, 1, 1000, 768, 12)


@pytest.fixture
def lse_only_state(rt):
    """Every D = 64 forward keeps only the log-sum-exp (state limit 0); the
    default limit is restored afterwards."""
    rt.lib.gptc_attention_set_state_limit(0)
    yield
    rt.lib.gptc_attention_set_state_limit(-1)


def ds_floats_per_head(T):
    """Floats of one head's packed causal dS blocks ([64 queries][32 keys]
    for key blocks 0 .. 2qt+1 of each 64-query tile qt)."""
    nqt = (T + 63) // 64
    return nqt * (nqt + 1) * 64 * 32


@contextlib.contextmanager
def scratch_limit(rt, floats):
    rt.lib.gptc_attention_set_scratch_limit(floats)
    try:
        yield
    finally:
        rt.lib.gptc_attention_set_scratch_limit(-1)


@pytest.mark.parametrize("scratch", ["whole", "chunks", "none"])
@pytest.mark.parametrize("B,T,C,H", [(2, 1024, 768, 12), (1, 1000, 768, 12), (1, 200, 128, 2), (2, 100, 256, 4),
                                     (1, 129, 128, 2), (3, 65, 128, 2), (1, 1, 64, 1), (3, 333, 320, 5)])
def test_lse_only_state_fwd_bwd(rt, oracle, lse_only_state, B, T, C, H, scratch):
    """The backward of the LSE-only state (its state is O(T) per head), used
    when the probability blocks would exceed the state limit: the dk/dv
    kernel recomputes P from the saved log-sum-exp, and dQ comes from dS
    written to a scratch of every head at once ("whole"), of heads in chunks
    of at most 5 ("chunks": uneven last chunk where B*H is not a multiple of
    5), or, with no scratch ("none"), from a dq kernel that recomputes S and
    dP too.  Each meets the same tolerance."""
    n = rt.lib.gptc_attention_state_floats(B, T, C, H)
    assert n < B * H * T * 8 + B * ((T + 63) // 64) * C + 4 * B * ((T + 127) // 128) * C + 4096
    limit = {"whole": -1, "chunks": 5 * ds_floats_per_head(T), "none": 0}[scratch]
    with scratch_limit(rt, limit):
        compare_with_oracle(rt, oracle, B, T, C, H)


def test_long_sequence_past_the_state_cap(rt, oracle):
    """B=8 H=12 T=6700: the probability blocks would need 2.19e9 floats, past
    the int length of a tensor_t, so the forward keeps the LSE-only state by
    default (it refused the shape before that state existed).  Causality pins
    the result: with dy zero past row 1024, the first 1024 rows of y and of
    dq, dk, dv equal those of a T = 1024 run of the same rows (the
    probability-block path), which is checked against the oracle."""
    B, T, C, H, T0 = 8, 6700, 768, 12, 1024
    n = rt.lib.gptc_attention_state_floats(B, T, C, H)
    assert n < 2 * B * H * T + B * ((T + 63) // 64) * C + 4 * B * ((T + 127) // 128) * C + 4096
    x, dy = qkv_inputs(rt, B, T, C, 41, 42)
    dy[:, T0:] = 0.0
    y, lse, d = run_layer(rt, x, dy, H)
    assert np.isfinite(y).all() and np.isfinite(d).all()
    y0, lse0, d0 = run_layer(rt, np.ascontiguousarray(x[:, :T0]), np.ascontiguousarray(dy[:, :T0]), H)
    check("y rows < 1024 vs T=1024", y[:, :T0], y0)
    check("lse rows < 1024", lse[:, :, :T0], lse0)
    check("dqkv rows < 1024 vs T=1024", d[:, :T0], d0)
    y_ref, q, k, v, att = oracle.forward(np.ascontiguousarray(x[:, :T0]), H)
    check("y vs oracle", y0, y_ref)
    check("dqkv vs oracle", d0, oracle.backward(np.ascontiguousarray(dy[:, :T0]), H, q, k, v, att))


def test_lse_only_state_deterministic(rt, lse_only_state):
    x, dy = qkv_inputs(rt, 2, 300, 256, 11, 12)
    a = run_layer(rt, x, dy, 4)
    b = run_layer(rt, x, dy, 4)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


def test_causality_at_full_length(rt):
    B, T, C, H = 2, 1024, 768, 12
    x, dy = qkv_inputs(rt, B, T, C, 21, 22)
    y, _, d = run_layer(rt, x, dy, H)
    x2 = x.copy()
    x2[:, 600:] = rt.normal((B, T - 600, 3 * C), 23)
    y2, _, d2 = run_layer(rt, x2, dy, H)
    assert np.array_equal(y[:, :600], y2[:, :600])
    assert np.array_equal(d[:, :600, :C], d2[:, :600, :C])
    assert not np.array_equal(y[:, 600:], y2[:, 600:])


def test_forward_twice_then_backward(rt, oracle):
    """A second forward without backward drops the first cache (no leak, no mix-up)."""
    B, T, C, H = 1, 90, 128, 2
    layer = gptc.AttentionLayer(rt, C, H, T)
    layer.to(gptc.CUDA)
    x1, _ = qkv_inputs(rt, B, T, C, 31, 32)
    x2, dy = qkv_inputs(rt, B, T, C, 33, 34)
    rt.free(layer.forward(rt.from_numpy(x1)))
    yt = layer.forward(rt.from_numpy(x2))
    dt = layer.backward(rt.from_numpy(dy))
    y_ref, q, k, v, att = oracle.forward(x2, H)
    check("y", rt.to_numpy(yt), y_ref)
    check("dqkv", rt.to_numpy(dt), oracle.backward(dy, H, q, k, v, att))
    rt.free(yt)
    rt.free(dt)
    layer.free()
    rt.sync()


def test_device_tensor_ops(rt):
    lib = rt.lib
    a = rt.normal((3, 1001), 5)
    t = rt.from_numpy(a)
    assert np.array_equal(rt.to_numpy(t), a)
    c = rt.empty((3, 1001))
    lib.tensor_copy(c, t)
    assert np.array_equal(rt.to_numpy(c), a)
    f = lib.fill((ctypes.c_int * 1)(1003), 1, ctypes.c_float(-1.5), gptc.CUDA)
    z = lib.zeros((ctypes.c_int * 1)(7), 1, gptc.CUDA)
    r = lib.arange(2, 20, 3, gptc.CUDA)
    assert np.array_equal(rt.to_numpy(f), np.full(1003, -1.5, np.float32))
    assert np.array_equal(rt.to_numpy(z), np.zeros(7, np.float32))
    assert np.array_equal(rt.to_numpy(r), [[2, 5, 8, 11, 14, 17]])
    for x in (t, c, f, z, r):
        rt.free(x)
    rt.sync()


MASK_SCRIPT = """
import sys
sys.path.insert(0, {pkg!r})
import numpy as np
import gptc
lib = gptc.load()
rt = gptc.Runtime(lib)
rt.init()
B, T, C, H = 1, 96, 128, 2
x = rt.from_numpy(np.ones((B, T, 3 * C), np.float32))
n = lib.gptc_attention_state_floats(B, T, C, H)
caches = (gptc.TensorP * 4)(x, rt.empty((B, T, C)), rt.empty((B, H, T)), rt.empty((n,)))
m = np.tril(np.ones((T + 4, T + 4), np.float32))
m[T:, :] = 7.0  # outside the T x T block a call reads: ignored
mask = rt.from_numpy(m)
lib.attention_forward_cuda_kernel(x, mask, H, caches, caches[1])
rt.sync()
print("causal ok", flush=True)
{second}
lib.attention_forward_cuda_kernel(x, mask, H, caches, caches[1])
rt.sync()
print("returned", flush=True)
"""


def test_host_mask_is_checked_at_every_call(rt, oracle):
    """A mask in host memory (the C-ABI accepts one; gpt.c's dispatcher would
    not pass it) is read directly at every call: the causal buffer runs, and
    the result matches the oracle."""
    B, T, C, H = 1, 70, 128, 2
    x, _ = qkv_inputs(rt, B, T, C, 71, 72)
    lib = rt.lib
    xt = rt.from_numpy(x)
    mask = rt.from_numpy(np.tril(np.ones((T + 2, T + 2), np.float32)), gptc.CPU)
    n = lib.gptc_attention_state_floats(B, T, C, H)
    caches = (gptc.TensorP * 4)(xt, rt.empty((B, T, C)), rt.empty((B, H, T)), rt.empty((n,)))
    lib.attention_forward_cuda_kernel(xt, mask, H, caches, caches[1])
    y_ref, *_ = oracle.forward(x, H)
    check("y", rt.to_numpy(caches[1]), y_ref)
    for t in (mask, *caches):
        rt.free(t)
    rt.sync()


@pytest.mark.parametrize("case", ["edited_entry", "refilled_buffer", "host_mask"])
def test_non_causal_mask_is_refused(case):
    """gpt.c applies whatever the mask holds (kernels/src/cpu/Attention.c:139);
    these kernels apply the causal rule from indices, so a mask that differs
    from tril on the T x T block is a fatal error before any launch, including
    a mask the library already checked and then rewrote (the check follows
    the buffer's allocation serial)."""
    import os
    import subprocess
    import sys
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gpt.c_amd")
    second = {
        # A fresh buffer whose entry (5, 3) is not 1: a key at or below the diagonal masked out.
        "edited_entry": "m2 = np.tril(np.ones((T, T), np.float32)); m2[5, 3] = 0.0; mask = rt.from_numpy(m2)",
        # The checked buffer refilled with ones (future keys visible) through the library.
        "refilled_buffer": "lib.fill_tensor_data_cuda(mask, 1.0)",
        # A host-memory mask with a visible future key.
        "host_mask": "m3 = np.tril(np.ones((T, T), np.float32)); m3[2, 9] = 1.0; mask = rt.from_numpy(m3, gptc.CPU)",
    }[case]
    r = subprocess.run([sys.executable, "-c", MASK_SCRIPT.format(pkg=pkg, second=second)], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout, r.stderr[-400:])
    assert "causal ok" in r.stdout, r.stderr
    assert r.returncode != 0 and "returned" not in r.stdout and "causal mask" in r.stderr, r.stderr
