"""GPU parity of the rest of gpt.c's device back end (include/gpu_kernels.h):
Linear, LayerNorm, GELU, Softmax, Embedding, CrossEntropy, AdamW, saxpy and
the sgemm entry points, each called through the C-ABI and compared with the
CPU oracle (oracle/ops_oracle.c, the restatement of gpt.c's CPU kernels that
tests/test_oracle_ops.py pins) on the same seeded inputs.

Tolerances (max abs error): 1e-5 for elementwise and row ops on O(1)
values; for GEMM results 2e-5 x max|reference| (fp32 sums of up to a few
thousand products, rocBLAS and OpenBLAS summing in different orders).
Integer-like work (embedding gather, deterministic scatter) is bit-exact.
"""
import ctypes

import numpy as np
import pytest

import gptc
import oracle as oracle_mod

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1234)


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def check(name, got, ref, atol=1e-5, rtol=0.0):
    ref = np.asarray(ref, np.float64)
    tol = atol + rtol * (float(np.abs(ref).max()) if ref.size else 0.0)
    err = float(np.abs(got.astype(np.float64) - ref).max()) if got.size else 0.0
    print(f"  {name}: max abs err {err:.3e} (tol {tol:.1e})")
    assert np.isfinite(got).all(), name
    assert err <= tol, f"{name}: {err:.3e} > {tol:.1e}"


@pytest.fixture(scope="module")
def ops(oracle):
    return oracle_mod.Ops(oracle)


class Dev:
    """Device copies of numpy arrays, freed together."""

    def __init__(self, rt):
        self.rt, self.ts = rt, []

    def __call__(self, a):
        t = self.rt.from_numpy(a)
        self.ts.append(t)
        return t

    def empty(self, shape):
        t = self.rt.empty(shape)
        self.ts.append(t)
        return t

    def list(self, arrays):
        ts = [self(a) for a in arrays]
        return (gptc.TensorP * len(ts))(*ts)

    def get(self, t):
        return self.rt.to_numpy(t)

    def free(self):
        for t in self.ts:
            self.rt.free(t)
        self.ts = []


@pytest.fixture
def dev(rt):
    d = Dev(rt)
    yield d
    d.free()


@pytest.mark.parametrize("B,T,in_f,out_f,bias", [
    (2, 9, 24, 40, True),
    (1, 5, 7, 3, False),
    (4, 256, 768, 3072, True),   # GPT-2 c_fc
    (2, 128, 3072, 768, True),   # GPT-2 mlp c_proj
    (1, 64, 768, 2304, True),    # GPT-2 qkv
    (2, 64, 768, 50257, False),  # GPT-2 lm_head: dx split over 4 slices of 12564 terms + 1 leftover term
    (1, 3, 7, 16391, True),      # dx split over 2 slices + 1 leftover term, scalar (in_f % 4 != 0) add
    (1, 16, 64, 32768, True),    # dx split over 4 slices, no leftover terms
])
def test_linear(dev, ops, B, T, in_f, out_f, bias):
    print(f"case linear B={B} T={T} in={in_f} out={out_f} bias={bias}")
    x, W, g = rnd(B, T, in_f), rnd(out_f, in_f, scale=0.02), rnd(B, T, out_f)
    b = rnd(out_f) if bias else None
    dW0, db0 = rnd(out_f, in_f), rnd(out_f)
    y = dev.empty((B, T, out_f))
    dev.rt.lib.linear_forward_cuda_kernel(dev(W), dev(b) if bias else None, dev(x), y)
    y_ref = ops.linear_forward(W, b, x)
    check("y", dev.get(y), y_ref, rtol=2e-5)
    dW_t, db_t, dx_t = dev(dW0), dev(db0) if bias else None, dev.empty((B, T, in_f))
    dev.rt.lib.linear_backward_cuda_kernel(dev(g), dev(x), dev(W), dW_t, db_t, dx_t)
    dW, db = dW0.copy(), db0.copy()
    dx_ref = ops.linear_backward(g, x, W, dW, db if bias else None)
    check("dx", dev.get(dx_t), dx_ref, rtol=2e-5)
    check("dW (accumulated)", dev.get(dW_t), dW, rtol=2e-5)
    if bias:
        check("db (accumulated)", dev.get(db_t), db, rtol=2e-5)


@pytest.mark.parametrize("in_f,out_f", [(768, 3072), (3072, 768), (768, 2304)])
def test_linear_tuned_gemm_shapes(dev, in_f, out_f):
    """GPT-2's Linear shapes at C3's 8192 rows run rocBLAS solutions from
    the library's tuned table (csrc/gemm_tuned.inc).  Outputs prefilled with
    NaN: a solution's first call (validated, then run) must compute every
    entry and read nothing of C where beta = 0.  Checked against float64
    numpy: y and dx on every 61st row, dW in full (accumulated onto dW0)."""
    print(f"case tuned linear in={in_f} out={out_f}")
    B, T = 8, 1024
    x, W, g = rnd(B, T, in_f), rnd(out_f, in_f, scale=0.02), rnd(B, T, out_f)
    b, dW0, db0 = rnd(out_f), rnd(out_f, in_f), rnd(out_f)
    y = dev(np.full((B, T, out_f), np.nan, np.float32))
    dev.rt.lib.linear_forward_cuda_kernel(dev(W), dev(b), dev(x), y)
    x2, g2 = x.reshape(-1, in_f).astype(np.float64), g.reshape(-1, out_f).astype(np.float64)
    W64 = W.astype(np.float64)
    y_ref = x2[::61] @ W64.T + b
    check("y (every 61st row)", dev.get(y).reshape(-1, out_f)[::61], y_ref, rtol=2e-5)
    dW_t, db_t = dev(dW0), dev(db0)
    dx = dev(np.full((B, T, in_f), np.nan, np.float32))
    dev.rt.lib.linear_backward_cuda_kernel(dev(g), dev(x), dev(W), dW_t, db_t, dx)
    check("dx (every 61st row)", dev.get(dx).reshape(-1, in_f)[::61], g2[::61] @ W64, rtol=2e-5)
    check("dW (accumulated)", dev.get(dW_t), dW0 + g2.T @ x2, rtol=2e-5)
    check("db (accumulated)", dev.get(db_t), db0 + g2.sum(0), rtol=2e-5)


@pytest.mark.parametrize("B,T,C", [(2, 7, 48), (4, 64, 768), (3, 5, 1600), (1, 3, 2048), (2, 3, 5), (8, 33, 1024)])
def test_layer_norm(dev, ops, B, T, C):
    print(f"case layer_norm B={B} T={T} C={C}")
    x, W, b, g = rnd(B, T, C, scale=2.0) + 0.5, rnd(C), rnd(C), rnd(B, T, C)
    mean, rstd, y = dev.empty((B, T)), dev.empty((B, T)), dev.empty((B, T, C))
    cache = (gptc.TensorP * 2)(mean, rstd)
    dev.rt.lib.layer_norm_forward_cuda_kernel(dev(W), dev(b), dev(x), 1e-5, cache, y)
    y_ref, m_ref, r_ref = ops.layer_norm_forward(x, W, b)
    check("y", dev.get(y), y_ref)
    check("mean", dev.get(mean), m_ref)
    check("rstd", dev.get(rstd), r_ref, rtol=1e-6)
    dW0, db0, dx0 = rnd(C), rnd(C), rnd(B, T, C)
    dW_t, db_t, dx_t = dev(dW0), dev(db0), dev(dx0)
    cache3 = (gptc.TensorP * 3)(dev(m_ref), dev(r_ref), dev(x))
    dev.rt.lib.layer_norm_backward_cuda_kernel(dev(g), cache3, dev(W), dW_t, db_t, dx_t)
    dW, db, dx = dW0.copy(), db0.copy(), dx0.copy()
    ops.layer_norm_backward(g, x, m_ref, r_ref, W, dW, db, dx)
    check("dx (accumulated)", dev.get(dx_t), dx, atol=2e-5)
    check("dW (accumulated)", dev.get(dW_t), dW, rtol=2e-6, atol=2e-5)
    check("db (accumulated)", dev.get(db_t), db, rtol=2e-6, atol=2e-5)
    # The layer's form writes dx over whatever dout holds (NaN here) and
    # still accumulates dW and db.
    dx_set = dev(np.full((B, T, C), np.nan, np.float32))
    dev.rt.lib.gptc_layer_norm_backward_set(dev(g), cache3, dev(W), dW_t, db_t, dx_set)
    dx2 = np.zeros_like(dx0)
    ops.layer_norm_backward(g, x, m_ref, r_ref, W, dW, db, dx2)
    check("dx (written)", dev.get(dx_set), dx2, atol=2e-5)
    check("dW (accumulated twice)", dev.get(dW_t), dW, rtol=2e-6, atol=4e-5)
    check("db (accumulated twice)", dev.get(db_t), db, rtol=2e-6, atol=4e-5)


def test_layer_norm_without_bias(dev, ops):
    x, W = rnd(3, 4, 100), rnd(100)
    mean, rstd, y = dev.empty((3, 4)), dev.empty((3, 4)), dev.empty((3, 4, 100))
    dev.rt.lib.layer_norm_forward_cuda_kernel(dev(W), None, dev(x), 1e-5, (gptc.TensorP * 2)(mean, rstd), y)
    check("y (no bias)", dev.get(y), ops.layer_norm_forward(x, W, None)[0])


@pytest.mark.parametrize("n", [1, 3, 4 * 97 * 33 + 3, 1 << 20])
def test_gelu(dev, ops, n):
    x, g = rnd(n, scale=3.0), rnd(n)
    y, dx = dev.empty((n,)), dev.empty((n,))
    xt = dev(x)
    dev.rt.lib.gelu_forward_cuda_kernel(xt, y)
    dev.rt.lib.gelu_backward_cuda_kernel(dev(g), xt, dx)
    check("gelu", dev.get(y), ops.gelu_forward(x))
    check("gelu'", dev.get(dx), ops.gelu_backward(g, x))


def test_gelu_extreme_inputs(dev, ops):
    """Saturated inputs give exactly x and 0 (and slopes 1 and 0), tiny ones
    the linear part, NaN stays NaN; errors stay within the elementwise
    tolerance over [-30, 30]."""
    x = np.concatenate([np.linspace(-30, 30, 6001), [-1e30, -100.0, 100.0, 1e30], np.logspace(-30, -1, 31),
                        -np.logspace(-30, -1, 31), [0.0, -0.0]]).astype(np.float32)
    g = np.ones_like(x)
    y, dx = dev.empty(x.shape), dev.empty(x.shape)
    xt = dev(x)
    dev.rt.lib.gelu_forward_cuda_kernel(xt, y)
    dev.rt.lib.gelu_backward_cuda_kernel(dev(g), xt, dx)
    yg, dg = dev.get(y), dev.get(dx)
    ok = np.abs(x) < 1e29  # x**3 overflows past about 1e12 (both sides give inf * 0 or saturate)
    check("gelu (wide range)", yg[ok], ops.gelu_forward(x)[ok])
    check("gelu' (wide range)", dg[ok], ops.gelu_backward(g, x)[ok])
    big = (np.abs(x) >= 10) & ok
    assert np.array_equal(yg[big & (x > 0)], x[big & (x > 0)]) and np.all(yg[big & (x < 0)] == 0)
    assert np.all(dg[big & (x > 0)] == 1) and np.all(dg[big & (x < 0)] == 0)
    xn = dev(np.array([np.nan, 1.0], np.float32))
    yn = dev.empty((2,))
    dev.rt.lib.gelu_forward_cuda_kernel(xn, yn)
    assert np.isnan(dev.get(yn)[0])


@pytest.mark.parametrize("B,T,C", [(8, 33, 3072), (2, 5, 7), (1, 1, 4), (3, 100, 768)])
def test_gelu_with_bias(dev, ops, B, T, C):
    """The MLP's fused form: gelu(x + b) forward; backward dx = g gelu'(x + b)
    and db += the column sums of dx (float4 path for C % 4 == 0, the scalar
    path plus the column-sum kernels otherwise)."""
    print(f"case gelu+bias B={B} T={T} C={C}")
    x, b, g = rnd(B, T, C, scale=2.0), rnd(C), rnd(B, T, C)
    db0 = rnd(C)
    y, dx = dev.empty((B, T, C)), dev.empty((B, T, C))
    xt, bt, db_t = dev(x), dev(b), dev(db0)
    dev.rt.lib.gptc_gelu_forward_bias_cuda(xt, bt, y)
    xb = (x + b).astype(np.float32)
    check("gelu(x + b)", dev.get(y), ops.gelu_forward(xb))
    dev.rt.lib.gptc_gelu_backward_bias_cuda(dev(g), xt, bt, dx, db_t)
    dx_ref = ops.gelu_backward(g, xb)
    check("dx", dev.get(dx), dx_ref)
    db_ref = db0.astype(np.float64) + dx_ref.astype(np.float64).reshape(-1, C).sum(0)
    check("db (accumulated)", dev.get(db_t), db_ref, atol=1e-5 * max(1, B * T) ** 0.5)


@pytest.mark.parametrize("rows,C", [(15, 37), (8, 50257), (3, 1), (700, 64)])
def test_softmax(dev, ops, rows, C):
    x, g = rnd(rows, C, scale=3.0), rnd(rows, C)
    if C > 4:
        x[0, :C // 2] = -np.inf  # masked entries contribute exp(-inf) = 0
    y, dx = dev.empty((rows, C)), dev.empty((rows, C))
    dev.rt.lib.softmax_forward_cuda_kernel(dev(x), y)
    p_ref = ops.softmax_forward(x)
    # The oracle adds the C exponentials one after another in fp32 (relative
    # error growing like sqrt(C) eps, about 1e-5 at C = 50257); the kernel
    # adds them in a tree.  Hence a tolerance relative to the largest value.
    check("softmax", dev.get(y), p_ref, atol=1e-6, rtol=5e-5)
    dev.rt.lib.softmax_backward_cuda_kernel(dev(g), dev(p_ref), dx)
    check("softmax'", dev.get(dx), ops.softmax_backward(g, p_ref), atol=1e-6, rtol=5e-5)
    np.testing.assert_allclose(dev.get(y).sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("V,C,B,T", [(50257, 768, 8, 1024), (11, 8, 3, 7), (1024, 768, 8, 1024), (5, 6, 2, 3)])
def test_embedding(dev, ops, V, C, B, T):
    print(f"case embedding V={V} C={C} B={B} T={T}")
    W, g = rnd(V, C), rnd(B, T, C)
    ids = RNG.integers(0, V, (B, T)).astype(np.float32)
    ids[0, :3] = ids[-1, -1]  # repeated ids
    y = dev.empty((B, T, C))
    dev.rt.lib.embedding_forward_cuda_kernel(dev(W), dev(ids), y)
    assert np.array_equal(dev.get(y), ops.embedding_forward(W, ids)), "gather"
    # token ids, then the position table's shared arange(T)
    for cache in (ids, np.arange(T, dtype=np.float32)[None, :]):
        if cache.max() >= V:
            continue
        dW0 = rnd(V, C)
        dW_t = dev(dW0)
        dev.rt.lib.embedding_backward_cuda_kernel(dev(g), dev(cache), dW_t)
        dW = dW0.copy()
        ops.embedding_backward(g, cache, dW)
        # the same row order as gpt.c's loop: bit-exact
        assert np.array_equal(dev.get(dW_t), dW), "scatter-add"


def test_embedding_out_of_range_ids(dev, ops):
    V, C = 10, 16
    W, g = rnd(V, C), rnd(1, 4, C)
    ids = np.array([[1, 10, -1, 3]], np.float32)
    y = dev.empty((1, 4, C))
    dev.rt.lib.embedding_forward_cuda_kernel(dev(W), dev(ids), y)
    out = dev.get(y)
    assert np.array_equal(out[0, 0], W[1]) and np.array_equal(out[0, 3], W[3])
    assert np.isnan(out[0, 1]).all() and np.isnan(out[0, 2]).all()
    dW = dev(np.zeros((V, C), np.float32))
    dev.rt.lib.embedding_backward_cuda_kernel(dev(g), dev(ids), dW)
    ref = np.zeros((V, C), np.float32)
    ref[1] += g[0, 0]
    ref[3] += g[0, 3]
    assert np.array_equal(dev.get(dW), ref)


@pytest.mark.parametrize("B,T,V", [(3, 5, 37), (2, 64, 50257), (1, 1, 1)])
def test_cross_entropy(dev, ops, B, T, V):
    print(f"case cross_entropy B={B} T={T} V={V}")
    logits = rnd(B, T, V, scale=2.0)
    tg = RNG.integers(0, V, (B, T)).astype(np.float32)
    lsm, loss = dev.empty((B, T, V)), dev.empty((1,))
    tg_t = dev(tg)
    dev.rt.lib.cross_entropy_forward_cuda_kernel(dev(logits), tg_t, (gptc.TensorP * 1)(lsm), loss)
    lsm_ref, loss_ref = ops.cross_entropy_forward(logits, tg)
    # log of a 50257-term fp32 sum (sequential in the oracle): ~1e-5 apart
    check("log-softmax", dev.get(lsm), lsm_ref, atol=1e-4)
    check("loss", dev.get(loss), np.array([loss_ref]), atol=1e-4)
    g = rnd(B, T)
    d = dev.empty((B, T, V))
    dev.rt.lib.cross_entropy_backward_cuda_kernel(dev(g), (gptc.TensorP * 2)(dev(lsm_ref), tg_t), d)
    check("dlogits", dev.get(d), ops.cross_entropy_backward(g, lsm_ref, tg), atol=1e-7)


@pytest.mark.parametrize("B,T,V", [(2, 3, 8 * 2048 + 3), (2, 2, 8 * 2048 + 5), (1, 3, 25 * 2048 + 3),
                                   (2, 2, 32 * 2048 + 1), (1, 2, 70001)])
def test_cross_entropy_row_sizes_and_masked_logits(dev, ops, B, T, V):
    """Rows at the edges of the register-resident forms (8, 25 and 32 float4
    per lane) and one longer row (the streaming kernels), with -inf logits
    (masked entries) in every row and one row masked but for its target."""
    print(f"case cross_entropy rows B={B} T={T} V={V}")
    logits = rnd(B, T, V, scale=2.0)
    logits[..., 7::13] = -np.inf
    tg = RNG.integers(0, V, (B, T)).astype(np.float32)
    tg = np.where(tg % 13 == 7, tg - 1, tg)  # targets on unmasked entries
    logits[0, 0, :] = -np.inf
    logits[0, 0, int(tg[0, 0])] = 3.0
    lsm, loss = dev.empty((B, T, V)), dev.empty((1,))
    tg_t = dev(tg)
    dev.rt.lib.cross_entropy_forward_cuda_kernel(dev(logits), tg_t, (gptc.TensorP * 1)(lsm), loss)
    lsm_ref, loss_ref = ops.cross_entropy_forward(logits, tg)
    got = dev.get(lsm)
    assert np.array_equal(np.isneginf(got), np.isneginf(lsm_ref))
    fin = np.isfinite(lsm_ref)
    check("log-softmax (finite entries)", got[fin], lsm_ref[fin], atol=1e-4)
    assert abs(got[0, 0, int(tg[0, 0])]) <= 1e-6  # the only unmasked logit of its row
    check("loss", dev.get(loss), np.array([loss_ref]), atol=1e-4)
    g = rnd(B, T)
    d = dev.empty((B, T, V))
    dev.rt.lib.cross_entropy_backward_cuda_kernel(dev(g), (gptc.TensorP * 2)(dev(lsm_ref), tg_t), d)
    check("dlogits", dev.get(d), ops.cross_entropy_backward(g, lsm_ref, tg), atol=1e-7)


def test_cross_entropy_uniform_logits_and_bad_target(dev):
    B, T, V = 2, 3, 50257
    logits = np.zeros((B, T, V), np.float32)
    tg = np.array([[0, 5, 50256], [7, 50257, 1]], np.float32)  # 50257 is out of range
    lsm, loss = dev.empty((B, T, V)), dev.empty((1,))
    dev.rt.lib.cross_entropy_forward_cuda_kernel(dev(logits), dev(tg), (gptc.TensorP * 1)(lsm), loss)
    np.testing.assert_allclose(dev.get(lsm), -np.log(V), rtol=1e-6)
    assert np.isnan(dev.get(loss)[0])  # a target outside [0, V) makes the mean NaN
    tg[1, 1] = 2
    dev.rt.lib.cross_entropy_forward_cuda_kernel(dev(logits), dev(tg), (gptc.TensorP * 1)(lsm), loss)
    assert abs(dev.get(loss)[0] - np.log(V)) <= 1e-5


def test_adamw_multi_tensor(dev, ops):
    # 40 tensors (two launches of at most 36), odd lengths, a 0-length one
    sizes = [1, 3, 4, 5, 17, 4096, 4097, 65536 + 3, 0, 768] * 4
    params = [rnd(n) for n in sizes]
    grads_seq = [[rnd(n) for n in sizes] for _ in range(3)]
    m = [np.zeros(n, np.float32) for n in sizes]
    v = [np.zeros(n, np.float32) for n in sizes]
    pt, gt = dev.list(params), dev.list(grads_seq[0])
    mt, vt = dev.list(m), dev.list(v)
    lr, b1, b2, wd, eps = 1e-3, 0.9, 0.99, 0.1, 1e-8
    for step, grads in enumerate(grads_seq, 1):
        for i, g in enumerate(grads):  # write this step's gradients into the listed tensors
            dev.rt.lib.tensor_copy(gt[i], dev(g))
        dev.rt.lib.step_adamW_cuda_kernel(pt, gt, mt, vt, len(sizes), lr, b1, b2, wd, eps, step)
        for i in range(len(sizes)):
            ops.adamw(params[i], grads[i], m[i], v[i], lr, b1, b2, wd, eps, step)
    for i in range(len(sizes)):
        check(f"p[{i}]", dev.get(pt[i]), params[i], atol=1e-6)
        check(f"m[{i}]", dev.get(mt[i]), m[i], atol=1e-6)
        check(f"v[{i}]", dev.get(vt[i]), v[i], atol=1e-6)
    dev.rt.lib.zero_grad_adamW_cuda_kernel(gt, len(sizes))
    for i, n in enumerate(sizes):
        assert not dev.get(gt[i]).any()


def test_saxpy_offsets_and_strides(dev):
    x, y = rnd(100), rnd(300)
    yt = dev(y)
    dev.rt.lib.saxpy_cuda(7, 2.5, dev(x), 3, 5, yt, 11, 9)
    ref = y.copy()
    ref[11:11 + 9 * 7:9] += np.float32(2.5) * x[3:3 + 5 * 7:5]
    check("strided", dev.get(yt), ref, atol=1e-6)
    x2, y2 = rnd(1 << 20 | 3), rnd(1 << 20 | 3)
    yt2 = dev(y2)
    dev.rt.lib.saxpy_cuda(x2.size, -0.5, dev(x2), 0, 1, yt2, 0, 1)
    check("unit stride", dev.get(yt2), y2 - 0.5 * x2, atol=1e-6)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_transposes_offsets(dev, ta, tb):
    M, N, K = 37, 29, 53
    A = rnd(K, M) if ta else rnd(M, K)
    Bm = rnd(N, K) if tb else rnd(K, N)
    C0 = rnd(M, N + 3)  # ldc = N + 3
    a_off, b_off, c_off = 5, 2, 4
    Af = np.concatenate([rnd(a_off), A.ravel()])
    Bf = np.concatenate([rnd(b_off), Bm.ravel()])
    Cf = np.concatenate([rnd(c_off), C0.ravel()])
    Ct = dev(Cf)
    lda, ldb = A.shape[1], Bm.shape[1]
    dev.rt.lib.sgemm_cuda(ta, tb, M, N, K, 0.75, dev(Af), a_off, lda, dev(Bf), b_off, ldb, 0.5, Ct, c_off, N + 3)
    opA = A.T if ta else A
    opB = Bm.T if tb else Bm
    ref = C0.astype(np.float64).copy()
    ref[:, :N] = 0.75 * (opA.astype(np.float64) @ opB) + 0.5 * C0[:, :N]
    check("C", dev.get(Ct)[c_off:].reshape(M, N + 3), ref, rtol=2e-6, atol=1e-5)


def test_sgemm_strided_batched(dev):
    batch, M, N, K = 5, 16, 24, 40
    A, Bm = rnd(batch, M, K), rnd(batch, N, K)
    Ct = dev.empty((batch, M, N))
    dev.rt.lib.sgemm_strided_batched_cuda(0, 1, M, N, K, 1.0, dev(A), K, M * K, dev(Bm), K, N * K, 0.0, Ct, N, M * N,
                                          batch)
    check("C", dev.get(Ct), np.einsum("bmk,bnk->bmn", A.astype(np.float64), Bm), rtol=2e-6)
