"""Pins the CPU oracle of the non-attention layers (oracle/ops_oracle.c) and
the GPT-2 step composed from it (oracle/gpt2_oracle.py), before they are
trusted as the checker of the GPU back end.

gpt.c's tests hold no expected values for these layers (tests/ only prints
them), so the pins are:
  * gpt.c's own CPU kernels (kernels/src/cpu/{LayerNorm,GeLU,Softmax,
    Embedding,CrossEntropyLoss,AdamW}.c compiled unmodified under
    oracle/_ref): the restatement must agree to float rounding;
  * torch float64 autograd of the same mathematics (an independent
    formulation: its gradients come from autodiff, not from the backward
    formulas restated here), and torch.optim.AdamW for the optimizer;
  * Linear (whose gpt.c kernel needs <cblas.h>, absent here) against numpy
    float64 products;
  * planted mistakes (a dropped term, a transposed operand) in copies of the
    inputs fail these checks.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle as oracle_mod
from gpt2_oracle import GPT2Oracle, param_shapes

RNG = np.random.default_rng(7)
F64 = torch.float64


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


@pytest.fixture(scope="module")
def ops(oracle):
    return oracle_mod.Ops(oracle)


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(oracle_mod.REF_OPS_PATH):
        pytest.skip("oracle/_ref not built (needs /root/reference): make -C oracle ref")
    return oracle_mod.RefOps()


def t64(a, grad=False):
    return torch.tensor(np.asarray(a, dtype=np.float64), dtype=F64, requires_grad=grad)


def maxerr(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


# ---------------------------------------------------------------- vs gpt.c's own kernels

def test_layer_norm_matches_gpt_c_kernel(ops, ref):
    B, T, C = 3, 5, 48
    x, W, b, g = rnd(B, T, C), rnd(C), rnd(C), rnd(B, T, C)
    y, mean, rstd = ops.layer_norm_forward(x, W, b)
    outs = ref.call("layer_norm_forward_cpu_kernel", W, b, x, ctypes.c_float(1e-5),
                    [np.empty((B, T), np.float32), np.empty((B, T), np.float32)], np.empty_like(x))
    assert maxerr(y, outs[5]) <= 1e-6 and maxerr(mean, outs[4][0]) <= 1e-6 and maxerr(rstd, outs[4][1]) <= 1e-6
    dW, db, dx = np.zeros(C, np.float32), np.zeros(C, np.float32), np.zeros_like(x)
    ops.layer_norm_backward(g, x, mean, rstd, W, dW, db, dx)
    r = ref.call("layer_norm_backward_cpu_kernel", g, [mean, rstd, x], W, np.zeros(C, np.float32),
                 np.zeros(C, np.float32), np.zeros_like(x))
    assert maxerr(dW, r[3]) <= 1e-5 and maxerr(db, r[4]) <= 1e-5 and maxerr(dx, r[5]) <= 1e-5


def test_gelu_softmax_match_gpt_c_kernels(ops, ref):
    x, g = rnd(4, 6, 33, scale=3.0), rnd(4, 6, 33)
    assert maxerr(ops.gelu_forward(x), ref.call("gelu_forward_cpu_kernel", x, np.empty_like(x))[1]) <= 1e-6
    assert maxerr(ops.gelu_backward(g, x),
                  ref.call("gelu_backward_cpu_kernel", g, x, np.empty_like(x))[2]) <= 1e-6
    p = ops.softmax_forward(x)
    assert maxerr(p, ref.call("softmax_forward_cpu_kernel", x, np.empty_like(x))[1]) <= 1e-7
    assert maxerr(ops.softmax_backward(g, p),
                  ref.call("softmax_backward_cpu_kernel", g, p, np.empty_like(x))[2]) <= 1e-7


def test_embedding_matches_gpt_c_kernel(ops, ref):
    V, C, B, T = 11, 8, 3, 7
    W = rnd(V, C)
    ids = RNG.integers(0, V, (B, T)).astype(np.float32)
    y = ops.embedding_forward(W, ids)
    assert np.array_equal(y, ref.call("embedding_forward_cpu_kernel", W, ids, np.empty((B, T, C), np.float32))[2])
    g = rnd(B, T, C)
    for cache in (ids, np.arange(T, dtype=np.float32)[None, :]):  # token ids, and wpe's shared arange
        dW = np.zeros((V, C), np.float32)
        ops.embedding_backward(g, cache, dW)
        r = ref.call("embedding_backward_cpu_kernel", g, cache, np.zeros((V, C), np.float32))[2]
        assert np.array_equal(dW, r)


def test_cross_entropy_matches_gpt_c_kernel(ops, ref):
    B, T, V = 2, 5, 37
    logits = rnd(B, T, V, scale=2.0)
    tg = RNG.integers(0, V, (B, T)).astype(np.float32)
    lsm, loss = ops.cross_entropy_forward(logits, tg)
    r = ref.call("cross_entropy_forward_cpu_kernel", logits, tg, [np.empty_like(logits)], np.zeros(1, np.float32))
    assert maxerr(lsm, r[2][0]) <= 1e-6 and abs(loss - float(r[3][0])) <= 1e-6
    g = np.ones((B, T), np.float32)
    d = ops.cross_entropy_backward(g, lsm, tg)
    rd = ref.call("cross_entropy_backward_cpu_kernel", g, [lsm, tg], np.zeros_like(lsm))[2]
    assert maxerr(d, rd) <= 1e-7


def test_adamw_matches_gpt_c_kernel(ops, ref):
    n = 1000
    p, g = rnd(n), rnd(n)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    p1, m1, v1 = p.copy(), m.copy(), v.copy()
    rp, rm, rv = p.copy(), m.copy(), v.copy()
    for step in (1, 2, 3):
        ops.adamw(p1, g, m1, v1, 1e-3, 0.9, 0.99, 0.1, 1e-8, step)
        ref.call("step_adamW_cpu_kernel", [rp], [g], [rm], [rv], ctypes.c_int(1), ctypes.c_float(1e-3),
                 ctypes.c_float(0.9), ctypes.c_float(0.99), ctypes.c_float(0.1), ctypes.c_float(1e-8),
                 ctypes.c_int(step))
    assert maxerr(p1, rp) <= 1e-7 and maxerr(m1, rm) <= 1e-7 and maxerr(v1, rv) <= 1e-7


# ---------------------------------------------------------------- vs torch float64 autograd

def test_linear_vs_fp64(ops):
    x, W, b, g = rnd(2, 9, 24), rnd(40, 24), rnd(40), rnd(2, 9, 40)
    y = ops.linear_forward(W, b, x)
    assert maxerr(y, x.astype(np.float64) @ W.T.astype(np.float64) + b) <= 1e-5
    dW0, db0 = rnd(40, 24), rnd(40)
    dW, db = dW0.copy(), db0.copy()
    dx = ops.linear_backward(g, x, W, dW, db)
    g2, x2 = g.reshape(-1, 40).astype(np.float64), x.reshape(-1, 24).astype(np.float64)
    assert maxerr(dx.reshape(-1, 24), g2 @ W.astype(np.float64)) <= 1e-5
    assert maxerr(dW, dW0 + g2.T @ x2) <= 1e-5  # accumulates
    assert maxerr(db, db0 + g2.sum(0)) <= 1e-5
    # planted: a transposed weight product is far off
    assert maxerr(dW, dW0 + (g2.T @ x2)[::-1]) > 1e-2


def test_layer_norm_gelu_softmax_ce_vs_torch_fp64(ops):
    B, T, C = 2, 4, 20
    x, W, b, g = rnd(B, T, C), rnd(C), rnd(C), rnd(B, T, C)
    xt, Wt, bt = t64(x, True), t64(W, True), t64(b, True)
    yt = torch.nn.functional.layer_norm(xt, (C,), Wt, bt, eps=1e-5)
    yt.backward(t64(g))
    y, mean, rstd = ops.layer_norm_forward(x, W, b)
    dW, db, dx = np.zeros(C, np.float32), np.zeros(C, np.float32), np.zeros_like(x)
    ops.layer_norm_backward(g, x, mean, rstd, W, dW, db, dx)
    assert maxerr(y, yt.detach()) <= 1e-5
    assert maxerr(dx, xt.grad) <= 1e-5 and maxerr(dW, Wt.grad) <= 1e-5 and maxerr(db, bt.grad) <= 1e-5

    xg = t64(x * 3, True)
    yg = torch.nn.functional.gelu(xg, approximate="tanh")
    yg.backward(t64(g))
    assert maxerr(ops.gelu_forward(x * 3), yg.detach()) <= 1e-5
    assert maxerr(ops.gelu_backward(g, x * 3), xg.grad) <= 1e-5

    xs = t64(x, True)
    ps = torch.softmax(xs, -1)
    ps.backward(t64(g))
    p = ops.softmax_forward(x)
    assert maxerr(p, ps.detach()) <= 1e-6 and maxerr(ops.softmax_backward(g, p), xs.grad) <= 1e-6

    V = 29
    logits, tg = rnd(B, T, V, scale=2.0), RNG.integers(0, V, (B, T))
    lt = t64(logits, True)
    loss_t = torch.nn.functional.cross_entropy(lt.reshape(-1, V), torch.tensor(tg.reshape(-1)))
    loss_t.backward()
    lsm, loss = ops.cross_entropy_forward(logits, tg.astype(np.float32))
    assert abs(loss - loss_t.item()) <= 1e-5
    d = ops.cross_entropy_backward(np.ones((B, T), np.float32), lsm, tg.astype(np.float32))
    assert maxerr(d, lt.grad) <= 1e-6
    # closed form: uniform logits give loss = ln V
    _, l0 = ops.cross_entropy_forward(np.zeros((1, 3, V), np.float32), np.zeros((1, 3), np.float32))
    assert abs(l0 - np.log(V)) <= 1e-6


def test_adamw_vs_torch_optim():
    o = oracle_mod.Ops(oracle_mod.Oracle())
    p0, grads = rnd(300), [rnd(300) for _ in range(3)]
    pt = t64(p0, True)
    opt = torch.optim.AdamW([pt], lr=1e-2, betas=(0.9, 0.99), eps=1e-8, weight_decay=0.1)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for step, g in enumerate(grads, 1):
        pt.grad = t64(g)
        opt.step()
        o.adamw(p, g, m, v, 1e-2, 0.9, 0.99, 0.1, 1e-8, step)
    assert maxerr(p, pt.detach()) <= 1e-6


# ---------------------------------------------------------------- the composed GPT-2 step

def torch_gpt2_step(params, ids, targets, L, H, lr=3e-4, beta1=0.9, beta2=0.99, wd=0.0, eps=1e-8):
    """float64 GPT-2 (pre-LN, tanh GELU, tied lm_head) with autograd and
    torch.optim.AdamW: (loss, logits, grads, updated params)."""
    P = [t64(a, True) for a in params]
    wte, wpe = P[0], P[1]
    B, T = ids.shape
    C = wte.shape[1]
    D = C // H
    x = wte[torch.tensor(ids)] + wpe[:T][None]
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    for i in range(L):
        (l1w, l1b, qw, qb, pw, pb, l2w, l2b, fw, fb, mw, mb) = P[2 + 12 * i: 14 + 12 * i]
        h = torch.nn.functional.layer_norm(x, (C,), l1w, l1b, 1e-5)
        qkv = h @ qw.T + qb
        q, k, v = (qkv[..., j * C:(j + 1) * C].reshape(B, T, H, D).transpose(1, 2) for j in range(3))
        s = (q @ k.transpose(-1, -2)) / np.sqrt(D)
        s = s.masked_fill(~causal, float("-inf"))
        a = (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, T, C)
        x = x + a @ pw.T + pb
        h2 = torch.nn.functional.layer_norm(x, (C,), l2w, l2b, 1e-5)
        f = torch.nn.functional.gelu(h2 @ fw.T + fb, approximate="tanh")
        x = x + f @ mw.T + mb
    x = torch.nn.functional.layer_norm(x, (C,), P[-2], P[-1], 1e-5)
    logits = x @ wte.T
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.shape[-1]), torch.tensor(targets.reshape(-1)))
    loss.backward()
    grads = [p.grad.detach().numpy().copy() for p in P]
    opt = torch.optim.AdamW(P, lr=lr, betas=(beta1, beta2), eps=eps, weight_decay=wd)
    opt.step()
    return loss.item(), logits.detach().numpy(), grads, [p.detach().numpy() for p in P]


def tiny_params(V, block, L, C, seed=3):
    rng = np.random.default_rng(seed)
    out = []
    for name, shp in param_shapes(V, block, L, C):
        if name.endswith("ln1.W") or name.endswith("ln2.W") or name == "ln_f.W":
            out.append((1.0 + 0.1 * rng.standard_normal(shp)).astype(np.float32))
        else:
            out.append((0.2 * rng.standard_normal(shp)).astype(np.float32))
    return out


def test_gpt2_step_oracle_vs_torch_fp64(oracle):
    V, block, L, H, C, B, T = 53, 12, 2, 2, 16, 2, 9
    params = tiny_params(V, block, L, C)
    ids = RNG.integers(0, V, (B, T))
    tg = RNG.integers(0, V, (B, T))
    loss_t, logits_t, grads_t, new_t = torch_gpt2_step(params, ids, tg, L, H, lr=1e-2, wd=0.1)
    g = GPT2Oracle(oracle, params, L, H)
    logits = g.forward(ids)
    loss = g.loss(logits, tg)
    grads = g.backward()
    g.step(lr=1e-2, weight_decay=0.1)
    assert abs(loss - loss_t) <= 1e-5
    assert maxerr(logits, logits_t) <= 1e-5
    names = [n for n, _ in param_shapes(V, block, L, C)]
    for n, a, b in zip(names, grads, grads_t):
        assert maxerr(a, b) <= 1e-5, n
    # AdamW normalises each gradient entry, so entries whose exact gradient is
    # zero (the key bias: softmax ignores a per-row shift) move by up to lr
    # in either direction on float rounding noise.  Compare the update where
    # the gradient is well above rounding noise, bound it elsewhere.
    for n, a, b, p0, gt in zip(names, g.p, new_t, params, grads_t):
        live = np.abs(gt) > 1e-4
        assert maxerr(a[live], b[live]) <= 1e-5, n
        bound = 1e-2 * (1.0 + 0.1 * np.abs(p0[~live])) + 1e-6  # lr (1 + wd |p|)
        assert (np.abs(a[~live].astype(np.float64) - p0[~live]) <= bound).all(), n
