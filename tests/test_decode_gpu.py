"""GPU parity of the KV-cache decode step (attention_decode_cuda_kernel).

gpt.c generates text by running the whole window through attention for every
new token and keeping one row (infer_gpt.c:339-351).  The decode step returns
that row from the K/V caches.  Each case checks, on the same seeded inputs:
- the decode output of every position against the oracle's forward over the
  tokens up to it (the C restatement of gpt.c's CPU path), max abs err <= 1e-4;
- the same rows against this library's full forward (which is itself
  checked against the oracle in test_attention_gpu.py);
- that the caches hold exactly the permuted k and v that gpt.c's forward
  caches (attention.c:105-120), bit for bit.
"""
import numpy as np
import pytest

import gptc

pytestmark = pytest.mark.gpu

TOL = 1e-4


def check(name, got, ref, tol=TOL):
    err = float(np.abs(got.astype(np.float64) - ref).max()) if got.size else 0.0
    print(f"  {name}: max abs err {err:.3e}")
    assert np.isfinite(got).all(), name
    assert err <= tol, f"{name}: max abs err {err:.3e} > {tol}"
    return err


def full_forward(rt, x, H):
    """y of this library's forward over the whole (B, T, 3C) input."""
    B, T, C3 = x.shape
    layer = gptc.AttentionLayer(rt, C3 // 3, H, T)
    layer.to(gptc.CUDA)
    yt = layer.forward(rt.from_numpy(x))
    y = rt.to_numpy(yt)
    rt.free(yt)
    layer.free()
    return y


def decode_all(rt, x, H, L=None):
    """Decode positions 0 .. T-1 one at a time from empty caches of length L."""
    B, T, C3 = x.shape
    C = C3 // 3
    D = C // H
    L = L or T
    kc, vc = rt.empty((B, H, L, D)), rt.empty((B, H, L, D))
    out = rt.empty((B, 1, C))
    ys = np.empty((B, T, C), np.float32)
    for pos in range(T):
        row = rt.from_numpy(x[:, pos:pos + 1, :])
        rt.lib.attention_decode_cuda_kernel(row, kc, vc, pos, H, out)
        ys[:, pos, :] = rt.to_numpy(out)[:, 0, :]
        rt.free(row)
    k_cache, v_cache = rt.to_numpy(kc)[:, :, :T], rt.to_numpy(vc)[:, :, :T]
    for t in (kc, vc, out):
        rt.free(t)
    return ys, k_cache, v_cache


@pytest.mark.parametrize("B,T,C,H,L", [
    (1, 1, 64, 1, 1),        # one key: y = v
    (2, 37, 128, 2, 40),     # cache longer than the sequence
    (1, 300, 768, 12, 300),  # GPT-2 small heads: the one-launch kernel (pos + 1 <= 512)
    (1, 600, 768, 12, 640),  # past 512 keys: the split-key pair from position 512 on
    (3, 520, 256, 4, 520),   # B = 3, both kernels
    (2, 70, 96, 4, 70),      # D = 24 (plain loads)
    (2, 9, 6, 2, 16),        # D = 3 (gpt.c's tests/test_self_attention.c shape class)
    (1, 64, 100, 25, 64),    # H = 25, D = 4
    (2, 33, 192, 2, 40),     # D = 96
    (1, 40, 256, 2, 48),     # D = 128
    (1, 30, 600, 2, 32),     # D = 300 (the generic head-size build)
    (2, 20, 1024, 1, 24),    # D = 1024
])
def test_decode_every_position(rt, oracle, B, T, C, H, L):
    x = rt.normal((B, T, 3 * C), 1337)
    ys, k_cache, v_cache = decode_all(rt, x, H, L)
    y_ref, q, k, v, _ = oracle.forward(x, H)
    print(f"case B={B} T={T} C={C} H={H} D={C // H} L={L}")
    check("decode vs oracle", ys, y_ref)
    check("decode vs forward", ys, full_forward(rt, x, H))
    assert np.array_equal(k_cache, k), "k cache"
    assert np.array_equal(v_cache, v), "v cache"


def test_decode_c4_window_positions(rt, oracle):
    """C4 (B=1, GPT-2 small heads): caches filled with the window's k, v, then the
    decode of single positions up to gpt.c's block size, against the oracle's
    forward over the full 1024-token window (the row gpt.c's infer_gpt.c keeps)."""
    B, T, C, H = 1, 1024, 768, 12
    D = C // H
    x = rt.normal((B, T, 3 * C), 42)
    y_ref, q, k, v, _ = oracle.forward(x, H)
    out = rt.empty((B, 1, C))
    for pos in (0, 63, 64, 255, 511, 512, 1000, 1023):
        kc = rt.from_numpy(np.where(np.arange(T)[None, None, :, None] < pos, k, 0.0))
        vc = rt.from_numpy(np.where(np.arange(T)[None, None, :, None] < pos, v, 0.0))
        row = rt.from_numpy(x[:, pos:pos + 1, :])
        rt.lib.attention_decode_cuda_kernel(row, kc, vc, pos, H, out)
        check(f"pos {pos}", rt.to_numpy(out)[:, 0, :], y_ref[:, pos, :])
        assert np.array_equal(rt.to_numpy(kc)[:, :, pos], k[:, :, pos])
        assert np.array_equal(rt.to_numpy(vc)[:, :, pos], v[:, :, pos])
        for t in (kc, vc, row):
            rt.free(t)
    rt.free(out)


def test_decode_dominant_key_and_uniform_closed_forms(rt):
    """Closed forms: q = 0 gives the mean of v over keys 0..pos; one key with a
    huge score gives that key's v."""
    B, T, C, H = 1, 50, 64, 1
    rng = np.random.default_rng(0)
    x = rng.standard_normal((B, T, 3 * C)).astype(np.float32)
    x[:, :, :C] = 0.0  # q = 0: uniform attention
    ys, _, _ = decode_all(rt, x, H)
    v = x[0, :, 2 * C:].astype(np.float64)
    check("uniform", ys[0], np.cumsum(v, 0) / np.arange(1, T + 1)[:, None], 1e-5)
    x2 = x.copy()
    x2[:, :, :C] = 1.0
    x2[:, :, C:2 * C] = 0.0
    x2[:, 20, C:2 * C] = 100.0  # key 20 dominates every query from 20 on
    ys2, _, _ = decode_all(rt, x2, H)
    check("dominant", ys2[0, 20:], np.broadcast_to(x2[0, 20, 2 * C:], (T - 20, C)), 1e-5)
