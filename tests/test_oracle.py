"""Pins the CPU oracle (oracle/attention_oracle.c) before it is trusted.

gpt.c's own tests hold no expected attention outputs (its tests/ only print
values), so the oracle is pinned by:
  * an fp64 brute force (oracle_attention_fp64, per-row loops in double),
    itself pinned by finite differences and by an independent numpy fp64
    formulation;
  * closed forms: T = 1, q = 0 (uniform prefix average), one dominant key
    (copy of its value), scaling V;
  * invariants: rows of P sum to 1 with P[i, j] = 0 for j > i, causality,
    head-permutation equivariance, (b, h) independence;
  * planted mistakes: a dropped scale, a transposed product or a flipped
    mask in a variant of the fp64 reference fail these checks.
"""
import numpy as np
import pytest

RNG = np.random.default_rng(20240415)


def rand_qkv(B, T, C, scale=1.0):
    return (RNG.standard_normal((B, T, 3 * C)) * scale).astype(np.float32)


def np_attention_fp64(x, H, dy=None, scale_override=None, transpose_bug=False, mask_bug=False):
    """Independent fp64 formulation with whole-matrix numpy ops (einsum)."""
    x = x.astype(np.float64)
    B, T, C3 = x.shape
    C = C3 // 3
    D = C // H
    q, k, v = (x[..., i * C:(i + 1) * C].reshape(B, T, H, D).transpose(0, 2, 1, 3) for i in range(3))
    scale = 1.0 / np.sqrt(D) if scale_override is None else scale_override
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if transpose_bug:
        s = s.transpose(0, 1, 3, 2)
    allowed = np.tril(np.ones((T, T), bool))
    if mask_bug:
        allowed = allowed.T
    s = np.where(allowed, s, -np.inf)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    p /= p.sum(-1, keepdims=True)
    y = np.einsum("bhij,bhjd->bhid", p, v)
    lse = (m + np.log(np.exp(s - m).sum(-1, keepdims=True)))[..., 0]
    out = y.transpose(0, 2, 1, 3).reshape(B, T, C)
    if dy is None:
        return out, lse, None, p
    g = dy.astype(np.float64).reshape(B, T, H, D).transpose(0, 2, 1, 3)
    dv = np.einsum("bhij,bhid->bhjd", p, g)
    dp = np.einsum("bhid,bhjd->bhij", g, v)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq = np.einsum("bhij,bhjd->bhid", ds, k) * scale
    dk = np.einsum("bhij,bhid->bhjd", ds, q) * scale
    dqkv = np.concatenate([t.transpose(0, 2, 1, 3).reshape(B, T, C) for t in (dq, dk, dv)], -1)
    return out, lse, dqkv, p


SHAPES = [  # (B, T, C, H)
    (1, 1, 64, 1),
    (2, 5, 6, 2),      # D = 3, the shape of gpt.c's tests/test_self_attention.c
    (2, 16, 16, 2),    # D = 8
    (1, 33, 128, 2),   # D = 64
    (1, 20, 100, 25),  # D = 4, H = 25 (C5's head count)
    (3, 40, 96, 3),    # D = 32
]


@pytest.mark.parametrize("B,T,C,H", SHAPES)
def test_c_fp64_matches_numpy_fp64(oracle, B, T, C, H):
    x = rand_qkv(B, T, C)
    dy = RNG.standard_normal((B, T, C)).astype(np.float32)
    y, lse, dqkv = oracle.fp64(x, H, dy)
    y2, lse2, dqkv2, _ = np_attention_fp64(x, H, dy)
    np.testing.assert_allclose(y, y2, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, lse2, rtol=0, atol=1e-12)
    np.testing.assert_allclose(dqkv, dqkv2, rtol=0, atol=1e-12)


def test_fp64_gradient_matches_finite_differences(oracle):
    B, T, C, H = 1, 6, 8, 2
    x = rand_qkv(B, T, C)
    dy = RNG.standard_normal((B, T, C)).astype(np.float32)
    _, _, dqkv = oracle.fp64(x, H, dy)
    # L(x) = sum(dy * y(x)); central differences in fp64 through the numpy form.
    eps = 1e-5
    xd = x.astype(np.float64)
    num = np.zeros_like(xd)
    for idx in np.ndindex(xd.shape):
        xp = xd.copy()
        xp[idx] += eps
        xm = xd.copy()
        xm[idx] -= eps
        lp = (np_fwd64(xp, H) * dy).sum()
        lm = (np_fwd64(xm, H) * dy).sum()
        num[idx] = (lp - lm) / (2 * eps)
    np.testing.assert_allclose(dqkv, num, rtol=0, atol=1e-7)


def np_fwd64(x64, H):
    B, T, C3 = x64.shape
    C = C3 // 3
    D = C // H
    q, k, v = (x64[..., i * C:(i + 1) * C].reshape(B, T, H, D).transpose(0, 2, 1, 3) for i in range(3))
    s = np.einsum("bhid,bhjd->bhij", q, k) / np.sqrt(D)
    s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, v).transpose(0, 2, 1, 3).reshape(B, T, C)


@pytest.mark.parametrize("B,T,C,H", SHAPES)
def test_oracle_matches_fp64(oracle, B, T, C, H):
    x = rand_qkv(B, T, C)
    dy = RNG.standard_normal((B, T, C)).astype(np.float32)
    y, q, k, v, att = oracle.forward(x, H)
    dqkv = oracle.backward(dy, H, q, k, v, att)
    y64, lse64, d64 = oracle.fp64(x, H, dy)
    assert np.abs(y - y64).max() < 2e-6
    assert np.abs(dqkv - d64).max() < 1e-5
    # P rebuilt from the fp64 log-sum-exp equals the oracle's cached P.
    D = C // H
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(D)
    p64 = np.where(np.tril(np.ones((T, T), bool)), np.exp(s - lse64[..., None]), 0.0)
    assert np.abs(att - p64).max() < 2e-6


def test_oracle_caches_are_the_permuted_inputs(oracle):
    B, T, C, H = 2, 7, 12, 3
    D = C // H
    x = rand_qkv(B, T, C)
    _, q, k, v, _ = oracle.forward(x, H)
    for i, cache in enumerate((q, k, v)):
        ref = x[..., i * C:(i + 1) * C].reshape(B, T, H, D).transpose(0, 2, 1, 3)
        assert np.array_equal(cache, ref)


def test_closed_form_single_token(oracle):
    B, T, C, H = 3, 1, 64, 4
    x = rand_qkv(B, T, C)
    dy = RNG.standard_normal((B, T, C)).astype(np.float32)
    y, q, k, v, att = oracle.forward(x, H)
    dqkv = oracle.backward(dy, H, q, k, v, att)
    assert np.array_equal(y, x[..., 2 * C:])
    assert np.all(dqkv[..., :2 * C] == 0)
    assert np.array_equal(dqkv[..., 2 * C:], dy)


def test_closed_form_zero_queries_average_prefix(oracle):
    B, T, C, H = 2, 9, 16, 2
    x = rand_qkv(B, T, C)
    x[..., :C] = 0.0
    y, *_ = oracle.forward(x, H)
    v = x[..., 2 * C:].astype(np.float64)
    prefix_mean = np.cumsum(v, axis=1) / np.arange(1, T + 1)[None, :, None]
    np.testing.assert_allclose(y, prefix_mean, rtol=0, atol=2e-6)


def test_closed_form_dominant_key_is_copied(oracle):
    B, T, C, H = 1, 6, 8, 1
    x = rand_qkv(B, T, C, scale=0.01)
    x[0, :, :C] = 1.0          # every query the same
    x[0, 2, C:2 * C] = 40.0    # key 2 dominates every row that can see it
    y, *_ = oracle.forward(x, H)
    np.testing.assert_allclose(y[0, 2:], np.broadcast_to(x[0, 2, 2 * C:], (T - 2, C)), rtol=0, atol=1e-5)


def test_value_scaling_is_linear(oracle):
    B, T, C, H = 2, 11, 24, 3
    x = rand_qkv(B, T, C)
    y, *_ = oracle.forward(x, H)
    x2 = x.copy()
    x2[..., 2 * C:] *= 4.0     # power of two: exact in fp32
    y2, *_ = oracle.forward(x2, H)
    assert np.array_equal(y2, 4.0 * y)


def test_probabilities_are_causal_rows_summing_to_one(oracle):
    B, T, C, H = 2, 17, 32, 4
    _, _, _, _, att = oracle.forward(rand_qkv(B, T, C), H)
    assert np.all(att[..., np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0)
    np.testing.assert_allclose(att.sum(-1), 1.0, rtol=0, atol=1e-6)


def test_causality_future_tokens_do_not_matter(oracle):
    B, T, C, H = 1, 12, 16, 2
    x = rand_qkv(B, T, C)
    dy = RNG.standard_normal((B, T, C)).astype(np.float32)
    y, q, k, v, att = oracle.forward(x, H)
    d = oracle.backward(dy, H, q, k, v, att)
    x2 = x.copy()
    x2[:, 8:] = rand_qkv(B, T - 8, C)
    y2, q2, k2, v2, att2 = oracle.forward(x2, H)
    d2 = oracle.backward(dy, H, q2, k2, v2, att2)
    assert np.array_equal(y[:, :8], y2[:, :8])
    assert np.array_equal(d[:, :8, :C], d2[:, :8, :C])  # dq of early rows


def test_head_permutation_equivariance(oracle):
    B, T, C, H = 1, 10, 24, 3
    D = C // H
    x = rand_qkv(B, T, C)
    perm = [2, 0, 1]
    cols = np.concatenate([np.arange(p * D, (p + 1) * D) for p in perm])
    xp = np.concatenate([x[..., i * C:(i + 1) * C][..., cols] for i in range(3)], -1)
    y, *_ = oracle.forward(x, H)
    yp, *_ = oracle.forward(xp, H)
    assert np.array_equal(yp, y[..., cols])


@pytest.mark.parametrize("bug", ["scale", "transpose", "mask"])
def test_planted_mistakes_are_caught(oracle, bug):
    """A plausible mistake in a reference implementation fails the pins above."""
    B, T, C, H = 1, 9, 16, 2
    x = rand_qkv(B, T, C)
    kw = {"scale": dict(scale_override=1.0), "transpose": dict(transpose_bug=True), "mask": dict(mask_bug=True)}[bug]
    bad, *_ = np_attention_fp64(x, H, **kw)
    ref, *_ = oracle.fp64(x, H)
    assert np.abs(bad - ref).max() > 1e-3
