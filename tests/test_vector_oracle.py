"""Pins the oracle's vector-level ops, single-row attention and rmsnormInto
(oracle/vector_oracle.c) before they serve as the parity reference.

Checks that do not share the oracle's code: fp64 closed forms in numpy,
fp64 central differences, algebraic identities (a rotation's transpose is
its inverse, softmax rows sum to one, RoPE scores depend only on the
position difference), the reference's own procedures (attention.js I-50..I-52
from verify.js:378-406 and l3-l5.test.js:174-200), and known answers where
the reference's fp32 running sum differs from an exact sum.
"""
import numpy as np
import pytest

import oracle


def f32(rs, n, s=1.0):
    return (rs.standard_normal(n) * s).astype(np.float32)


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(a - b))) if a.size else 0


# ── mul / scale / dot: products of fp32 values are exact in fp64 ───────────
def test_mul_scale_dot_closed_forms():
    rs = np.random.default_rng(1)
    a, b, g = f32(rs, 257), f32(rs, 257), f32(rs, 257)
    assert np.array_equal(oracle.vec_mul_fwd(a, b), (a.astype(np.float64) * b).astype(np.float32))
    assert np.array_equal(oracle.vec_mul_fwd(a, b[:1]), (a.astype(np.float64) * b[0]).astype(np.float32))
    ga, gb = oracle.vec_mul_bwd(g, a, b)
    assert np.array_equal(ga, (g.astype(np.float64) * b).astype(np.float32))
    assert np.array_equal(gb, (g.astype(np.float64) * a).astype(np.float32))
    assert np.array_equal(oracle.vec_scale_fwd(a, 0.3), (0.3 * a.astype(np.float64)).astype(np.float32))
    gx0 = f32(rs, 257)
    assert np.array_equal(oracle.vec_scale_bwd(g, -1.7, gx=gx0),
                          (gx0.astype(np.float64) + g.astype(np.float64) * -1.7).astype(np.float32))
    d = oracle.vec_dot_fwd(a, b)
    assert abs(float(d) - float(np.dot(a.astype(np.float64), b))) <= 1e-6 * np.sum(np.abs(a * b))
    ga, gb = oracle.vec_dot_bwd(np.float32(0.7), a, b)
    assert np.array_equal(ga, (np.float64(np.float32(0.7)) * b.astype(np.float64)).astype(np.float32))
    assert np.array_equal(gb, (np.float64(np.float32(0.7)) * a.astype(np.float64)).astype(np.float32))


def test_mul_scalar_gradient_is_an_fp32_running_sum():
    # gb[0] += g[i]*a[i] into a Float32Array (autograd.js:77): 1e8 + 1 is
    # 1e8 in fp32, so the running sum ends at 0, not at the exact 1.
    a = np.array([1e8, 1.0, -1e8], np.float32)
    g = np.ones(3, np.float32)
    _, gb = oracle.vec_mul_bwd(g, a, np.array([2.0], np.float32))
    assert gb[0] == 0.0
    ga, _ = oracle.vec_mul_bwd(g, a, np.array([2.0], np.float32))
    assert np.array_equal(ga, np.full(3, 2.0, np.float32))
    # dot's sum is fp64 (a JS number): the same inputs give the exact 1
    assert oracle.vec_dot_fwd(a, g) == 1.0


def test_accumulating_gradients_add_in_fp64_then_round():
    rs = np.random.default_rng(2)
    a, b, g, ga0 = f32(rs, 64), f32(rs, 64), f32(rs, 64), f32(rs, 64)
    ga, _ = oracle.vec_mul_bwd(g, a, b, ga=ga0)
    assert np.array_equal(ga, (ga0.astype(np.float64) + g.astype(np.float64) * b).astype(np.float32))


# ── silu ────────────────────────────────────────────────────────────────
def test_silu_closed_form_and_central_differences():
    rs = np.random.default_rng(3)
    x = f32(rs, 300, 3.0)
    y, s = oracle.vec_silu_fwd(x)
    x64 = x.astype(np.float64)
    s64 = 1.0 / (1.0 + np.exp(-x64))
    assert ulps(s, s64.astype(np.float32)) <= 1
    assert ulps(y, (x64 * s.astype(np.float64)).astype(np.float32)) == 0
    g = f32(rs, 300)
    gx = oracle.vec_silu_bwd(g, x, s)
    h = 1e-6
    num = ((x64 + h) / (1 + np.exp(-(x64 + h))) - (x64 - h) / (1 + np.exp(-(x64 - h)))) / (2 * h)
    ref = g.astype(np.float64) * num
    assert np.max(np.abs(gx - ref)) <= 2e-6 * max(1.0, np.max(np.abs(ref)))


# ── ropeNode ──────────────────────────────────────────────────────────────
def rope_tables(dH, pos, theta=10000.0):
    half = (dH + 1) // 2
    ang = pos * theta ** (-(2 * np.arange(half)) / dH)
    return np.cos(ang), np.sin(ang)


@pytest.mark.parametrize("n,dH", [(16, 16), (20, 16), (9, 7), (8, 0)])
def test_rope_rotation_and_transpose(n, dH):
    rs = np.random.default_rng(4)
    x = f32(rs, n)
    c, s = rope_tables(dH, 5.0)
    y = oracle.vec_rope_fwd(x, c, s, dH)
    npair = 2 * ((dH + 1) // 2)
    assert np.all(y[npair:] == 0)
    xp = x[:npair].astype(np.float64).reshape(-1, 2)
    yp = y[:npair].astype(np.float64).reshape(-1, 2)
    # a rotation keeps each pair's length; the first component is a c - b s
    assert np.allclose(np.hypot(yp[:, 0], yp[:, 1]), np.hypot(xp[:, 0], xp[:, 1]), rtol=1e-6, atol=1e-7)
    assert np.allclose(yp[:, 0], xp[:, 0] * c - xp[:, 1] * s, rtol=1e-6, atol=1e-7)
    # the backward is R^T: backward(forward(x)) == x on the pairs
    back = oracle.vec_rope_bwd(y, c, s, dH)
    assert np.allclose(back[:npair], x[:npair], rtol=1e-5, atol=1e-6)
    assert np.all(back[npair:] == 0)


def test_rope_scores_depend_on_position_difference():
    # RoPE relativity (attention.js I-53): (R_m q)·(R_n k) depends on m - n only
    rs = np.random.default_rng(5)
    q, k = f32(rs, 32), f32(rs, 32)

    def score(m, n):
        cq, sq = rope_tables(32, float(m))
        ck, sk = rope_tables(32, float(n))
        return float(np.dot(oracle.vec_rope_fwd(q, cq, sq, 32).astype(np.float64),
                            oracle.vec_rope_fwd(k, ck, sk, 32).astype(np.float64)))

    assert abs(score(7, 3) - score(12, 8)) < 1e-4
    assert abs(score(7, 3) - score(3, 7)) > 1e-3


# ── softmaxVec ───────────────────────────────────────────────────────────
def test_softmax_closed_form_and_jacobian():
    rs = np.random.default_rng(6)
    x = f32(rs, 200, 2.0)
    out, p = oracle.vec_softmax_fwd(x)
    assert np.array_equal(out, p)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max())
    assert np.max(np.abs(p - e / e.sum())) < 1e-7
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-5
    g = f32(rs, 200)
    gx = oracle.vec_softmax_bwd(g, p)
    p64, g64 = p.astype(np.float64), g.astype(np.float64)
    ref = p64 * (g64 - np.dot(g64, p64))
    assert np.max(np.abs(gx - ref)) < 1e-7
    # central differences of L = g · softmax(x)
    h = 1e-5
    num = np.empty(8)
    for i in range(8):
        xp, xm = x64.copy(), x64.copy()
        xp[i] += h
        xm[i] -= h
        sp = np.exp(xp - xp.max()); sp /= sp.sum()
        sm = np.exp(xm - xm.max()); sm /= sm.sum()
        num[i] = (np.dot(g64, sp) - np.dot(g64, sm)) / (2 * h)
    assert np.max(np.abs(gx[:8] - num)) < 1e-6


# ── single-row attention ─────────────────────────────────────────────────────
def attn64(q, K, V, n, d, scale, causal, qOff):
    s = (K.reshape(n, d).astype(np.float64) @ q.astype(np.float64)) * scale
    if causal:
        s[np.arange(n) > qOff] = -np.inf
    w = np.exp(s - s.max())
    w /= w.sum()
    return w @ V.reshape(n, d).astype(np.float64)


@pytest.mark.parametrize("n,d,causal,qOff", [(64, 16, True, 63), (40, 24, True, 17), (33, 8, False, 0),
                                             (130, 64, True, 129), (1, 4, True, 0)])
def test_row_attention_variants_vs_closed_form(n, d, causal, qOff):
    rs = np.random.default_rng(7)
    q, K, V = f32(rs, d), f32(rs, n * d), f32(rs, n * d)
    scale = 1 / np.sqrt(d)
    ref = attn64(q, K, V, n, d, scale, causal, qOff)
    od, sc = oracle.attention_decode(q, K, V, n, d, scale, causal, qOff)
    on = oracle.attention_naive(q, K, V, n, d, scale, causal, qOff)
    of = oracle.flash_attention(q, K, V, n, d, scale, causal, qOff, 16)
    for o in (od, on, of):
        assert np.max(np.abs(o - ref)) < 2e-6 * max(1.0, np.max(np.abs(ref)))
    # the decode variant leaves the fp32 scores, -inf where masked
    s64 = (K.reshape(n, d).astype(np.float64) @ q.astype(np.float64)) * scale
    live = ~(causal & (np.arange(n) > qOff))
    assert np.array_equal(sc[live], s64[live].astype(np.float32))
    assert np.all(np.isneginf(sc[~live]))


def test_row_attention_reference_procedures():
    # I-50 (verify.js:385-387, l3-l5.test.js:174-185): flash == naive;
    # l3-l5.test.js:187-200: keys after qOff take no part.
    rs = np.random.default_rng(8)
    n, d = 64, 16
    q, K, V = f32(rs, d), f32(rs, n * d), f32(rs, n * d)
    sc = 1 / np.sqrt(d)
    assert np.max(np.abs(oracle.flash_attention(q, K, V, n, d, sc, True, n - 1)
                         - oracle.attention_naive(q, K, V, n, d, sc, True, n - 1))) < 1e-5
    pos = 5
    o = oracle.flash_attention(q, K, V, n, d, sc, True, pos)
    o_ref = oracle.attention_naive(q, K[:(pos + 1) * d], V[:(pos + 1) * d], pos + 1, d, sc, True, pos)
    assert np.max(np.abs(o - o_ref)) < 1e-6
    # everything masked: the decode and flash rows are zero (attention.js:52-55, :91)
    assert np.all(oracle.attention_decode(q, K, V, n, d, sc, True, -1)[0] == 0)
    assert np.all(oracle.flash_attention(q, K, V, n, d, sc, True, -1) == 0)


# ── rmsnormInto ──────────────────────────────────────────────────────────
def test_row_rmsnorm_closed_form():
    rs = np.random.default_rng(9)
    x, w = f32(rs, 777, 2.0), f32(rs, 777)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
    out = oracle.row_rmsnorm(x, w, 1e-5)
    assert np.max(np.abs(out - ref)) <= 2e-7 * np.max(np.abs(ref))
