"""Pins the C oracle (oracle/forge_oracle.c) before it is trusted as the parity reference.

Each function is checked against something that does not share its code:
the fp64 closed forms of oracle/np_ref.py, fp64 central differences, the
reference's own known answers (l2-l6.test.js, verify.js), brute force on tiny
inputs, and an independent Python restatement of the RNG.  The checks are
chosen so a plausible slip (dropped term, wrong sign or index, transposed
operand, off-by-one mask) fails at least one of them.
"""
import numpy as np
import pytest

import np_ref
import oracle


def r64(rs, *shape, s=1.0):
    return (rs.standard_normal(shape) * s).astype(np.float32)


# ───────────────────────── RNG (numeric.js:27-49) ─────────────────────────
class PyRNG:
    """Integer restatement of splitmix32 seeding + xorshift128+ in Python."""
    M = 0xFFFFFFFF

    def __init__(self, seed):
        s = (seed & self.M) or 1

        def mix():
            nonlocal s
            s = (s + 0x9E3779B9) & self.M
            z = s
            z = ((z ^ (z >> 16)) * 0x21F0AAAD) & self.M
            z = ((z ^ (z >> 15)) * 0x735A2D97) & self.M
            return (z ^ (z >> 15)) & self.M

        self.s0, self.s1 = mix(), mix()

    def next(self):
        x, y = self.s0, self.s1
        self.s0 = y
        x = (x ^ (x << 23)) & self.M
        x ^= x >> 17
        x ^= y
        x ^= y >> 26
        self.s1 = x & self.M
        return ((self.s1 + y) & self.M) / 4294967296.0


@pytest.mark.parametrize("seed", [0, 1, 7, 12345, 20260101, 0xFFFFFFFF])
def test_rng_matches_integer_restatement(seed):
    a, b = oracle.RNG(seed), PyRNG(seed)
    for _ in range(1000):
        assert a.next() == b.next()


def test_rng_normal_and_int():
    a, b = oracle.RNG(99), PyRNG(99)
    for _ in range(500):
        u = max(b.next(), 1e-12)
        v = b.next()
        want = np.sqrt(-2 * np.log(u)) * np.cos(2 * np.pi * v)
        assert abs(a.normal() - want) <= 4e-16 * max(1.0, abs(want))
    r1, r2 = oracle.RNG(5), PyRNG(5)
    assert all(r1.int(31) == int(np.floor(r2.next() * 31)) for _ in range(200))


# ───────────────────────── matmulT ─────────────────────────
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 5, 4), (7, 9, 3), (33, 64, 17)])
def test_gemm_vs_fp64(M, K, N):
    rs = np.random.default_rng(M * 100 + K)
    X, W = r64(rs, M, K), r64(rs, N, K)
    Y = oracle.matmulT_fwd(X.ravel(), W.ravel(), M, K, N).reshape(M, N)
    ref = X.astype(np.float64) @ W.astype(np.float64).T
    # fp64 accumulation, one rounding: within 1 ulp of the correctly rounded value
    np.testing.assert_array_max_ulp(Y, ref.astype(np.float32), maxulp=1)


def test_gemm_brute_force_triple_loop():
    X = np.arange(6, dtype=np.float32).reshape(2, 3)
    W = np.array([[1, 0, -1], [2, 1, 0.5]], np.float32)
    Y = oracle.matmulT_fwd(X.ravel(), W.ravel(), 2, 3, 2)
    want = [sum(X[m, k] * W[n, k] for k in range(3)) for m in range(2) for n in range(2)]
    assert list(Y) == want


@pytest.mark.parametrize("M,K,N", [(3, 5, 4), (16, 24, 8)])
def test_matmulT_bwd_vs_closed_form(M, K, N):
    rs = np.random.default_rng(11)
    X, W, G = r64(rs, M, K), r64(rs, N, K), r64(rs, M, N)
    gX, gW = oracle.matmulT_bwd(G.ravel(), X.ravel(), W.ravel(), M, K, N)
    rX, rW = np_ref.matmulT_grads(G.astype(np.float64), X.astype(np.float64), W.astype(np.float64))
    np.testing.assert_allclose(gX.reshape(M, K), rX, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gW.reshape(N, K), rW, rtol=1e-5, atol=1e-5)


def test_matmulT_bwd_accumulates_and_skips_zero_rows():
    X = np.ones(4, np.float32)
    W = np.full(4, np.inf, np.float32)
    g = np.zeros(2, np.float32)  # gY == 0 rows are skipped (tensor.js:44): no inf*0 NaN
    gX, gW = oracle.matmulT_bwd(g, X, W, 2, 2, 1, gX=np.ones(4, np.float32))
    assert np.all(gX == 1) and np.all(gW == 0)


def test_matmulT_bwd_split_loops_equal_interleaved_loop():
    """Above its size threshold the oracle runs gX and gW as two blocked,
    threaded loops; each element must still take the reference's sequence of
    fp32 `+=` (tensor.js:44-51), so the result equals the single interleaved
    m, n, k loop bit for bit (zero gY entries included, which both skip)."""
    rs = np.random.default_rng(5)
    M, K, N = 70, 96, 200
    X, W, G = r64(rs, M, K), r64(rs, N, K), r64(rs, M, N)
    G[rs.random((M, N)) < 0.1] = 0.0
    assert M * N * K > (1 << 20)
    gX, gW = oracle.matmulT_bwd(G.ravel(), X.ravel(), W.ravel(), M, K, N)
    sX, sW = oracle.matmulT_bwd_serial(G.ravel(), X.ravel(), W.ravel(), M, K, N)
    np.testing.assert_array_equal(gX, sX)
    np.testing.assert_array_equal(gW, sW)


def test_oracle_results_do_not_depend_on_thread_count():
    """One thread against all of them: model step (GQA, untied head, rows of
    several samples), attention and CE at sizes above every threading
    threshold give identical bits."""
    cfg = oracle.Cfg(dim=96, hidden=160, nLayers=2, nHeads=6, nKvHeads=2, vocab=300, tied=0)
    p = oracle.init_weights(cfg, 3)
    rs = np.random.default_rng(2)
    B, T = 3, 70
    ids = rs.integers(0, 300, B * T).astype(np.int32)
    tg = rs.integers(0, 300, B * T).astype(np.int32)
    runs = []
    import os
    for n in (1, max(2, os.cpu_count() or 2)):
        oracle.set_threads(n)
        lg, loss, g = oracle.model_fwd_bwd(cfg, p, ids, tg, B, T)
        runs.append(np.concatenate([lg.ravel(), [loss], g.ravel()]))
    oracle.set_threads(os.cpu_count() or 1)
    np.testing.assert_array_equal(runs[0], runs[1])


# ───────────────────────── rmsNorm ─────────────────────────
def test_rmsnorm_fwd_bwd_vs_closed_form_and_fd():
    rs = np.random.default_rng(3)
    T, D, eps = 4, 6, 1e-5
    X, w, G = r64(rs, T, D), r64(rs, D, s=0.5) + 1, r64(rs, T, D)
    Y, inv = oracle.rmsnorm_fwd(X.ravel(), w, T, D, eps)
    rY, rinv = np_ref.rmsnorm(X.astype(np.float64), w.astype(np.float64), eps)
    np.testing.assert_allclose(Y.reshape(T, D), rY, rtol=2e-7, atol=1e-7)
    np.testing.assert_allclose(inv, rinv, rtol=2e-7)
    gX, gw = oracle.rmsnorm_bwd(G.ravel(), X.ravel(), w, inv, T, D)
    rX, rw = np_ref.rmsnorm_grads(G.astype(np.float64), X.astype(np.float64), w.astype(np.float64), eps)
    np.testing.assert_allclose(gX.reshape(T, D), rX, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gw, rw, rtol=1e-5, atol=1e-6)
    # the closed form itself against fp64 central differences of the forward
    X64, w64, G64 = X.astype(np.float64), w.astype(np.float64), G.astype(np.float64)
    f = lambda x: float(np.sum(np_ref.rmsnorm(x, w64, eps)[0] * G64))
    num = np.zeros_like(X64)
    for idx in np.ndindex(*X64.shape):
        e = np.zeros_like(X64)
        e[idx] = 1e-6
        num[idx] = (f(X64 + e) - f(X64 - e)) / 2e-6
    np.testing.assert_allclose(rX, num, rtol=1e-6, atol=1e-7)


def test_rmsnorm_unit_norm_invariant():
    """I-12: with w = 1 every output row has RMS 1."""
    rs = np.random.default_rng(4)
    Y, _ = oracle.rmsnorm_fwd(r64(rs, 8 * 16).ravel(), np.ones(16, np.float32), 8, 16, 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(Y.reshape(8, 16).astype(np.float64) ** 2, 1)), 1.0, atol=1e-6)


# ───────────────────────── RoPE ─────────────────────────
@pytest.mark.parametrize("T,nH,dH,pos0,theta,stride", [(3, 2, 4, 0, 1e4, 0), (16, 3, 8, 5, 1e4, 0),
                                                       (24, 2, 16, 0, 5e5, 8)])
def test_rope_vs_complex_rotation(T, nH, dH, pos0, theta, stride):
    rs = np.random.default_rng(5)
    X, G = r64(rs, T, nH * dH), r64(rs, T, nH * dH)
    Y = oracle.rope_fwd(X.ravel(), T, nH, dH, pos0, theta, stride).reshape(T, -1)
    ref = np_ref.rope(X.astype(np.float64), nH, dH, pos0, theta, stride)
    np.testing.assert_allclose(Y, ref, rtol=1e-6, atol=1e-6)
    gX = oracle.rope_bwd(G.ravel(), T, nH, dH, pos0, theta, stride).reshape(T, -1)
    np.testing.assert_allclose(gX, np_ref.rope(G.astype(np.float64), nH, dH, pos0, theta, stride, inverse=True),
                               rtol=1e-6, atol=1e-6)
    # adjointness <R x, g> = <x, R^T g>
    assert abs(np.sum(ref * G) - np.sum(X.astype(np.float64) * gX)) < 1e-4


def test_rope_relativity():
    """I-13: (R_m q)·(R_n k) depends only on m - n."""
    rs = np.random.default_rng(6)
    q, k = r64(rs, 1, 8), r64(rs, 1, 8)
    def rot(x, p):
        return oracle.rope_fwd(x.ravel(), 1, 1, 8, p, 1e4, 0).astype(np.float64)
    assert abs(rot(q, 3) @ rot(k, 9) - rot(q, 0) @ rot(k, 6)) < 1e-5


def test_rope_table_matches_angles():
    c, s = oracle.rope_table(10, 8, 1e4)
    ang = np_ref.rope_angles(10, 8, 0, 1e4, 0)
    np.testing.assert_array_equal(c, np.cos(ang).ravel())
    np.testing.assert_array_equal(s, np.sin(ang).ravel())


# ───────────────────────── attention ─────────────────────────
@pytest.mark.parametrize("B,T,nH,nKV,dH", [(1, 4, 4, 2, 4), (2, 7, 4, 4, 8), (2, 5, 6, 2, 3), (1, 9, 2, 1, 16)])
def test_attention_vs_closed_form(B, T, nH, nKV, dH):
    rs = np.random.default_rng(B * 10 + T)
    Q, K, V, G = r64(rs, B * T, nH * dH), r64(rs, B * T, nKV * dH), r64(rs, B * T, nKV * dH), r64(rs, B * T, nH * dH)
    O, P = oracle.attn_fwd(Q.ravel(), K.ravel(), V.ravel(), B, T, nH, nKV, dH)
    rO, grads = np_ref.attention(Q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), B, T, nH, nKV, dH)
    np.testing.assert_allclose(O.reshape(rO.shape), rO, rtol=1e-5, atol=1e-6)
    P4 = P.reshape(B, nH, T, T)
    assert np.all(P4[:, :, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] == 0)  # causal (I-52)
    np.testing.assert_allclose(P4.sum(-1), 1.0, atol=1e-6)  # rows sum to 1 (I-51)
    gQ, gK, gV = oracle.attn_bwd(G.ravel(), P, Q.ravel(), K.ravel(), V.ravel(), B, T, nH, nKV, dH)
    rQ, rK, rV = grads(G.astype(np.float64))
    for a, b in [(gQ, rQ), (gK, rK), (gV, rV)]:
        np.testing.assert_allclose(a.reshape(b.shape), b, rtol=1e-4, atol=1e-5)


def test_attention_closed_form_vs_fd():
    rs = np.random.default_rng(8)
    B, T, nH, nKV, dH = 1, 4, 2, 1, 3
    Q, K, V, G = (rs.standard_normal((B * T, n * dH)) for n in (nH, nKV, nKV, nH))
    _, grads = np_ref.attention(Q, K, V, B, T, nH, nKV, dH)
    rQ, rK, rV = grads(G)
    f = lambda q, k, v: float(np.sum(np_ref.attention(q, k, v, B, T, nH, nKV, dH)[0] * G))
    for which, ref in ((0, rQ), (1, rK), (2, rV)):
        args = [Q, K, V]
        for idx in np.ndindex(*args[which].shape):
            e = np.zeros_like(args[which]); e[idx] = 1e-6
            ap, am = list(args), list(args)
            ap[which] = args[which] + e; am[which] = args[which] - e
            assert abs((f(*ap) - f(*am)) / 2e-6 - ref[idx]) < 1e-6


def test_batch_attention_equals_per_sample():
    rs = np.random.default_rng(9)
    B, T, nH, nKV, dH = 3, 5, 2, 1, 4
    Q, K, V = r64(rs, B * T, nH * dH), r64(rs, B * T, nKV * dH), r64(rs, B * T, nKV * dH)
    O, _ = oracle.attn_fwd(Q.ravel(), K.ravel(), V.ravel(), B, T, nH, nKV, dH)
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        Ob, _ = oracle.attn_fwd(Q[sl].ravel(), K[sl].ravel(), V[sl].ravel(), 1, T, nH, nKV, dH)
        np.testing.assert_array_equal(O.reshape(B * T, -1)[sl].ravel(), Ob)


# ───────────────────────── SwiGLU, CE, embed, slice, weightedSum ─────────────────────────
def test_swiglu_vs_closed_form_and_fd():
    rs = np.random.default_rng(10)
    G, U, dO = r64(rs, 50, s=2), r64(rs, 50), r64(rs, 50)
    O, sig = oracle.swiglu_fwd(G, U)
    np.testing.assert_allclose(O, np_ref.swiglu(G.astype(np.float64), U.astype(np.float64)), rtol=2e-7, atol=1e-7)
    gG, gU = oracle.swiglu_bwd(dO, sig, G, U)
    rG, rU = np_ref.swiglu_grads(dO.astype(np.float64), G.astype(np.float64), U.astype(np.float64))
    np.testing.assert_allclose(gG, rG, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gU, rU, rtol=1e-6, atol=1e-7)
    G64, U64, d64 = G.astype(np.float64), U.astype(np.float64), dO.astype(np.float64)
    num = (np_ref.swiglu(G64 + 1e-6, U64) - np_ref.swiglu(G64 - 1e-6, U64)) / 2e-6 * d64
    np.testing.assert_allclose(rG, num, rtol=1e-6, atol=1e-7)


def test_ce_known_answers():
    # l2-l6.test.js:139-156 / verify.js I-34: gradient = (P - OneHot)/T
    rs = np.random.default_rng(7)
    T, V = 3, 6
    L = r64(rs, T, V)
    tg = np.array([1, 3, 0], np.int32)
    loss, probs = oracle.ce_fwd(L.ravel(), tg, T, V)
    g = oracle.ce_bwd(1.0, probs, tg, T, V).reshape(T, V)
    rl, rg = np_ref.ce(L.astype(np.float64), tg)
    assert abs(loss - rl) < 1e-6
    assert np.max(np.abs(g - rg)) < 1e-7
    # softmaxCE of verify.js I-31 logits [1.2, 0.3, -0.5, 2.1], target 1
    x = np.array([1.2, 0.3, -0.5, 2.1], np.float32)
    loss1, p1 = oracle.ce_fwd(x, np.array([1], np.int32), 1, 4)
    e = np.exp(x.astype(np.float64) - 2.1)
    assert abs(loss1 - (-np.log(e[1] / e.sum()))) < 1e-6
    g1 = oracle.ce_bwd(1.0, p1, np.array([1], np.int32), 1, 4)
    np.testing.assert_allclose(g1, e / e.sum() - np.eye(4)[1], atol=1e-7)


def test_embed_known_answer():
    # l2-l6.test.js:158-173: E[i] = 0.1 i, ids [0,2,2], t = i+1
    V, D = 4, 3
    E = (np.arange(V * D) * 0.1).astype(np.float32)
    ids = np.array([0, 2, 2], np.int32)
    X = oracle.embed_fwd(E, ids, D)
    np.testing.assert_array_equal(X, E.reshape(V, D)[ids].ravel())
    t = np.arange(1, len(ids) * D + 1, dtype=np.float32)
    gE = oracle.embed_bwd(t, ids, V, D).reshape(V, D)
    want = np.zeros((V, D))
    np.add.at(want, ids, t.reshape(-1, D))
    np.testing.assert_array_equal(gE, want)


def test_slice_and_add():
    rs = np.random.default_rng(12)
    X = r64(rs, 5, 10)
    Y = oracle.slice_fwd(X.ravel(), 5, 10, 3, 4).reshape(5, 4)
    np.testing.assert_array_equal(Y, X[:, 3:7])
    g = r64(rs, 5, 4)
    gX = oracle.slice_bwd(g.ravel(), 5, 10, 3, 4).reshape(5, 10)
    assert np.all(gX[:, :3] == 0) and np.all(gX[:, 7:] == 0) and np.array_equal(gX[:, 3:7], g)
    a, b = r64(rs, 9), r64(rs, 9)
    np.testing.assert_array_equal(oracle.add_fwd(a, b), a + b)


def test_weighted_sum():
    rs = np.random.default_rng(13)
    Y, t = r64(rs, 40), r64(rs, 40)
    assert abs(oracle.weighted_sum_fwd(Y, t) - float(Y.astype(np.float64) @ t)) < 1e-5
    np.testing.assert_array_equal(oracle.weighted_sum_bwd(2.0, t), (2.0 * t.astype(np.float64)).astype(np.float32))


# ───────────────────────── Adam ─────────────────────────
def test_adam_known_answer():
    # l2-l6.test.js:205-211: lr 0.1, g = 1, total 100 -> dw = 0.1 (1+cos(pi/100))/2/(1+1e-8)
    p, g = [np.ones(1, np.float32)], [np.ones(1, np.float32)]
    m, v = [np.zeros(1, np.float32)], [np.zeros(1, np.float32)]
    info = oracle.adam_step(p, g, m, v, 1, lr=0.1, total=100)
    want = 0.1 * 0.5 * (1 + np.cos(np.pi / 100)) / (1 + 1e-8)
    assert abs((1 - p[0][0]) - want) < 1e-7
    assert info["gnorm"] == 1.0 and info["scale"] == 1.0


def test_adam_vs_closed_form_with_clip_wd_and_skipped_grads():
    rs = np.random.default_rng(14)
    sizes = [7, 30, 5]
    p = [r64(rs, n) for n in sizes]
    g = [r64(rs, n, s=3) for n in sizes]
    g[1] = None  # a param without a gradient is skipped (autograd.js:225,231)
    m = [r64(rs, n, s=0.1) for n in sizes]
    v = [np.abs(r64(rs, n, s=0.1)) for n in sizes]
    ref, gnorm, scale, lr_t = np_ref.adam([x.astype(np.float64) for x in p],
                                          [None if x is None else x.astype(np.float64) for x in g],
                                          [x.astype(np.float64) for x in m], [x.astype(np.float64) for x in v],
                                          4, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1.0, 10)
    p0 = [x.copy() for x in p]
    info = oracle.adam_step(p, g, m, v, 4, lr=3e-4, wd=0.01, clip=1.0, total=10)
    assert abs(info["gnorm"] - gnorm) < 1e-9 * gnorm and scale < 1 and abs(info["scale"] - scale) < 1e-12
    assert abs(info["lr"] - lr_t) < 1e-18
    np.testing.assert_array_equal(p[1], p0[1])
    for (rp, rm, rv), pp, mm, vv in zip(ref, p, m, v):
        np.testing.assert_allclose(pp, rp, rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(mm, rm, rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(vv, rv, rtol=1e-6, atol=1e-12)


def test_adam_given_norm_on_a_subset_equals_the_full_step():
    """The step checked on a subset of the tensors with the whole set's norm
    given updates that subset with the full step's bits; with its own norm
    it is the plain step."""
    rs = np.random.default_rng(15)
    sizes = [9, 40, 3, 17]
    mk = lambda s: [r64(rs, n, s=s) for n in sizes]
    p, g, m = mk(1.0), mk(2.0), mk(0.1)
    v = [np.abs(x) for x in mk(0.1)]
    full = [[x.copy() for x in a] for a in (p, g, m, v)]
    info = oracle.adam_step(*full, 3, lr=1e-3, wd=0.01, clip=1.0, total=50)
    assert info["scale"] < 1
    keep = [1, 3]
    sub = [[a[j].copy() for j in keep] for a in (p, g, m, v)]
    info2 = oracle.adam_step(*sub, 3, lr=1e-3, wd=0.01, clip=1.0, total=50, gnorm=info["gnorm"])
    assert info2["gnorm"] == info["gnorm"] and info2["scale"] == info["scale"]
    for a_full, a_sub in zip(full, sub):
        for k, j in enumerate(keep):
            np.testing.assert_array_equal(a_sub[k], a_full[j])
    own = [[a[j].copy() for j in keep] for a in (p, g, m, v)]
    tot = 0.0
    for j in keep:  # the oracle's own summation order: one element at a time
        for x in g[j].astype(np.float64):
            tot += x * x
    n_own = float(np.sqrt(tot))
    plain = [[a[j].copy() for j in keep] for a in (p, g, m, v)]
    oracle.adam_step(*own, 3, lr=1e-3, wd=0.01, clip=1.0, total=50, gnorm=n_own)
    oracle.adam_step(*plain, 3, lr=1e-3, wd=0.01, clip=1.0, total=50)
    for x, y in zip(own, plain):
        for a, b in zip(x, y):
            np.testing.assert_array_equal(a, b)


# ───────────────────────── model ─────────────────────────
TINY = dict(dim=16, hidden=24, nLayers=2, nHeads=4, nKvHeads=2, vocab=11)


def _tiny(tied=True, seed=3):
    cfg = oracle.Cfg(**TINY, tied=1 if tied else 0)
    params = oracle.init_weights(cfg, seed, std=0.3)
    return cfg, params


@pytest.mark.parametrize("tied", [True, False])
def test_model_forward_vs_fp64_restatement(tied):
    cfg, params = _tiny(tied)
    rs = np.random.default_rng(1)
    B, T = 2, 5
    ids = rs.integers(0, cfg.vocab, B * T).astype(np.int32)
    tg = rs.integers(0, cfg.vocab, B * T).astype(np.int32)
    logits, loss, _ = oracle.model_fwd_bwd(cfg, params, ids, tg, B, T)
    P = {k: v.astype(np.float64) for k, v in oracle.split_params(cfg, params).items()}
    rl, rlog = np_ref.model_loss(P, ids, tg, B, T, tied=tied, **TINY)
    np.testing.assert_allclose(logits.reshape(rlog.shape), rlog, rtol=1e-5, atol=1e-5)
    assert abs(loss - rl) < 1e-5


@pytest.mark.parametrize("tied", [True, False])
def test_model_gradients_vs_fp64_central_differences(tied):
    cfg, params = _tiny(tied)
    rs = np.random.default_rng(2)
    B, T = 2, 4
    ids = rs.integers(0, cfg.vocab, B * T).astype(np.int32)
    tg = rs.integers(0, cfg.vocab, B * T).astype(np.int32)
    _, _, grads = oracle.model_fwd_bwd(cfg, params, ids, tg, B, T)
    P = {k: v.astype(np.float64) for k, v in oracle.split_params(cfg, params).items()}
    G = oracle.split_params(cfg, grads)
    for name, n in cfg.param_shapes():
        for i in rs.choice(n, size=min(n, 4), replace=False):
            Pp = {k: v.copy() for k, v in P.items()}
            Pm = {k: v.copy() for k, v in P.items()}
            Pp[name][i] += 1e-5
            Pm[name][i] -= 1e-5
            num = (np_ref.model_loss(Pp, ids, tg, B, T, tied=tied, **TINY)[0]
                   - np_ref.model_loss(Pm, ids, tg, B, T, tied=tied, **TINY)[0]) / 2e-5
            scale = max(float(np.max(np.abs(G[name]))), 1e-3)
            assert abs(num - G[name][i]) / scale < 1e-3, (name, i, num, G[name][i])


def test_i70_training_forward_equals_inference_forward():
    """verify.js:288-310 on the oracle: the batched training forward and the
    token-by-token decode with a KV cache are independent code paths."""
    cfg = oracle.Cfg(dim=32, hidden=64, nLayers=2, nHeads=4, nKvHeads=2, vocab=40, tied=1)
    params = oracle.init_weights(cfg, 4242)
    ids = np.array([1, 5, 9, 13, 2, 7], np.int32)
    tl, _, _ = oracle.model_fwd_bwd(cfg, params, ids, ids, 1, 6)
    il = oracle.infer_forward(cfg, params, ids)
    assert np.max(np.abs(tl - il)) < 1e-6


def test_model_batch_equals_per_sample_and_overfit():
    cfg = oracle.Cfg(dim=32, hidden=64, nLayers=2, nHeads=4, nKvHeads=2, vocab=20, tied=1)
    params = oracle.init_weights(cfg, 11)
    rows = np.array([[1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12]], np.int32)
    ids, tg = rows[:, :-1].ravel(), rows[:, 1:].ravel()
    _, lb, _ = oracle.model_fwd_bwd(cfg, params, ids, tg, 2, 5)
    per = [oracle.model_fwd_bwd(cfg, params, r[:-1], r[1:], 1, 5)[1] for r in rows]
    assert abs(lb - np.mean(per)) < 1e-5
    # I-71: repeated Adam steps on one batch reduce the loss
    cfg2 = oracle.Cfg(dim=32, hidden=64, nLayers=1, nHeads=4, nKvHeads=4, vocab=20, tied=1)
    p = oracle.init_weights(cfg2, 777)
    data = np.arange(1, 9, dtype=np.int32)
    parts = [a.copy() for a in oracle.split_params(cfg2, p).values()]
    m = [np.zeros_like(a) for a in parts]
    v = [np.zeros_like(a) for a in parts]
    first = None
    for s in range(60):
        _, loss, g = oracle.model_fwd_bwd(cfg2, np.concatenate(parts), data[:-1], data[1:], 1, 7)
        first = loss if first is None else first
        gs = [a.copy() for a in oracle.split_params(cfg2, g).values()]
        oracle.adam_step(parts, gs, m, v, s + 1, lr=0.05, total=60)
    _, last, _ = oracle.model_fwd_bwd(cfg2, np.concatenate(parts), data[:-1], data[1:], 1, 7)
    assert last < 0.6 * first


def test_init_weights_layout_and_scaling():
    cfg = oracle.Cfg(dim=8, hidden=16, nLayers=2, nHeads=2, nKvHeads=1, vocab=5, tied=1)
    w = oracle.split_params(cfg, oracle.init_weights(cfg, 1337))
    r = PyRNG(1337)

    def normal():
        u = max(r.next(), 1e-12)
        v = r.next()
        return np.sqrt(-2 * np.log(u)) * np.cos(2 * np.pi * v)
    tok = np.array([normal() * 0.02 for _ in range(5 * 8)], np.float32)
    np.testing.assert_array_equal(w["tok_emb"], tok)  # first draws = tok_emb
    assert np.all(w["ln_f"] == 1) and np.all(w["layer.0.ln1"] == 1) and np.all(w["layer.1.ln2"] == 1)
    qkv = np.array([normal() * 0.02 for _ in range(cfg.qkvOut * 8)], np.float32)
    np.testing.assert_array_equal(w["layer.0.wqkv"], qkv)
    wo = np.array([normal() * 0.02 for _ in range(64)], np.float32)
    np.testing.assert_array_equal(w["layer.0.wo"], (wo.astype(np.float64) / np.sqrt(4)).astype(np.float32))
