"""Seeded random shapes through the GEMM planner and the attention routes.

The fixed-shape tests pin each kernel variant at chosen sizes; these draw
shapes at random (a fixed seed, so every run checks the same cases): log-
uniform sizes mixed with tile multiples and tile multiples +- 1, so the
planner's choices (tile kernel, K split, tail split) and the attention
routes (scalar, MFMA, head-padded, batched GEMMs), the cross-entropy row
kernels (registers, registers + LDS, two reads) and the RMSNorm row kernels
(wave per row, workgroup per row) meet edges no list names.

matmulT (tensor.js:34-53) is checked against the fp64 product on sampled
rows and columns; causalAttnBatch (tensor.js:299-376), crossEntropyMean
(tensor.js:393-417) and rmsNorm (tensor.js:103-128) against the oracle.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from util import TOL_ADAM, TOL_FWD, TOL_GRAD, max_rel, rel_l2

_TILE_STEPS = (32, 64, 128, 192, 256)


def _dim(rs, hi):
    """A log-uniform size in [1, hi], or a tile multiple, or one off it."""
    if rs.random() < 0.5:
        return int(min(hi, max(1, round(math.exp(rs.uniform(0.0, math.log(hi)))))))
    step = int(rs.choice(_TILE_STEPS))
    v = step * int(rs.integers(1, max(2, hi // step + 1))) + int(rs.integers(-1, 2))
    return int(min(hi, max(1, v)))


def _gemm_shapes(n, seed, cap=1 << 24):
    rs = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, K, N = _dim(rs, 9000), _dim(rs, 9000), _dim(rs, 9000)
        if M * K <= cap and N * K <= cap and M * N <= cap:
            out.append((M, K, N))
    return out


GEMM_SWEEP = _gemm_shapes(48, 20261202)


def _pick(rs, n, k=40):
    return np.sort(rs.choice(n, min(n, k), replace=False))


def _tol(kred):
    # fp32-class accumulation: error of a kred-term sum grows like sqrt(kred)
    return 2e-6 * max(1.0, (kred / 4096) ** 0.5)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", GEMM_SWEEP)
def test_matmulT_random_shapes_vs_fp64(fh, M, K, N):
    """Forward, input gradient and (grouped) weight gradient, each with and
    without accumulation onto an existing gradient, on 40 x 40 sampled
    outputs against fp64."""
    rs = np.random.default_rng(M * 7919 + K * 104729 + N)
    X = rs.standard_normal((M, K), dtype=np.float32)
    W = rs.standard_normal((N, K), dtype=np.float32) * np.float32(0.05)
    gY = rs.standard_normal((M, N), dtype=np.float32)
    bx, bw = int(rs.integers(0, 2)), int(rs.integers(0, 2))
    gX0 = rs.standard_normal((M, K), dtype=np.float32) if bx else np.zeros((M, K), np.float32)
    gW0 = rs.standard_normal((N, K), dtype=np.float32) if bw else np.zeros((N, K), np.float32)
    DA = fh.DeviceArray
    dX, dW, dg = DA.from_numpy(X.ravel()), DA.from_numpy(W.ravel()), DA.from_numpy(gY.ravel())
    Y = DA((M * N,))
    fh.call("matmulT_fwd", Y, dX, dW, M, K, N)
    gX = DA.from_numpy(gX0.ravel())
    fh.call("matmulT_bwd_x", gX, dg, dW, M, K, N, bx)
    gW = DA.from_numpy(gW0.ravel())
    jobs = (fh.WgradJob * 1)(fh.WgradJob(gW.ptr, dg.ptr, dX.ptr, M, K, N, bw))
    fh.check(fh.lib.fg_matmulT_bwd_w_grouped(ctypes.cast(jobs, ctypes.c_void_p), 1), "fg_matmulT_bwd_w_grouped")
    Yn, gXn, gWn = Y.numpy().reshape(M, N), gX.numpy().reshape(M, K), gW.numpy().reshape(N, K)
    X64, W64, g64 = X.astype(np.float64), W.astype(np.float64), gY.astype(np.float64)

    r, c = _pick(rs, M), _pick(rs, N)
    ref = X64[r] @ W64[c].T
    got = Yn[np.ix_(r, c)]
    assert rel_l2(got, ref) < max(_tol(K), TOL_FWD / 5)
    assert max_rel(got, ref) < TOL_GRAD

    r, c = _pick(rs, M), _pick(rs, K)
    ref = gX0[np.ix_(r, c)].astype(np.float64) + g64[r] @ W64[:, c]
    got = gXn[np.ix_(r, c)]
    assert rel_l2(got, ref) < max(_tol(N), TOL_FWD / 5)
    assert max_rel(got, ref) < TOL_GRAD

    r, c = _pick(rs, N), _pick(rs, K)
    ref = gW0[np.ix_(r, c)].astype(np.float64) + g64[:, r].T @ X64[:, c]
    got = gWn[np.ix_(r, c)]
    assert rel_l2(got, ref) < max(_tol(M), TOL_FWD / 5)
    assert max_rel(got, ref) < TOL_GRAD


_EDGE_DH = (1, 2, 16, 31, 32, 33, 63, 64, 65, 80, 127, 128, 129, 192, 256, 257)


def _attn_cases(n, seed):
    rs = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dH = int(rs.choice(_EDGE_DH)) if rs.random() < 0.6 else int(rs.integers(1, 301))
        T = int(rs.choice([1, 31, 32, 33, 127, 128, 129])) if rs.random() < 0.3 else int(rs.integers(1, 301))
        B = int(rs.integers(1, 4))
        nKV = int(rs.integers(1, 5))
        group = int(rs.integers(1, 5))
        nH = nKV * group
        if rs.random() < 0.1:  # fewer query heads than kv heads
            nH, nKV = nKV, nKV * group
        # keep the oracle's work to a second or two
        if B * nH * T * T * dH <= 6e8:
            out.append((B, T, nH, nKV, dH))
    return out


ATTN_SWEEP = _attn_cases(40, 7)


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,nH,nKV,dH", ATTN_SWEEP)
def test_attention_random_shapes_vs_oracle(fh, B, T, nH, nKV, dH):
    """Forward output and every gradient against the oracle, then the same
    backward accumulated onto existing gradients."""
    rng = oracle.RNG(B * 1000003 + T * 1009 + nH * 101 + nKV * 11 + dH)
    Q = rng.normal_f32(B * T * nH * dH)
    K = rng.normal_f32(B * T * nKV * dH)
    V = rng.normal_f32(B * T * nKV * dH)
    g = rng.normal_f32(B * T * nH * dH)
    O_ref, P = oracle.attn_fwd(Q, K, V, B, T, nH, nKV, dH)
    gQ_ref, gK_ref, gV_ref = oracle.attn_bwd(g, P, Q, K, V, B, T, nH, nKV, dH)
    DA = fh.DeviceArray
    dq, dk, dv, dg = DA.from_numpy(Q), DA.from_numpy(K), DA.from_numpy(V), DA.from_numpy(g)
    O, lse = DA((B * T * nH * dH,)), DA((B * nH * T,))
    fh.call("attn_fwd", O, lse, dq, dk, dv, B, T, nH, nKV, dH)
    assert rel_l2(O.numpy(), O_ref) < TOL_FWD
    gQ, gK, gV = DA(Q.shape), DA(K.shape), DA(V.shape)
    fh.call("attn_bwd", gQ, 0, gK, 0, gV, 0, dg, dq, dk, dv, O, lse, B, T, nH, nKV, dH)
    if T == 1:
        # one key per query: dQ = dK = 0 exactly, both sides rounding noise
        assert np.max(np.abs(gQ.numpy())) < 1e-5 and np.max(np.abs(gK.numpy())) < 1e-5
        assert max_rel(gV.numpy(), gV_ref) < TOL_GRAD
        return
    for got, ref in ((gQ, gQ_ref), (gK, gK_ref), (gV, gV_ref)):
        assert max_rel(got.numpy(), ref) < TOL_GRAD
    fh.call("attn_bwd", gQ, 1, gK, 1, gV, 1, dg, dq, dk, dv, O, lse, B, T, nH, nKV, dH)
    for got, ref in ((gQ, gQ_ref), (gK, gK_ref), (gV, gV_ref)):
        assert max_rel(got.numpy(), 2.0 * ref.astype(np.float64)) < TOL_GRAD


def _row_cases(n, seed, edges, hi, cap):
    rs = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        if rs.random() < 0.5:
            w = int(rs.choice(edges)) + int(rs.integers(-1, 2))
        else:
            w = int(round(math.exp(rs.uniform(0.0, math.log(hi)))))
        w = max(1, min(hi, w))
        rows = int(rs.integers(1, max(2, min(4096, cap // w) + 1)))
        out.append((rows, w))
    return out


CE_SWEEP = _row_cases(20, 11, (4, 1024, 4096, 32000, 32768, 65536, 131072), 140000, 1 << 23)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,V", CE_SWEEP)
def test_ce_random_shapes_vs_oracle(fh, rows, V):
    """Loss and logits gradient of the separate forward / backward and of the
    fused training loss, against the oracle."""
    DA = fh.DeviceArray
    rng = oracle.RNG(rows * 131 + V)
    logits = rng.normal_f32(rows * V, 2.0)
    targets = rng.ints(rows, V)
    loss_ref, probs = oracle.ce_fwd(logits, targets, rows, V)
    gl_ref = oracle.ce_bwd(1.0, probs, targets, rows, V)
    L, T = DA.from_numpy(logits), DA.from_numpy(targets)
    g1 = DA.from_numpy(np.ones(1, np.float32))
    loss, lse, gl = DA((1,)), DA((rows,)), DA((rows * V,))
    fh.call("ce_fwd", loss, lse, L, T, rows, V)
    fh.call("ce_bwd", gl, L, lse, T, g1, rows, V, 0)
    assert rel_l2([loss.numpy()[0]], [loss_ref]) < TOL_FWD
    assert max_rel(gl.numpy(), gl_ref) < TOL_GRAD
    loss2, lse2, gl2 = DA((1,)), DA((rows,)), DA((rows * V,))
    fh.call("ce_fwd_bwd", loss2, lse2, gl2, L, T, rows, V)
    assert rel_l2([loss2.numpy()[0]], [loss_ref]) < TOL_FWD
    assert max_rel(gl2.numpy(), gl_ref) < TOL_GRAD


NORM_SWEEP = _row_cases(20, 12, (64, 256, 1024, 2048, 3072, 4096, 8192), 9000, 1 << 23)


@pytest.mark.gpu
@pytest.mark.parametrize("T,D", NORM_SWEEP)
def test_rmsnorm_random_shapes_vs_oracle(fh, T, D):
    """Forward (output and inverse RMS) and the backward accumulated onto
    existing input and weight gradients, against the oracle."""
    DA = fh.DeviceArray
    rng = oracle.RNG(T * 257 + D)
    X, w, g = rng.normal_f32(T * D), rng.normal_f32(D, 0.5), rng.normal_f32(T * D)
    gX0, gw0 = rng.normal_f32(T * D), rng.normal_f32(D)
    eps = 1e-5
    Y_ref, inv_ref = oracle.rmsnorm_fwd(X, w, T, D, eps)
    gX_ref, gw_ref = oracle.rmsnorm_bwd(g, X, w, inv_ref, T, D, gX=gX0, gw=gw0)
    dX, dw, dg = DA.from_numpy(X), DA.from_numpy(w), DA.from_numpy(g)
    Y, inv = DA((T * D,)), DA((T,))
    fh.call("rmsnorm_fwd", Y, inv, dX, dw, T, D, eps)
    gX, gw = DA.from_numpy(gX0), DA.from_numpy(gw0)
    fh.call("rmsnorm_bwd", gX, 1, gw, 1, dg, dX, dw, inv, T, D)
    assert rel_l2(Y.numpy(), Y_ref) < TOL_FWD
    assert rel_l2(inv.numpy(), inv_ref) < TOL_FWD
    assert max_rel(gX.numpy(), gX_ref) < TOL_GRAD
    assert max_rel(gw.numpy(), gw_ref) < TOL_GRAD


# ───── the remaining row ops and Adam at seeded random shapes ─────
def _rope_cases(n, seed):
    rs = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        dH = 2 * int(rs.integers(1, 80))
        nH = int(rs.integers(1, 9))
        T = int(rs.integers(1, max(2, min(3000, (1 << 21) // (nH * dH)))))
        stride = int(rs.choice([0, max(1, T // int(rs.integers(1, 4)))]))
        out.append((T, nH, dH, int(rs.integers(0, 40)), float(rs.choice([1e4, 5e5])), stride))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("T,nH,dH,pos0,theta,stride", _rope_cases(16, 21))
def test_rope_random_shapes_vs_oracle(fh, T, nH, dH, pos0, theta, stride):
    """ropeRows forward and accumulated backward, bit for bit (fp64 angles
    and arithmetic on both sides)."""
    rng = oracle.RNG(T * 31 + nH * 7 + dH)
    X, g, g0 = rng.normal_f32(T * nH * dH), rng.normal_f32(T * nH * dH), rng.normal_f32(T * nH * dH)
    Y_ref = oracle.rope_fwd(X, T, nH, dH, pos0, theta, stride)
    gX_ref = oracle.rope_bwd(g, T, nH, dH, pos0, theta, stride, gX=g0)
    npos = pos0 + (min(T, stride) if stride > 0 else T)
    c, s = oracle.rope_table(npos, dH, theta)
    DA = fh.DeviceArray
    dc, ds = DA.from_numpy(c), DA.from_numpy(s)
    Y = DA((T * nH * dH,))
    fh.call("rope_fwd", Y, DA.from_numpy(X), dc, ds, npos, T, nH, dH, pos0, stride)
    gX = DA.from_numpy(g0)
    fh.call("rope_bwd", gX, DA.from_numpy(g), dc, ds, npos, T, nH, dH, pos0, stride, 1)
    np.testing.assert_array_equal(Y.numpy(), Y_ref)
    np.testing.assert_array_equal(gX.numpy(), gX_ref)


def _embed_cases(n, seed):
    rs = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        D = int(rs.choice([int(rs.integers(1, 2100)), 4 * int(rs.integers(1, 520))]))
        V = int(round(math.exp(rs.uniform(0.0, math.log(140000)))))
        V = max(1, min(V, (1 << 24) // D))
        T = int(rs.integers(1, max(2, min(9000, (1 << 23) // D))))
        out.append((T, V, D))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("T,V,D", _embed_cases(16, 22))
def test_embed_random_shapes_vs_oracle(fh, T, V, D):
    """embedLookup forward and the planned backward onto an existing gradient
    (ids with many repeats), bit for bit."""
    from test_gpu_ops import embed_plan
    rng = oracle.RNG(T * 13 + V * 3 + D)
    W, g = rng.normal_f32(V * D), rng.normal_f32(T * D)
    ids = rng.ints(T, max(1, min(V, T // 3 + 1)))
    gW0 = rng.normal_f32(V * D, 0.1)
    DA = fh.DeviceArray
    X = DA((T * D,))
    fh.call("embed_fwd", X, DA.from_numpy(W), DA.from_numpy(ids), T, V, D)
    np.testing.assert_array_equal(X.numpy(), oracle.embed_fwd(W, ids, D))
    perm, ss, sid, ns = embed_plan(fh, ids, V)
    gW = DA.from_numpy(gW0)
    fh.call("embed_bwd", gW, DA.from_numpy(g), DA.from_numpy(perm), DA.from_numpy(ss), DA.from_numpy(sid), ns, D)
    np.testing.assert_array_equal(gW.numpy(), oracle.embed_bwd(g, ids, V, D, gW=gW0))


def _gu_cases(n, seed):
    rs = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        H = int(rs.choice([int(rs.integers(1, 6000)), 4 * int(rs.integers(1, 1500))]))
        rows = int(rs.integers(1, max(2, min(5000, (1 << 22) // H))))
        out.append((rows, H))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("rows,H", _gu_cases(12, 23))
def test_swiglu_gate_up_random_shapes_vs_oracle(fh, rows, H):
    """swigluRows over the packed [gate | up] rows: forward against the
    oracle, backward (accumulating) against the oracle."""
    rng = oracle.RNG(rows * 17 + H)
    G, U, g = rng.normal_f32(rows * H, 2.0), rng.normal_f32(rows * H), rng.normal_f32(rows * H)
    g0 = rng.normal_f32(2 * rows * H)
    GU = np.concatenate([G.reshape(rows, H), U.reshape(rows, H)], axis=1).ravel()
    O_ref, sig = oracle.swiglu_fwd(G, U)
    g0r = g0.reshape(rows, 2 * H)
    gG_ref, gU_ref = oracle.swiglu_bwd(g, sig, G, U, gG=np.ascontiguousarray(g0r[:, :H]).ravel(),
                                       gU=np.ascontiguousarray(g0r[:, H:]).ravel())
    DA = fh.DeviceArray
    dGU = DA.from_numpy(GU)
    O = DA((rows * H,))
    fh.call("swiglu_gu_fwd", O, dGU, rows, H)
    assert rel_l2(O.numpy(), O_ref) < TOL_FWD
    gGU = DA.from_numpy(g0)
    fh.call("swiglu_gu_bwd", gGU, 1, DA.from_numpy(g), dGU, rows, H)
    got = gGU.numpy().reshape(rows, 2 * H)
    assert max_rel(got[:, :H].ravel(), gG_ref) < TOL_GRAD
    assert max_rel(got[:, H:].ravel(), gU_ref) < TOL_GRAD


def _adam_cases(n, seed):
    rs = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        k = int(rs.integers(1, 9))
        sizes = [int(round(math.exp(rs.uniform(0.0, math.log(300000))))) for _ in range(k)]
        out.append((tuple(sizes), float(rs.choice([0.0, 0.01, 0.1])), float(rs.choice([0.1, 1.0, 1e9])),
                    int(rs.integers(1, 50))))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("sizes,wd,clip,t", _adam_cases(12, 24))
def test_adam_random_lists_vs_oracle(fh, sizes, wd, clip, t):
    """Adam over random tensor lists (ragged chunk tails, clipping on and
    off, weight decay, later steps with moments): parameters bit for bit,
    moments and the norm against the oracle."""
    from test_gpu_ops import _gpu_adam
    rng = oracle.RNG(sum(sizes) + t)
    ps = [rng.normal_f32(n) for n in sizes]
    gs = [rng.normal_f32(n) for n in sizes]
    ms = [rng.normal_f32(n, 0.01) if t > 1 else np.zeros(n, np.float32) for n in sizes]
    vs = [np.abs(rng.normal_f32(n, 0.01)) if t > 1 else np.zeros(n, np.float32) for n in sizes]
    ref_p, ref_m, ref_v = [p.copy() for p in ps], [m.copy() for m in ms], [v.copy() for v in vs]
    info = oracle.adam_step(ref_p, gs, ref_m, ref_v, t, lr=3e-4, wd=wd, clip=clip, total=1000)
    got, stats = _gpu_adam(fh, ps, gs, ms, vs, t, 3e-4, 0.9, 0.999, 1e-8, wd, clip, 1000)
    assert abs(stats[0] - info["gnorm"]) <= 1e-12 * info["gnorm"]
    assert abs(stats[1] - info["scale"]) <= 1e-12
    for (p, m, v), rp, rm, rv in zip(got, ref_p, ref_m, ref_v):
        np.testing.assert_array_equal(p, rp)
        assert rel_l2(m, rm) < TOL_ADAM and rel_l2(v, rv) < TOL_ADAM
