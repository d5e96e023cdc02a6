"""Per-op GPU parity through the C ABI against the C oracle (same seeded inputs).

Tolerances: forward outputs relative-L2 <= 1e-5, gradients max-relative
(to the tensor's max |value|) <= 1e-4, Adam state relative <= 1e-6; integer /
copy work (embedding rows, slices) bit-exact.
"""
import ctypes

import numpy as np
import pytest

import oracle
from util import TOL_ADAM, TOL_FWD, TOL_GRAD, max_rel, rel_l2


def up(fh, a):
    return fh.DeviceArray.from_numpy(np.ascontiguousarray(a))


# ───────────────────────── rmsNorm (tensor.js:103-128) ─────────────────────────
@pytest.mark.gpu
@pytest.mark.parametrize("T,D", [(2, 6), (3, 8), (256, 64), (33, 300), (8192, 768), (64, 4096), (5, 1), (1, 1), (1, 4),
                                 (33, 1028), (17, 2048), (9, 3076), (7, 1500),
                                 # rows over 8192 floats: the generic backward in column chunks
                                 (3, 8193), (40, 16384), (2, 20001)])
@pytest.mark.parametrize("beta", [0, 1])
def test_rmsnorm(fh, T, D, beta):
    rng = oracle.RNG(3)
    X, w, g = rng.normal_f32(T * D), rng.normal_f32(D, 0.5), rng.normal_f32(T * D)
    eps = 1e-5
    Y_ref, inv_ref = oracle.rmsnorm_fwd(X, w, T, D, eps)
    gX0 = rng.normal_f32(T * D) if beta else None
    gw0 = rng.normal_f32(D) if beta else None
    gX_ref, gw_ref = oracle.rmsnorm_bwd(g, X, w, inv_ref, T, D, gX=gX0, gw=gw0)
    dX, dw, dg = up(fh, X), up(fh, w), up(fh, g)
    Y, inv = fh.DeviceArray((T * D,)), fh.DeviceArray((T,))
    fh.call("rmsnorm_fwd", Y, inv, dX, dw, T, D, eps)
    gX = up(fh, gX0) if beta else fh.DeviceArray((T * D,))
    gw = up(fh, gw0) if beta else fh.DeviceArray((D,))
    fh.call("rmsnorm_bwd", gX, beta, gw, beta, dg, dX, dw, inv, T, D)
    assert rel_l2(Y.numpy(), Y_ref) < TOL_FWD
    assert rel_l2(inv.numpy(), inv_ref) < TOL_FWD
    assert max_rel(gX.numpy(), gX_ref) < TOL_GRAD
    assert max_rel(gw.numpy(), gw_ref) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("T,D", [(37, 768), (8192, 768), (64, 96), (16, 5000)])
def test_rmsnorm_bwd_from_equals_in_place(fh, T, D):
    """gX = gX_in + dX into another buffer (a shared gradient) equals the
    in-place accumulation bit for bit; gX_in = NULL equals beta 0."""
    rng = oracle.RNG(4)
    X, w, g, old = rng.normal_f32(T * D), rng.normal_f32(D, 0.5), rng.normal_f32(T * D), rng.normal_f32(T * D)
    dX, dw, dg = up(fh, X), up(fh, w), up(fh, g)
    Y, inv = fh.DeviceArray((T * D,)), fh.DeviceArray((T,))
    fh.call("rmsnorm_fwd", Y, inv, dX, dw, T, D, 1e-5)
    a, gwa = up(fh, old), fh.DeviceArray((D,))
    fh.call("rmsnorm_bwd", a, 1, gwa, 0, dg, dX, dw, inv, T, D)
    src, b, gwb = up(fh, old), fh.DeviceArray((T * D,)), fh.DeviceArray((D,))
    fh.call("rmsnorm_bwd_from", b, src, gwb, 0, dg, dX, dw, inv, T, D)
    np.testing.assert_array_equal(a.numpy(), b.numpy())
    np.testing.assert_array_equal(src.numpy(), old)  # the shared input is not written
    np.testing.assert_array_equal(gwa.numpy(), gwb.numpy())
    c, d = fh.DeviceArray((T * D,)), fh.DeviceArray((T * D,))
    fh.call("rmsnorm_bwd", c, 0, None, 0, dg, dX, dw, inv, T, D)
    fh.call("rmsnorm_bwd_from", d, None, None, 0, dg, dX, dw, inv, T, D)
    np.testing.assert_array_equal(c.numpy(), d.numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("T,D", [(37, 768), (8192, 768), (64, 96), (16, 5000), (50, 4096), (9, 770), (33, 1028),
                                 (17, 2048), (9, 3076)])
def test_rmsnorm_bwd_from_halves_equals_summed_gradient(fh, T, D):
    """The incoming gradient as two halves (the K pieces of the GEMM that
    wrote it) gives the same bits as the backward of their fp32 sum, fresh
    and accumulating (vector rows, wide rows, and the generic kernel at
    D = 770)."""
    rng = oracle.RNG(5)
    X, w, old = rng.normal_f32(T * D), rng.normal_f32(D, 0.5), rng.normal_f32(T * D)
    h0, h1 = rng.normal_f32(T * D), rng.normal_f32(T * D)
    dX, dw = up(fh, X), up(fh, w)
    Y, inv = fh.DeviceArray((T * D,)), fh.DeviceArray((T,))
    fh.call("rmsnorm_fwd", Y, inv, dX, dw, T, D, 1e-5)
    halves = up(fh, np.concatenate([h0, h1]))
    gsum = fh.DeviceArray((T * D,))
    fh.call("add_fwd", gsum, up(fh, h0), up(fh, h1), T * D)
    np.testing.assert_array_equal(gsum.numpy(), h0 + h1)
    for src0 in (None, old):
        a, gwa = fh.DeviceArray((T * D,)), fh.DeviceArray((D,))
        b, gwb = fh.DeviceArray((T * D,)), fh.DeviceArray((D,))
        sa = up(fh, src0) if src0 is not None else None
        sb = up(fh, src0) if src0 is not None else None
        fh.call("rmsnorm_bwd_from", a, sa, gwa, 0, gsum, dX, dw, inv, T, D)
        fh.call("rmsnorm_bwd_from_halves", b, sb, gwb, 0, halves, dX, dw, inv, T, D)
        np.testing.assert_array_equal(a.numpy(), b.numpy())
        np.testing.assert_array_equal(gwa.numpy(), gwb.numpy())


@pytest.mark.gpu
def test_rmsnorm_bwd_partial_and_grouped_colsum_equal_one_call(fh):
    """The deferred weight gradient: fg_rmsnorm_bwd_partial (plain and
    two-halves gradient, fresh and accumulated gX) followed by one
    fg_colsum_grouped launch gives gX and gw bit-identical to the one-call
    backward, for several norms at once (fresh and accumulating gw), with two
    jobs on one output applied in order, and more jobs than one launch
    table holds (64)."""
    DA = fh.DeviceArray
    rng = oracle.RNG(6)
    shapes = [(8192, 768), (37, 768), (50, 4096), (4, 8), (1000, 96), (33, 1028), (17, 2048), (9, 3076)] + \
        [(16, 64 + 4 * i) for i in range(62)]
    jobs, checks = [], []
    for i, (T, D) in enumerate(shapes):
        X, w, old = rng.normal_f32(T * D), rng.normal_f32(D, 0.5), rng.normal_f32(T * D)
        h0, h1 = rng.normal_f32(T * D), rng.normal_f32(T * D)
        gw0 = rng.normal_f32(D)
        halves = i % 2 == 1
        beta_w = (i // 2) % 2
        dX, dw = up(fh, X), up(fh, w)
        Y, inv = DA((T * D,)), DA((T,))
        fh.call("rmsnorm_fwd", Y, inv, dX, dw, T, D, 1e-5)
        g = up(fh, np.concatenate([h0, h1]) if halves else h0)
        src = up(fh, old) if i % 3 == 0 else None
        ref_gx, ref_gw = DA((T * D,)), up(fh, gw0)
        if halves:
            fh.call("rmsnorm_bwd_from_halves", ref_gx, src, ref_gw, beta_w, g, dX, dw, inv, T, D)
        else:
            fh.call("rmsnorm_bwd_from", ref_gx, src, ref_gw, beta_w, g, dX, dw, inv, T, D)
        rows = fh.lib.fg_rmsnorm_bwd_parts(T, D)
        assert rows >= 1, fh.last_error()
        part, gx, gw = DA((rows * D,)), DA((T * D,)), up(fh, gw0)
        fh.call("rmsnorm_bwd_partial", gx, src, part, g, 1 if halves else 0, dX, dw, inv, T, D)
        jobs.append((gw, part, rows, D, beta_w))
        checks.append((gx, gw, ref_gx, ref_gw))
    # a second job on the first output accumulates onto the first job's sum
    T0, D0 = shapes[0]
    extra = DA.from_numpy(rng.normal_f32(jobs[0][2] * D0))
    jobs.insert(1, (jobs[0][0], extra, jobs[0][2], D0, 1))
    arr = (fh.ColsumJob * len(jobs))()
    for k, (out, part, rows, n, beta) in enumerate(jobs):
        arr[k] = fh.ColsumJob(out.ptr, part.ptr, rows, n, beta)
    fh.check(fh.lib.fg_colsum_grouped(ctypes.cast(arr, ctypes.c_void_p), len(jobs)), "fg_colsum_grouped")
    for i, (gx, gw, ref_gx, ref_gw) in enumerate(checks):
        np.testing.assert_array_equal(gx.numpy(), ref_gx.numpy())
        if i == 0:
            col = DA((D0,))
            ex = fh.ColsumJob(col.ptr, extra.ptr, jobs[0][2], D0, 0)
            fh.check(fh.lib.fg_colsum_grouped(ctypes.byref(ex), 1), "fg_colsum_grouped")
            np.testing.assert_array_equal(gw.numpy(), ref_gw.numpy() + col.numpy())
        else:
            np.testing.assert_array_equal(gw.numpy(), ref_gw.numpy())


@pytest.mark.gpu
def test_colsum_grouped_rejects_bad_jobs(fh):
    """Host-side checks: columns not a multiple of 4, and a job with no rows."""
    bad = fh.ColsumJob(16, 16, 4, 6, 0)
    assert fh.lib.fg_colsum_grouped(ctypes.byref(bad), 1) != 0
    assert "n % 4 == 0" in fh.last_error()
    bad = fh.ColsumJob(16, 16, 0, 8, 0)
    assert fh.lib.fg_colsum_grouped(ctypes.byref(bad), 1) != 0


# ───────────────────────── ropeRows (tensor.js:133-166) ─────────────────────────
@pytest.mark.gpu
@pytest.mark.parametrize("T,nH,dH,pos0,theta,stride", [
    (3, 2, 4, 0, 1e4, 0), (256, 4, 16, 0, 1e4, 32), (256, 2, 16, 0, 1e4, 32), (17, 3, 8, 5, 1e4, 0),
    (8192, 12, 64, 0, 1e4, 1024), (4096, 8, 128, 0, 5e5, 4096)])
def test_rope(fh, T, nH, dH, pos0, theta, stride):
    rng = oracle.RNG(4)
    X, g, g0 = rng.normal_f32(T * nH * dH), rng.normal_f32(T * nH * dH), rng.normal_f32(T * nH * dH)
    Y_ref = oracle.rope_fwd(X, T, nH, dH, pos0, theta, stride)
    gX_ref = oracle.rope_bwd(g, T, nH, dH, pos0, theta, stride, gX=g0)
    npos = pos0 + (min(T, stride) if stride > 0 else T)
    c, s = oracle.rope_table(npos, dH, theta)
    dc, ds = up(fh, c), up(fh, s)
    Y = fh.DeviceArray((T * nH * dH,))
    fh.call("rope_fwd", Y, up(fh, X), dc, ds, npos, T, nH, dH, pos0, stride)
    gX = up(fh, g0)
    fh.call("rope_bwd", gX, up(fh, g), dc, ds, npos, T, nH, dH, pos0, stride, 1)
    # same fp64 angles, fp64 arithmetic without contraction: bit-exact
    np.testing.assert_array_equal(Y.numpy(), Y_ref)
    np.testing.assert_array_equal(gX.numpy(), gX_ref)


@pytest.mark.gpu
def test_rope_rejects_short_table(fh):
    c, s = oracle.rope_table(8, 4, 1e4)
    X = fh.DeviceArray((16 * 4,))
    with pytest.raises(fh.ForgeError, match="exceed"):
        fh.call("rope_fwd", X, X, up(fh, c), up(fh, s), 8, 16, 1, 4, 0, 0)


# ───── fused sliceCols×3 + ropeRows×2 (train.js:133-138) ─────
@pytest.mark.gpu
@pytest.mark.parametrize("rows,T,nH,nKV,dH,pos0,theta", [
    (3, 3, 2, 1, 4, 0, 1e4), (10, 5, 2, 1, 6, 1, 1e4), (40, 20, 4, 2, 8, 3, 5e5), (8192, 1024, 12, 12, 64, 0, 1e4),
    (4096, 4096, 32, 8, 128, 0, 5e5)])
@pytest.mark.parametrize("beta", [0, 1])
def test_qkv_rope(fh, rows, T, nH, nKV, dH, pos0, theta, beta):
    rng = oracle.RNG(14)
    qD, kvD = nH * dH, nKV * dH
    W = qD + 2 * kvD
    qkv = rng.normal_f32(rows * W)
    gq, gk, gv = rng.normal_f32(rows * qD), rng.normal_f32(rows * kvD), rng.normal_f32(rows * kvD)
    g0 = rng.normal_f32(rows * W) if beta else None
    # the reference's composition: slices, then RoPE of q and k
    q_ref = oracle.rope_fwd(oracle.slice_fwd(qkv, rows, W, 0, qD), rows, nH, dH, pos0, theta, T)
    k_ref = oracle.rope_fwd(oracle.slice_fwd(qkv, rows, W, qD, kvD), rows, nKV, dH, pos0, theta, T)
    v_ref = oracle.slice_fwd(qkv, rows, W, qD + kvD, kvD)
    g_ref = oracle.slice_bwd(oracle.rope_bwd(gq, rows, nH, dH, pos0, theta, T), rows, W, 0, qD, gX=g0)
    g_ref = oracle.slice_bwd(oracle.rope_bwd(gk, rows, nKV, dH, pos0, theta, T), rows, W, qD, kvD, gX=g_ref)
    g_ref = oracle.slice_bwd(gv, rows, W, qD + kvD, kvD, gX=g_ref)
    npos = pos0 + min(rows, T)
    c, s = oracle.rope_table(npos, dH, theta)
    dc, ds = up(fh, c), up(fh, s)
    Q, K, V = fh.DeviceArray((rows * qD,)), fh.DeviceArray((rows * kvD,)), fh.DeviceArray((rows * kvD,))
    fh.call("qkv_rope_fwd", Q, K, V, up(fh, qkv), dc, ds, npos, rows, nH, nKV, dH, pos0, T)
    np.testing.assert_array_equal(Q.numpy(), q_ref)
    np.testing.assert_array_equal(K.numpy(), k_ref)
    np.testing.assert_array_equal(V.numpy(), v_ref)
    G = up(fh, g0) if beta else fh.DeviceArray((rows * W,))
    fh.call("qkv_rope_bwd", G, up(fh, gq), up(fh, gk), up(fh, gv), dc, ds, npos, rows, nH, nKV, dH, pos0, T, beta)
    if beta:  # one fp64 sum per element instead of two fp32 adds
        assert max_rel(G.numpy(), g_ref) < 1e-6
    else:
        np.testing.assert_array_equal(G.numpy(), g_ref)
    # a missing gradient counts as zero
    G2 = fh.DeviceArray((rows * W,))
    fh.call("qkv_rope_bwd", G2, None, up(fh, gk), None, dc, ds, npos, rows, nH, nKV, dH, pos0, T, 0)
    g_k = oracle.slice_bwd(oracle.rope_bwd(gk, rows, nKV, dH, pos0, theta, T), rows, W, qD, kvD)
    np.testing.assert_array_equal(G2.numpy(), g_k)


@pytest.mark.gpu
def test_qkv_rope_rejects_bad_args(fh):
    c, s = oracle.rope_table(4, 4, 1e4)
    X = fh.DeviceArray((64,))
    with pytest.raises(fh.ForgeError, match="exceed"):
        fh.call("qkv_rope_fwd", X, X, X, X, up(fh, c), up(fh, s), 4, 8, 1, 1, 4, 0, 0)
    with pytest.raises(fh.ForgeError, match="bad shape"):
        fh.call("qkv_rope_fwd", X, X, X, X, up(fh, c), up(fh, s), 4, 2, 1, 1, 3, 0, 0)


# ───── qkv projection with RoPE in the epilogue; attention over qkv column blocks ─────
@pytest.mark.gpu
@pytest.mark.parametrize("M,K,nH,nKV,dH,pos0,T", [
    (8192, 768, 12, 12, 64, 0, 1024),    # 125M shape
    (4096, 512, 32, 8, 128, 0, 4096),    # Llama-3-8B head layout
    (512, 4096, 12, 12, 64, 2, 256),     # pos0 > 0, positions wrapping at T
    (130, 70, 2, 1, 32, 0, 65),          # ragged edges
    (40, 24, 2, 1, 6, 1, 20)])           # dH % 4 != 0: one pair per thread
def test_matmulT_fwd_rope_equals_matmulT_then_qkv_rope(fh, M, K, nH, nKV, dH, pos0, T):
    """fg_matmulT_fwd_rope = fg_matmulT_fwd then the rotation of fg_qkv_rope_fwd,
    bit for bit: q and k column blocks rotated, v untouched."""
    rng = oracle.RNG(41)
    qD, kvD = nH * dH, nKV * dH
    N = qD + 2 * kvD
    X, W = rng.normal_f32(M * K), rng.normal_f32(N * K, 0.05)
    npos = pos0 + min(M, T)
    c, s = oracle.rope_table(npos, dH, 1e4)
    dc, ds = up(fh, c), up(fh, s)
    dX, dW = up(fh, X), up(fh, W)
    Y = fh.DeviceArray((M * N,))
    fh.call("matmulT_fwd_rope", Y, dX, dW, M, K, N, dc, ds, npos, nH, nKV, dH, pos0, T)
    P = fh.DeviceArray((M * N,))
    fh.call("matmulT_fwd", P, dX, dW, M, K, N)
    Q, Kr, V = fh.DeviceArray((M * qD,)), fh.DeviceArray((M * kvD,)), fh.DeviceArray((M * kvD,))
    fh.call("qkv_rope_fwd", Q, Kr, V, P, dc, ds, npos, M, nH, nKV, dH, pos0, T)
    y = Y.numpy().reshape(M, N)
    np.testing.assert_array_equal(y[:, :qD].ravel(), Q.numpy())
    np.testing.assert_array_equal(y[:, qD:qD + kvD].ravel(), Kr.numpy())
    np.testing.assert_array_equal(y[:, qD + kvD:].ravel(), V.numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,nH,nKV,dH", [(8, 1024, 12, 12, 64), (2, 100, 4, 2, 32), (1, 300, 8, 2, 128),
                                            (2, 100, 6, 2, 96)])
def test_attention_over_qkv_blocks_equals_separate(fh, B, T, nH, nKV, dH):
    """fg_attn_fwd_qkv / fg_attn_bwd_qkv on a fused qkv buffer = fg_attn_fwd /
    fg_attn_bwd on the separate q, k, v followed by fg_qkv_rope_bwd, bit for bit."""
    rng = oracle.RNG(42)
    qD, kvD = nH * dH, nKV * dH
    W, rows = qD + 2 * kvD, B * T
    qkv = rng.normal_f32(rows * W)
    dO = rng.normal_f32(rows * qD)
    q3 = qkv.reshape(rows, W)
    Q, K, V = (np.ascontiguousarray(q3[:, :qD]), np.ascontiguousarray(q3[:, qD:qD + kvD]),
               np.ascontiguousarray(q3[:, qD + kvD:]))
    npos = min(rows, T)
    c, s = oracle.rope_table(npos, dH, 1e4)
    dc, ds = up(fh, c), up(fh, s)
    DA = fh.DeviceArray
    dq, dk, dv, ddO, dqkv = up(fh, Q.ravel()), up(fh, K.ravel()), up(fh, V.ravel()), up(fh, dO), up(fh, qkv)
    O1, l1 = DA((rows * qD,)), DA((B * nH * T,))
    fh.call("attn_fwd", O1, l1, dq, dk, dv, B, T, nH, nKV, dH)
    O2, l2 = DA((rows * qD,)), DA((B * nH * T,))
    fh.call("attn_fwd_qkv", O2, l2, dqkv, B, T, nH, nKV, dH)
    np.testing.assert_array_equal(O2.numpy(), O1.numpy())
    np.testing.assert_array_equal(l2.numpy(), l1.numpy())
    gQ, gK, gV = DA((rows * qD,)), DA((rows * kvD,)), DA((rows * kvD,))
    fh.call("attn_bwd", gQ, 0, gK, 0, gV, 0, ddO, dq, dk, dv, O1, l1, B, T, nH, nKV, dH)
    G1 = DA((rows * W,))
    fh.call("qkv_rope_bwd", G1, gQ, gK, gV, dc, ds, npos, rows, nH, nKV, dH, 0, T, 0)
    G2 = DA((rows * W,))
    fh.call("attn_bwd_qkv", G2, ddO, dqkv, O2, l2, B, T, nH, nKV, dH, dc, ds, npos, 0, T)
    np.testing.assert_array_equal(G2.numpy(), G1.numpy())
    # the _p forms: the forward leaves the maxima of the q, k, v column blocks
    # (strided reads of qkv) and the backward reuses them, same bits
    xp = DA((3 * 256,))
    O3, l3 = DA((rows * qD,)), DA((B * nH * T,))
    fh.call("attn_fwd_qkv_p", O3, l3, dqkv, B, T, nH, nKV, dH, xp)
    np.testing.assert_array_equal(O3.numpy(), O1.numpy())
    np.testing.assert_array_equal(l3.numpy(), l1.numpy())
    parts = xp.numpy().reshape(3, 256)
    for p, ref in zip(parts, (Q, K, V)):
        assert p.max() == np.abs(ref).max() and (p <= p.max()).all()
    G3 = DA((rows * W,))
    fh.call("attn_bwd_qkv_p", G3, ddO, dqkv, O3, l3, B, T, nH, nKV, dH, dc, ds, npos, 0, T, xp)
    np.testing.assert_array_equal(G3.numpy(), G1.numpy())


@pytest.mark.gpu
def test_qkv_attention_rejects_bad_args(fh):
    c, s = oracle.rope_table(8, 16, 1e4)
    X = fh.DeviceArray((8 * 64,))
    with pytest.raises(fh.ForgeError, match="dH in"):
        fh.call("attn_fwd_qkv", X, X, X, 1, 8, 2, 1, 16)
    with pytest.raises(fh.ForgeError, match="exceed"):
        fh.call("matmulT_fwd_rope", X, X, X, 8, 8, 64, up(fh, c), up(fh, s), 4, 2, 1, 16, 0, 0)
    with pytest.raises(fh.ForgeError, match="do not fit"):
        fh.call("matmulT_fwd_rope", X, X, X, 8, 8, 16, up(fh, c), up(fh, s), 8, 2, 1, 16, 0, 0)


# ───────────────────────── swigluRows (tensor.js:272-290) ─────────────────────────
@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 10, 256 * 128, 8192 * 2048 + 3])
@pytest.mark.parametrize("beta", [0, 1])
def test_swiglu(fh, n, beta):
    rng = oracle.RNG(6)
    G, U, g = rng.normal_f32(n, 2.0), rng.normal_f32(n), rng.normal_f32(n)
    O_ref, sig = oracle.swiglu_fwd(G, U)
    gG0 = rng.normal_f32(n) if beta else None
    gU0 = rng.normal_f32(n) if beta else None
    gG_ref, gU_ref = oracle.swiglu_bwd(g, sig, G, U, gG=gG0, gU=gU0)
    O = fh.DeviceArray((n,))
    dG, dU = up(fh, G), up(fh, U)
    fh.call("swiglu_fwd", O, dG, dU, n)
    gG = up(fh, gG0) if beta else fh.DeviceArray((n,))
    gU = up(fh, gU0) if beta else fh.DeviceArray((n,))
    fh.call("swiglu_bwd", gG, beta, gU, beta, up(fh, g), dG, dU, n)
    assert rel_l2(O.numpy(), O_ref) < TOL_FWD
    assert max_rel(gG.numpy(), gG_ref) < TOL_GRAD
    assert max_rel(gU.numpy(), gU_ref) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("rows,H", [(3, 4), (256, 2048), (8192, 2048), (5, 7), (33, 230)])
@pytest.mark.parametrize("beta", [0, 1])
def test_swiglu_gate_up_layout(fh, rows, H, beta):
    """The [G | U] row layout kernels give the separate-tensor kernels' values bit for bit."""
    rng = oracle.RNG(12)
    G, U, g = rng.normal_f32(rows * H), rng.normal_f32(rows * H), rng.normal_f32(rows * H)
    GU = np.concatenate([G.reshape(rows, H), U.reshape(rows, H)], axis=1).ravel()
    g0 = rng.normal_f32(2 * rows * H) if beta else None
    O, Or = fh.DeviceArray((rows * H,)), fh.DeviceArray((rows * H,))
    fh.call("swiglu_gu_fwd", O, up(fh, GU), rows, H)
    fh.call("swiglu_fwd", Or, up(fh, G), up(fh, U), rows * H)
    np.testing.assert_array_equal(O.numpy(), Or.numpy())
    gGU = up(fh, g0) if beta else fh.DeviceArray((2 * rows * H,))
    fh.call("swiglu_gu_bwd", gGU, beta, up(fh, g), up(fh, GU), rows, H)
    gG0 = g0.reshape(rows, 2 * H)[:, :H].ravel() if beta else np.zeros(rows * H, np.float32)
    gU0 = g0.reshape(rows, 2 * H)[:, H:].ravel() if beta else np.zeros(rows * H, np.float32)
    gG, gU = up(fh, gG0), up(fh, gU0)
    fh.call("swiglu_bwd", gG, beta, gU, beta, up(fh, g), up(fh, G), up(fh, U), rows * H)
    got = gGU.numpy().reshape(rows, 2 * H)
    np.testing.assert_array_equal(got[:, :H].ravel(), gG.numpy())
    np.testing.assert_array_equal(got[:, H:].ravel(), gU.numpy())
    # the _p form: the same values, plus the partial maxima of [dG | dU]
    # (every one of the 256 parts written, the largest = max |gGU|); a
    # non-finite element counts as 0, as in the GEMMs' own maxima
    gGUp = up(fh, g0) if beta else fh.DeviceArray((2 * rows * H,))
    xp = up(fh, np.full(256, np.nan, np.float32))
    gx = g.copy()
    gx[rows * H // 2] = np.inf
    fh.call("swiglu_gu_bwd_p", gGUp, beta, up(fh, gx), up(fh, GU), rows, H, xp)
    gotp = gGUp.numpy()
    fin = np.isfinite(gotp)
    np.testing.assert_array_equal(gotp[fin], got.ravel()[fin])
    parts = xp.numpy()
    assert np.isfinite(parts).all() and parts.max() == np.abs(gotp[fin]).max()


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,H", [(8192, 768, 2048), (4096, 1024, 2048), (256, 64, 128), (300, 96, 100)])
def test_matmulT_fwd_swiglu_equals_gemm_then_swiglu(fh, M, K, H):
    """The gate/up projection with its SwiGLU formed in the GEMM epilogue
    (8192x768x2048: 512 tiles of 256x256; 4096x1024x2048: 256) stores the
    bits of matmulT followed by the [G | U] SwiGLU pass; other shapes run
    that pair."""
    rs = np.random.default_rng(M + K + H)
    X = rs.standard_normal(M * K).astype(np.float32)
    W = (rs.standard_normal(2 * H * K) * 0.05).astype(np.float32)
    dX, dW = up(fh, X), up(fh, W)
    O, GU = fh.DeviceArray((M * H,)), fh.DeviceArray((M * 2 * H,))
    fh.call("matmulT_fwd_swiglu", O, GU, dX, dW, M, K, H)
    Or, GUr = fh.DeviceArray((M * H,)), fh.DeviceArray((M * 2 * H,))
    fh.call("matmulT_fwd", GUr, dX, dW, M, K, 2 * H)
    fh.call("swiglu_gu_fwd", Or, GUr, M, H)
    np.testing.assert_array_equal(GU.numpy(), GUr.numpy())
    np.testing.assert_array_equal(O.numpy(), Or.numpy())
    rows = rs.integers(0, M, 4)
    ref = X.reshape(M, K)[rows].astype(np.float64) @ W.reshape(2 * H, K).T.astype(np.float64)
    assert rel_l2(GU.numpy().reshape(M, 2 * H)[rows].ravel(), ref.ravel()) < 2e-6


# ───────────────────────── embedLookup (tensor.js:85-99) ─────────────────────────
def embed_plan(fh, ids, V):
    import ctypes
    T = len(ids)
    ids = np.ascontiguousarray(ids, np.int32)
    perm = np.empty(T, np.int32)
    seg_start = np.empty(T + 1, np.int32)
    seg_id = np.empty(max(T, 1), np.int32)
    ns = ctypes.c_int()
    fh.check(fh.lib.fg_embed_plan(ids.ctypes.data, T, V, perm.ctypes.data, seg_start.ctypes.data,
                                  seg_id.ctypes.data, ctypes.byref(ns)), "fg_embed_plan")
    n = ns.value
    return perm, seg_start[:n + 1].copy(), seg_id[:n].copy(), n


@pytest.mark.gpu
@pytest.mark.parametrize("T,V,D", [(3, 4, 3), (256, 31, 64), (8192, 32000, 768), (4096, 128256, 64), (100, 50, 1028),
                                   (1, 1, 1), (5, 1, 4)])
def test_embed(fh, T, V, D):
    rng = oracle.RNG(8)
    W, g = rng.normal_f32(V * D), rng.normal_f32(T * D)
    ids = rng.ints(T, min(V, 50))  # many duplicates
    gW0 = rng.normal_f32(V * D, 0.1)
    X_ref = oracle.embed_fwd(W, ids, D)
    gW_ref = oracle.embed_bwd(g, ids, V, D, gW=gW0)
    X = fh.DeviceArray((T * D,))
    fh.call("embed_fwd", X, up(fh, W), up(fh, ids), T, V, D)
    perm, ss, sid, ns = embed_plan(fh, ids, V)
    gW = up(fh, gW0)
    fh.call("embed_bwd", gW, up(fh, g), up(fh, perm), up(fh, ss), up(fh, sid), ns, D)
    np.testing.assert_array_equal(X.numpy(), X_ref)
    # same sequence of fp32 additions per row as the reference: bit-exact
    np.testing.assert_array_equal(gW.numpy(), gW_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("D", [3, 8])
def test_embed_bad_id_is_nan_and_plan_rejects(fh, D):
    """An id outside [0, V) gives a NaN row (scalar kernel at D = 3, float4
    rows at D = 8, ids -1 and 7 at V = 4)."""
    W = np.arange(4 * D, dtype=np.float32)
    X = fh.DeviceArray((4 * D,))
    fh.call("embed_fwd", X, up(fh, W), up(fh, np.array([0, 7, 1, -1], np.int32)), 4, 4, D)
    x = X.numpy().reshape(4, D)
    assert np.isnan(x[1]).all() and np.isnan(x[3]).all()
    assert np.array_equal(x[0], W[0:D]) and np.array_equal(x[2], W[D:2 * D])
    with pytest.raises(fh.ForgeError, match="outside"):
        embed_plan(fh, np.array([0, 7, 1], np.int32), 4)


# ───────────────────────── sliceCols / add / weightedSum ─────────────────────────
@pytest.mark.gpu
@pytest.mark.parametrize("M,K,off,ln", [(3, 10, 2, 5), (8192, 2304, 768, 768), (256, 128, 96, 32), (1, 1, 0, 1), (4, 7, 6, 1)])
def test_slice(fh, M, K, off, ln):
    rng = oracle.RNG(9)
    X, g, gX0 = rng.normal_f32(M * K), rng.normal_f32(M * ln), rng.normal_f32(M * K)
    Y = fh.DeviceArray((M * ln,))
    fh.call("slice_cols_fwd", Y, up(fh, X), M, K, off, ln)
    np.testing.assert_array_equal(Y.numpy(), oracle.slice_fwd(X, M, K, off, ln))
    gX = up(fh, gX0)
    fh.call("slice_cols_bwd", gX, up(fh, g), M, K, off, ln)
    np.testing.assert_array_equal(gX.numpy(), oracle.slice_bwd(g, M, K, off, ln, gX=gX0))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 7, 8192 * 768])
def test_add_accum(fh, n):
    rng = oracle.RNG(10)
    a, b = rng.normal_f32(n), rng.normal_f32(n)
    Y = fh.DeviceArray((n,))
    fh.call("add_fwd", Y, up(fh, a), up(fh, b), n)
    np.testing.assert_array_equal(Y.numpy(), oracle.add_fwd(a, b))
    fh.call("accum", Y, up(fh, a), n, 1)
    np.testing.assert_array_equal(Y.numpy(), oracle.add_fwd(oracle.add_fwd(a, b), a))
    fh.call("accum", Y, up(fh, b), n, 0)
    np.testing.assert_array_equal(Y.numpy(), b)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [5, 12, 100000])
def test_weighted_sum(fh, n):
    rng = oracle.RNG(11)
    Y, t = rng.normal_f32(n), rng.normal_f32(n)
    out = fh.DeviceArray((1,))
    fh.call("weighted_sum_fwd", out, up(fh, Y), up(fh, t), n)
    exact = float(np.dot(Y.astype(np.float64), t.astype(np.float64)))
    assert abs(out.numpy()[0] - exact) <= 1e-6 * max(1.0, abs(exact))
    # the reference rounds the running sum to fp32 at every step
    assert rel_l2([out.numpy()[0]], [oracle.weighted_sum_fwd(Y, t)]) < 1e-5 * max(1.0, n ** 0.5)
    g0 = np.array([1.5], np.float32)
    gY = fh.DeviceArray((n,))
    fh.call("weighted_sum_bwd", gY, up(fh, g0), up(fh, t), n, 0)
    np.testing.assert_array_equal(gY.numpy(), oracle.weighted_sum_bwd(1.5, t))


# ───────────────────────── causalAttn (tensor.js:191-268, 299-376) ─────────────────────────
ATTN = [
    (1, 4, 4, 2, 4),      # gradient-check shape (I-33d)
    (1, 6, 4, 2, 8),      # I-70 shape
    (8, 32, 4, 2, 16),    # forge-train demo shape (scalar kernels)
    (2, 100, 4, 2, 64),   # MFMA, ragged T
    (1, 128, 2, 1, 128),  # MFMA dH=128, GQA 2:1
    (2, 256, 4, 4, 32),   # MFMA dH=32
    (1, 300, 16, 4, 64),  # MFMA, GQA 4:1
    (2, 45, 4, 2, 80),    # head sizes without an MFMA kernel: the 96 kernels on head-padded copies
    (1, 70, 3, 3, 96),    # the dH 96 kernels
    (2, 130, 8, 2, 96),   # GQA 4:1, two query blocks
    (1, 300, 6, 3, 96),   # GQA 2:1, ragged last block
    (2, 50, 4, 2, 112),   # padded to the 128 kernels
    (1, 200, 4, 4, 48),   # padded to the 64 kernels
    (2, 64, 2, 1, 40),
    (1, 33, 2, 1, 256),   # head sizes above 128: per-head GEMM launches over a T x T workspace
    (1, 40, 2, 1, 130),   # ragged head size and row strides (the GEMMs' checked loads)
    (2, 70, 4, 2, 160),   # GQA 2:1: the kv gradients summed over the group in head order
    (1, 24, 2, 1, 300),   # above the old 256 limit
    (2, 37, 3, 3, 512),
    (2, 30, 2, 4, 144),   # nH < nKV: kv heads 2 and 3 get zero gradients
    (2, 1, 2, 1, 192),    # one position per sequence
    (2, 40, 2, 4, 80),    # nH < nKV at a padded size: padded MFMA forward, scalar backward
    (1, 50, 2, 4, 16),    # nH < nKV: kv heads 2 and 3 have no query head (zero gradients)
    (2, 40, 2, 4, 64),    # nH < nKV with the MFMA forward, scalar backward
    (3, 1, 4, 2, 64),     # one position per sequence (MFMA kernels, a single causal pair)
    (2, 1, 2, 1, 16),     # one position, scalar kernels
    (1, 33, 4, 4, 64),    # one query block and one position past it
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,nH,nKV,dH", ATTN)
def test_attention_vs_oracle(fh, B, T, nH, nKV, dH):
    rng = oracle.RNG(5)
    Q = rng.normal_f32(B * T * nH * dH)
    K = rng.normal_f32(B * T * nKV * dH)
    V = rng.normal_f32(B * T * nKV * dH)
    g = rng.normal_f32(B * T * nH * dH)
    O_ref, P = oracle.attn_fwd(Q, K, V, B, T, nH, nKV, dH)
    gQ_ref, gK_ref, gV_ref = oracle.attn_bwd(g, P, Q, K, V, B, T, nH, nKV, dH)
    dQ_, dK_, dV_ = up(fh, Q), up(fh, K), up(fh, V)
    O, lse = fh.DeviceArray((B * T * nH * dH,)), fh.DeviceArray((B * nH * T,))
    fh.call("attn_fwd", O, lse, dQ_, dK_, dV_, B, T, nH, nKV, dH)
    gQ, gK, gV = fh.DeviceArray(Q.shape), fh.DeviceArray(K.shape), fh.DeviceArray(V.shape)
    fh.call("attn_bwd", gQ, 0, gK, 0, gV, 0, up(fh, g), dQ_, dK_, dV_, O, lse, B, T, nH, nKV, dH)
    assert rel_l2(O.numpy(), O_ref) < TOL_FWD
    if T == 1:
        # one key per query: P = 1, so dS = dP - rowsum(dO*O) = 0 and dQ = dK = 0
        # exactly; both sides hold only rounding noise (|dS| ~ 1e-7 of |dP| ~ 10)
        assert np.max(np.abs(gQ.numpy())) < 1e-5 and np.max(np.abs(gK.numpy())) < 1e-5
        assert np.max(np.abs(gQ_ref)) < 1e-5 and np.max(np.abs(gK_ref)) < 1e-5
        assert max_rel(gV.numpy(), gV_ref) < TOL_GRAD
        return
    assert max_rel(gQ.numpy(), gQ_ref) < TOL_GRAD
    assert max_rel(gK.numpy(), gK_ref) < TOL_GRAD
    assert max_rel(gV.numpy(), gV_ref) < TOL_GRAD
    # accumulate mode adds onto existing gradients
    fh.call("attn_bwd", gQ, 1, gK, 1, gV, 1, up(fh, g), dQ_, dK_, dV_, O, lse, B, T, nH, nKV, dH)
    assert max_rel(gQ.numpy(), 2.0 * gQ_ref.astype(np.float64)) < TOL_GRAD
    assert max_rel(gK.numpy(), 2.0 * gK_ref.astype(np.float64)) < TOL_GRAD
    assert max_rel(gV.numpy(), 2.0 * gV_ref.astype(np.float64)) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,nH,nKV,dH", [(2, 100, 4, 2, 64), (1, 300, 16, 4, 64), (1, 128, 2, 1, 128),
                                            (1, 200, 4, 2, 96)])
def test_attention_bwd_recompute_path_vs_oracle(fh, B, T, nH, nKV, dH):
    """With the stored-dS limit at 0 the MFMA backward recomputes S and dP
    for dQ (the path long sequences take): against the oracle, fresh and
    accumulating, and within fp32 rounding of the stored-dS path."""
    rng = oracle.RNG(7)
    Q = rng.normal_f32(B * T * nH * dH)
    K = rng.normal_f32(B * T * nKV * dH)
    V = rng.normal_f32(B * T * nKV * dH)
    g = rng.normal_f32(B * T * nH * dH)
    _, P = oracle.attn_fwd(Q, K, V, B, T, nH, nKV, dH)
    refs = oracle.attn_bwd(g, P, Q, K, V, B, T, nH, nKV, dH)
    dQ_, dK_, dV_, dg = up(fh, Q), up(fh, K), up(fh, V), up(fh, g)
    O, lse = fh.DeviceArray((B * T * nH * dH,)), fh.DeviceArray((B * nH * T,))
    fh.call("attn_fwd", O, lse, dQ_, dK_, dV_, B, T, nH, nKV, dH)
    outs = {}
    try:
        for limit in (0, 8 << 30):
            fh.call("attn_set_ds_limit", limit)
            gs = [fh.DeviceArray(Q.shape), fh.DeviceArray(K.shape), fh.DeviceArray(V.shape)]
            fh.call("attn_bwd", gs[0], 0, gs[1], 0, gs[2], 0, dg, dQ_, dK_, dV_, O, lse, B, T, nH, nKV, dH)
            for got, ref in zip(gs, refs):
                assert max_rel(got.numpy(), ref) < TOL_GRAD
            fh.call("attn_bwd", gs[0], 1, gs[1], 1, gs[2], 1, dg, dQ_, dK_, dV_, O, lse, B, T, nH, nKV, dH)
            for got, ref in zip(gs, refs):
                assert max_rel(got.numpy(), 2.0 * ref.astype(np.float64)) < TOL_GRAD
            outs[limit] = [x.numpy() for x in gs]
    finally:
        fh.call("attn_set_ds_limit", 8 << 30)
    for a, b in zip(outs[0], outs[8 << 30]):
        assert max_rel(a, b) < 1e-5


@pytest.mark.gpu
def test_attention_rejects_unsupported_shapes(fh):
    """Shapes the kernels do not cover fail on the host with a message, and
    nothing is queued: head maps reaching past nKV, and the fused-qkv
    backward with kv heads that no query head uses."""
    x = fh.DeviceArray((4096,))
    with pytest.raises(fh.ForgeError, match="maps to kv head"):
        fh.call("attn_fwd", x, x, x, x, x, 1, 2, 6, 4, 8)
    with pytest.raises(fh.ForgeError, match="nH=2 < nKV=4"):
        fh.call("attn_bwd_qkv", x, x, x, x, x, 1, 2, 2, 4, 32, x, x, 64, 0, 0)


def _np_attention(Q, K, V, g, T, nH, nKV, dH, heads):
    """fp64 closed form for one sample: O, dQ, dK, dV restricted to `heads`."""
    group = max(1, nH // nKV)
    Q = Q.reshape(T, nH, dH).astype(np.float64)
    K = K.reshape(T, nKV, dH).astype(np.float64)
    V = V.reshape(T, nKV, dH).astype(np.float64)
    g = g.reshape(T, nH, dH).astype(np.float64)
    mask = np.triu(np.ones((T, T), bool), 1)
    out = {}
    for h in heads:
        kv = h // group
        S = Q[:, h] @ K[:, kv].T / np.sqrt(dH)
        S[mask] = -np.inf
        S -= S.max(1, keepdims=True)
        P = np.exp(S)
        P /= P.sum(1, keepdims=True)
        O = P @ V[:, kv]
        dP = g[:, h] @ V[:, kv].T
        dS = P * (dP - (dP * P).sum(1, keepdims=True))
        out[h] = (O, dS @ K[:, kv] / np.sqrt(dH), dS.T @ Q[:, h] / np.sqrt(dH), P.T @ g[:, h])
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,nH,nKV,dH,kvh,samples", [
    (8, 2048, 16, 4, 64, 1, (0, 7)),    # the isolated attention config
    (8, 1024, 12, 12, 64, 5, (0, 7)),   # the 125M training shape
    (1, 4096, 32, 8, 128, 3, (0,)),     # the Llama-3-8B-shaped slice
    (4, 2048, 32, 8, 96, 6, (0, 3)),    # dH 96 (Phi-3-mini's head size), GQA 4:1
])
def test_attention_full_size_closed_form(fh, B, T, nH, nKV, dH, kvh, samples):
    """Full-size launches checked against the fp64 closed form on the given
    samples, for every query head of one kv head's group."""
    rs = np.random.default_rng(7)
    Q = rs.standard_normal(B * T * nH * dH).astype(np.float32)
    K = rs.standard_normal(B * T * nKV * dH).astype(np.float32)
    V = rs.standard_normal(B * T * nKV * dH).astype(np.float32)
    g = rs.standard_normal(B * T * nH * dH).astype(np.float32)
    dQ_, dK_, dV_ = up(fh, Q), up(fh, K), up(fh, V)
    O, lse = fh.DeviceArray((B * T * nH * dH,)), fh.DeviceArray((B * nH * T,))
    fh.call("attn_fwd", O, lse, dQ_, dK_, dV_, B, T, nH, nKV, dH)
    gQ, gK, gV = fh.DeviceArray(Q.shape), fh.DeviceArray(K.shape), fh.DeviceArray(V.shape)
    fh.call("attn_bwd", gQ, 0, gK, 0, gV, 0, up(fh, g), dQ_, dK_, dV_, O, lse, B, T, nH, nKV, dH)
    On, gQn, gKn, gVn = O.numpy(), gQ.numpy(), gK.numpy(), gV.numpy()
    group = nH // nKV
    heads = list(range(kvh * group, (kvh + 1) * group))
    for b in samples:
        sl = slice(b * T * nH * dH, (b + 1) * T * nH * dH)
        skv = slice(b * T * nKV * dH, (b + 1) * T * nKV * dH)
        ref = _np_attention(Q[sl], K[skv], V[skv], g[sl], T, nH, nKV, dH, heads)
        Ob = On[sl].reshape(T, nH, dH)
        gQb = gQn[sl].reshape(T, nH, dH)
        gKb = gKn[skv].reshape(T, nKV, dH)
        gVb = gVn[skv].reshape(T, nKV, dH)
        dk = sum(ref[h][2] for h in heads)
        dv = sum(ref[h][3] for h in heads)
        for h in heads:
            assert rel_l2(Ob[:, h], ref[h][0]) < TOL_FWD
            assert max_rel(gQb[:, h], ref[h][1]) < TOL_GRAD
        assert max_rel(gKb[:, kvh], dk) < TOL_GRAD
        assert max_rel(gVb[:, kvh], dv) < TOL_GRAD


# ───────────────────────── Adam (autograd.js:214-244) ─────────────────────────
def _gpu_adam(fh, ps, gs, ms, vs, t, lr, b1, b2, eps, wd, clip, total):
    dev = [(up(fh, p), up(fh, g), up(fh, m), up(fh, v)) for p, g, m, v in zip(ps, gs, ms, vs)]
    stats = fh.DeviceArray((2,), np.float64)
    tt = min(t / total, 1.0)
    lr_t = lr * 0.5 * (1 + np.cos(np.pi * tt))
    fh.adam_step(dev, lr_t, b1, b2, eps, wd, clip, 1 - b1 ** t, 1 - b2 ** t, stats)
    return [(d[0].numpy(), d[2].numpy(), d[3].numpy()) for d in dev], stats.numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("sizes,wd,clip,t", [([1], 0.0, 1.0, 1), ([3, 1000, 77], 0.01, 1.0, 1),
                                              ([4096, 5], 0.01, 100.0, 3), ([1 << 20], 0.0, 1.0, 1)])
def test_adam_vs_oracle(fh, sizes, wd, clip, t):
    rng = oracle.RNG(12)
    ps = [rng.normal_f32(n) for n in sizes]
    gs = [rng.normal_f32(n) for n in sizes]
    ms = [rng.normal_f32(n, 0.01) if t > 1 else np.zeros(n, np.float32) for n in sizes]
    vs = [np.abs(rng.normal_f32(n, 0.01)) if t > 1 else np.zeros(n, np.float32) for n in sizes]
    ref_p = [p.copy() for p in ps]
    ref_m = [m.copy() for m in ms]
    ref_v = [v.copy() for v in vs]
    info = oracle.adam_step(ref_p, gs, ref_m, ref_v, t, lr=3e-4, wd=wd, clip=clip, total=1000)
    got, stats = _gpu_adam(fh, ps, gs, ms, vs, t, 3e-4, 0.9, 0.999, 1e-8, wd, clip, 1000)
    assert abs(stats[0] - info["gnorm"]) <= 1e-12 * info["gnorm"]
    assert abs(stats[1] - info["scale"]) <= 1e-12
    for (p, m, v), rp, rm, rv in zip(got, ref_p, ref_m, ref_v):
        assert rel_l2(p, rp) < TOL_ADAM and rel_l2(m, rm) < TOL_ADAM and rel_l2(v, rv) < TOL_ADAM
        # fp64 arithmetic in the reference's order without contraction
        np.testing.assert_array_equal(p, rp)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 2, 7, 100, 1000, 9999])
def test_adam_bit_exact_over_steps_and_edge_values(fh, t):
    """Parameters and moments bit-identical to the oracle at early and late
    steps (bias corrections 1 - b^t from 0.1 down to 1), with moments holding
    signed zeros, fp32 denormals and large values: the bias-corrected moments
    are divided through their reciprocals on the device."""
    rng = oracle.RNG(40 + t)
    n = 1 << 16
    p = rng.normal_f32(n)
    g = rng.normal_f32(n)
    m = rng.normal_f32(n, 0.01)
    v = np.abs(rng.normal_f32(n, 0.01))
    special = np.array([0.0, -0.0, 1e-45, -1e-45, 1.2e-38, -3e-39, 1e30, -1e30, 3e38, 1.0], np.float32)
    k = len(special)
    m[:k] = special
    v[:k] = np.abs(special)
    p[k:2 * k] = special        # signed-zero parameters meet zero updates
    m[k:2 * k] = -0.0
    g[k:2 * k] = -0.0
    v[k:2 * k] = 0.0
    g[2 * k:3 * k] = 0.0
    m[2 * k:3 * k] = special
    ref_p, ref_m, ref_v = p.copy(), m.copy(), v.copy()
    oracle.adam_step([ref_p], [g], [ref_m], [ref_v], t, lr=3e-4, wd=0.01, clip=1e30, total=10000)
    got, _ = _gpu_adam(fh, [p], [g], [m], [v], t, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1e30, 10000)
    gp, gm, gv = got[0]
    np.testing.assert_array_equal(gp.view(np.uint32), ref_p.view(np.uint32))
    np.testing.assert_array_equal(gm.view(np.uint32), ref_m.view(np.uint32))
    np.testing.assert_array_equal(gv.view(np.uint32), ref_v.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("b1,b2", [(1.0, 0.999), (0.9, 1.0)])
def test_adam_unit_beta_divides_by_zero_like_the_reference(fh, b1, b2):
    """b1 or b2 = 1 makes a bias correction 1 - b^t zero, with no finite
    reciprocal.  The by-value entry point rejects it; through a device
    schedule (the recorded-step path, whose values the host writes before
    each replay) the update divides, and parameters and moments agree with
    the oracle bit for bit where finite and are NaN at the same places."""
    rng = oracle.RNG(77)
    n = 4096
    p, g = rng.normal_f32(n), rng.normal_f32(n)
    m, v = rng.normal_f32(n, 0.01), np.abs(rng.normal_f32(n, 0.01))
    m[:4] = [0.0, -0.0, 1.0, -1.0]
    v[:4] = [0.0, 0.0, 1.0, 1.0]
    g[:2] = 0.0
    t, lr, total = 3, 3e-4, 1000
    ref_p, ref_m, ref_v = p.copy(), m.copy(), v.copy()
    oracle.adam_step([ref_p], [g], [ref_m], [ref_v], t, lr=lr, b1=b1, b2=b2, wd=0.0, clip=1e30, total=total)
    assert not np.isfinite(ref_p).all()  # the degenerate division is exercised
    dev = [(up(fh, p), up(fh, g), up(fh, m), up(fh, v))]
    with pytest.raises(fh.ForgeError, match="bias corrections must be positive"):
        fh.adam_step(dev, lr, b1, b2, 1e-8, 0.0, 1e30, 1 - b1 ** t, 1 - b2 ** t)
    lr_t = lr * 0.5 * (1 + np.cos(np.pi * min(t / total, 1.0)))
    sched = up(fh, np.array([lr_t, 1 - b1 ** t, 1 - b2 ** t], np.float64))
    arr = (fh.AdamTensor * 1)(fh.AdamTensor(dev[0][0].ptr, dev[0][1].ptr, dev[0][2].ptr, dev[0][3].ptr, n))
    fh.check(fh.lib.fg_adam_step_sched(ctypes.cast(arr, ctypes.c_void_p), 1, ctypes.c_void_p(sched.ptr), b1, b2,
                                       1e-8, 0.0, 1e30, None), "fg_adam_step_sched")
    for d, r in zip((dev[0][0], dev[0][2], dev[0][3]), (ref_p, ref_m, ref_v)):
        a = d.numpy()
        assert np.array_equal(np.isnan(a), np.isnan(r))
        fin = ~np.isnan(r)
        np.testing.assert_array_equal(a[fin].view(np.uint32), r[fin].view(np.uint32))


@pytest.mark.gpu
def test_adam_known_answer(fh):
    """l2-l6.test.js:205-211: lr 0.1, g=1, total 100 -> dw = 0.1*(1+cos(pi/100))/2/(1+1e-8)."""
    got, _ = _gpu_adam(fh, [np.ones(1, np.float32)], [np.ones(1, np.float32)], [np.zeros(1, np.float32)],
                       [np.zeros(1, np.float32)], 1, 0.1, 0.9, 0.999, 1e-8, 0.0, 1.0, 100)
    dw = 1.0 - float(got[0][0][0])
    want = 0.1 * 0.5 * (1 + np.cos(np.pi / 100)) / (1 + 1e-8)
    assert abs(dw - want) < 1e-7 and abs(1.0 - got[0][0][0] - 0.1) < 1e-4
