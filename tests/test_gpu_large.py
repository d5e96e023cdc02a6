"""Full-size checks of the isolated-op and Llama-3-8B-slice shapes.

* Adam over 2^26 parameters (the isolated Adam configuration) against the
  oracle over every element, through the tensor-list and the plan entry
  points (autograd.js:214-244);
* Adam over one tensor of 128256 x 4096 elements (the Llama-3-8B slice's LM
  head, 2.1 GB per array) on chunks at the start, across 2^31 bytes and at
  the end, bit for bit;
* crossEntropyMean at V = 128256 over 4096 rows (2.1 GB of logits) against
  an fp64 closed form for every row and the oracle on sampled rows
  (tensor.js:393-417);
* the matmulT GEMMs at the slice's widest shapes (LM head 4096 -> 128256,
  gate/up 4096 -> 2 x 14336, down 14336 -> 4096): forward, input gradient and
  the grouped weight gradient on sampled rows and columns against fp64.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from util import TOL_ADAM, TOL_FWD, TOL_GRAD, max_rel, rel_l2


def up(fh, a):
    return fh.DeviceArray.from_numpy(np.ascontiguousarray(a))


def _tensor_list(fh, dev):
    arr = (fh.AdamTensor * len(dev))()
    for i, (p, g, m, v) in enumerate(dev):
        arr[i] = fh.AdamTensor(p.ptr, g.ptr, m.ptr, v.ptr, int(np.prod(p.shape)))
    return arr


def _lr(lr, t, total):
    return lr * 0.5 * (1 + math.cos(math.pi * min(t / total, 1.0)))


@pytest.mark.gpu
def test_adam_2pow26_params_vs_oracle(fh):
    """The isolated Adam configuration: 2^26 params (three tensors), p and g
    ~ N(0,1), lr 3e-4, betas (0.9, 0.999), eps 1e-8, clip 1 (gnorm ~ 8192,
    so every gradient is scaled), wd 0.  The plan entry point gives the same
    bits as the tensor-list one."""
    sizes = [1 << 25, (1 << 24) + 3, (1 << 24) - 3]
    assert sum(sizes) == 1 << 26
    rs = np.random.default_rng(26)
    ps = [rs.standard_normal(n, dtype=np.float32) for n in sizes]
    gs = [rs.standard_normal(n, dtype=np.float32) for n in sizes]
    rp, rm, rv = [p.copy() for p in ps], [np.zeros(n, np.float32) for n in sizes], [np.zeros(n, np.float32) for n in sizes]
    info = oracle.adam_step(rp, gs, rm, rv, 1, lr=3e-4, wd=0.0, clip=1.0, total=1000)
    lr_t = _lr(3e-4, 1, 1000)
    outs = []
    for use_plan in (False, True):
        dev = [(up(fh, p), up(fh, g), fh.DeviceArray.zeros(p.shape), fh.DeviceArray.zeros(p.shape))
               for p, g in zip(ps, gs)]
        stats = fh.DeviceArray((2,), np.float64)
        arr = _tensor_list(fh, dev)
        if use_plan:
            plan = ctypes.c_void_p()
            fh.check(fh.lib.fg_adam_plan_create(ctypes.cast(arr, ctypes.c_void_p), len(dev), ctypes.byref(plan)),
                     "fg_adam_plan_create")
            match = ctypes.c_int(-1)
            fh.check(fh.lib.fg_adam_plan_matches(plan, ctypes.cast(arr, ctypes.c_void_p), len(dev),
                                                 ctypes.byref(match)), "fg_adam_plan_matches")
            assert match.value == 1
            fh.check(fh.lib.fg_adam_step_plan(plan, lr_t, 0.9, 0.999, 1e-8, 0.0, 1.0, 1 - 0.9, 1 - 0.999,
                                              ctypes.c_void_p(stats.ptr)), "fg_adam_step_plan")
            fh.check(fh.lib.fg_adam_plan_destroy(plan), "fg_adam_plan_destroy")
        else:
            fh.adam_step(dev, lr_t, 0.9, 0.999, 1e-8, 0.0, 1.0, 1 - 0.9, 1 - 0.999, stats)
        outs.append(([d[0].numpy() for d in dev], [d[2].numpy() for d in dev], [d[3].numpy() for d in dev],
                     stats.numpy()))
    (p0, m0, v0, s0), (p1, m1, v1, s1) = outs
    assert abs(s0[0] - info["gnorm"]) <= 1e-12 * info["gnorm"] and abs(s0[1] - info["scale"]) <= 1e-12 * info["scale"]
    for a, b in [(p0, rp), (m0, rm), (v0, rv)]:
        for x, y in zip(a, b):
            assert rel_l2(x, y) < TOL_ADAM
    for a, b in [(p0, p1), (m0, m1), (v0, v1), ([s0], [s1])]:
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)


@pytest.mark.gpu
def test_adam_plan_matches_only_its_own_list(fh):
    a = [(up(fh, np.ones(10, np.float32)),) * 4]
    b = [(up(fh, np.ones(10, np.float32)),) * 4]
    la, lb = _tensor_list(fh, a), _tensor_list(fh, b)
    plan = ctypes.c_void_p()
    fh.check(fh.lib.fg_adam_plan_create(ctypes.cast(la, ctypes.c_void_p), 1, ctypes.byref(plan)), "create")
    res = []
    for lst in (la, lb):
        m = ctypes.c_int(-1)
        fh.check(fh.lib.fg_adam_plan_matches(plan, ctypes.cast(lst, ctypes.c_void_p), 1, ctypes.byref(m)), "matches")
        res.append(m.value)
    fh.check(fh.lib.fg_adam_plan_destroy(plan), "destroy")
    assert res == [1, 0]


@pytest.mark.gpu
def test_adam_lm_head_tensor_over_2gib(fh):
    """One tensor of 128256 x 4096 fp32 (2.1 GB per array): t = 2 with
    moments, wd 0.01 and no clipping (scale exactly 1, so every chunk is
    independent of the global norm's summation order), checked bit for bit
    against the oracle on chunks at the start, around element 2^29 (byte
    2^31) and at the end; the gradient norm against an fp64 sum."""
    n = 128256 * 4096
    rs = np.random.default_rng(8)
    p = rs.standard_normal(n, dtype=np.float32)
    g = rs.standard_normal(n, dtype=np.float32)
    m = (rs.standard_normal(n, dtype=np.float32) * np.float32(0.01))
    v = np.abs(rs.standard_normal(n, dtype=np.float32)) * np.float32(0.01)
    dev = [(up(fh, p), up(fh, g), up(fh, m), up(fh, v))]
    stats = fh.DeviceArray((2,), np.float64)
    t = 2
    fh.adam_step(dev, _lr(3e-4, t, 1000), 0.9, 0.999, 1e-8, 0.01, 1e30, 1 - 0.9 ** t, 1 - 0.999 ** t, stats)
    gp, gm, gv = dev[0][0].numpy(), dev[0][2].numpy(), dev[0][3].numpy()
    st = stats.numpy()
    gn = float(np.sqrt(np.sum(np.square(g, dtype=np.float64))))
    assert abs(st[0] - gn) <= 1e-10 * gn and st[1] == 1.0
    L = 3 * 8192 + 17
    for start in (0, (1 << 29) - L // 2, n - L):
        sl = slice(start, start + L)
        rp, rm, rv = [p[sl].copy()], [m[sl].copy()], [v[sl].copy()]
        oracle.adam_step(rp, [g[sl].copy()], rm, rv, t, lr=3e-4, wd=0.01, clip=1e30, total=1000)
        np.testing.assert_array_equal(gp[sl], rp[0])
        np.testing.assert_array_equal(gm[sl], rm[0])
        np.testing.assert_array_equal(gv[sl], rv[0])


@pytest.mark.gpu
def test_ce_llama8b_vocab_over_2gib(fh):
    """Logits [4096 x 128256] ~ N(0, 2^2) (2.1 GB): the fused training loss
    (forward + seed-1 backward) equals the separate forward and backward bit
    for bit; lse of every row against an fp64 closed form; the loss against
    the fp64 mean; the gradient of rows at the start, middle and end against
    the oracle."""
    rows, V = 4096, 128256
    rs = np.random.default_rng(3)
    logits = rs.standard_normal(rows * V, dtype=np.float32) * np.float32(2.0)
    tg = rs.integers(0, V, rows).astype(np.int32)
    dl, dt = up(fh, logits), up(fh, tg)
    loss, lse, grad = fh.DeviceArray((1,)), fh.DeviceArray((rows,)), fh.DeviceArray((rows * V,))
    fh.call("ce_fwd_bwd", loss, lse, grad, dl, dt, rows, V)
    loss2, lse2, grad2 = fh.DeviceArray((1,)), fh.DeviceArray((rows,)), fh.DeviceArray((rows * V,))
    one = up(fh, np.ones(1, np.float32))
    fh.call("ce_fwd", loss2, lse2, dl, dt, rows, V)
    fh.call("ce_bwd", grad2, dl, lse2, dt, one, rows, V, 0)
    g1 = grad.numpy()
    np.testing.assert_array_equal(loss.numpy(), loss2.numpy())
    np.testing.assert_array_equal(lse.numpy(), lse2.numpy())
    np.testing.assert_array_equal(g1, grad2.numpy())
    del grad2
    X = logits.reshape(rows, V)
    ref_lse = np.empty(rows)
    for r0 in range(0, rows, 256):
        blk = X[r0:r0 + 256].astype(np.float64)
        mx = blk.max(1, keepdims=True)
        ref_lse[r0:r0 + 256] = (mx + np.log(np.exp(blk - mx).sum(1, keepdims=True)))[:, 0]
    assert rel_l2(lse.numpy(), ref_lse) < TOL_FWD
    ref_loss = float(np.mean(ref_lse - X[np.arange(rows), tg].astype(np.float64)))
    assert abs(float(loss.numpy()[0]) - ref_loss) <= 1e-6 * abs(ref_loss)
    sample = np.array([0, 1, 2047, 2048, 4094, 4095])
    sub = np.ascontiguousarray(X[sample])
    _, probs = oracle.ce_fwd(sub.ravel(), tg[sample], len(sample), V)
    ref_g = oracle.ce_bwd(len(sample) / rows, probs, tg[sample], len(sample), V)
    got = g1.reshape(rows, V)[sample].ravel()
    assert max_rel(got, ref_g) < TOL_GRAD and rel_l2(got, ref_g) < TOL_FWD


def _gemm_samples(M, K, N, seed):
    rs = np.random.default_rng(seed)
    return np.sort(rs.choice(M, 40, replace=False)), np.sort(rs.choice(N, 40, replace=False))


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(4096, 4096, 128256), (4096, 4096, 28672), (4096, 14336, 4096)])
def test_matmulT_llama8b_shapes_sampled_vs_fp64(fh, M, K, N):
    """Y = X·Wᵀ, gX = gY·W and (grouped launch) gW = gYᵀ·X at the slice's
    widest GEMMs; 40 x 40 sampled outputs of each against fp64."""
    rs = np.random.default_rng(M + K + N)
    X = rs.standard_normal((M, K), dtype=np.float32)
    W = rs.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    gY = rs.standard_normal((M, N), dtype=np.float32)
    dX, dW, dgY = up(fh, X), up(fh, W), up(fh, gY)
    Y = fh.DeviceArray((M * N,))
    fh.call("matmulT_fwd", Y, dX, dW, M, K, N)
    gX = fh.DeviceArray((M * K,))
    fh.call("matmulT_bwd_x", gX, dgY, dW, M, K, N, 0)
    gW = fh.DeviceArray((N * K,))
    jobs = (fh.WgradJob * 1)(fh.WgradJob(gW.ptr, dgY.ptr, dX.ptr, M, K, N, 0))
    fh.check(fh.lib.fg_matmulT_bwd_w_grouped(ctypes.cast(jobs, ctypes.c_void_p), 1), "fg_matmulT_bwd_w_grouped")
    Yn, gXn, gWn = Y.numpy().reshape(M, N), gX.numpy().reshape(M, K), gW.numpy().reshape(N, K)

    def tol(kred):
        # fp32 accumulation: the error of a sum of kred products grows like
        # sqrt(kred) (2e-6 holds up to 4096 terms; the reference itself adds
        # its kred terms one fp32 rounding at a time)
        return 2e-6 * max(1.0, (kred / 4096) ** 0.5)

    rows, cols = _gemm_samples(M, K, N, 1)
    X64, W64 = X.astype(np.float64), W.astype(np.float64)
    ref = X64[rows] @ W64[cols].T
    assert rel_l2(Yn[np.ix_(rows, cols)], ref) < tol(K)
    kr, kc = _gemm_samples(M, K, K, 2)
    ref = gY[kr].astype(np.float64) @ W64[:, kc]
    assert rel_l2(gXn[np.ix_(kr, kc)], ref) < tol(N)
    nr, kc2 = _gemm_samples(N, K, K, 3)
    ref = gY[:, nr].astype(np.float64).T @ X64[:, kc2]
    assert rel_l2(gWn[np.ix_(nr, kc2)], ref) < tol(M)


@pytest.mark.gpu
def test_matmulT_fwd_swiglu_llama8b_shape_sampled_vs_fp64(fh):
    """The gate/up projection with its SwiGLU epilogue at the slice's shape
    (M 4096, K 4096, H 14336: [G | U] = X·[Wg; Wu]ᵀ, O = silu(G)·U) on 40
    sampled rows: G and U at 40 sampled columns each against fp64 (the GEMM
    tolerance of a 4096-term sum), and O at those columns against the
    oracle's swigluRows of the GPU's own G and U and against the fp64
    closed form of the fp64 G and U (forward tolerance)."""
    M, K, H = 4096, 4096, 14336
    rs = np.random.default_rng(8)
    X = rs.standard_normal((M, K), dtype=np.float32)
    W = rs.standard_normal((2 * H, K), dtype=np.float32) * np.float32(0.02)
    dX, dW = up(fh, X), up(fh, W)
    O, GU = fh.DeviceArray((M * H,)), fh.DeviceArray((M * 2 * H,))
    fh.call("matmulT_fwd_swiglu", O, GU, dX, dW, M, K, H)
    rows = np.sort(rs.choice(M, 40, replace=False))
    cols = np.sort(rs.choice(H, 40, replace=False))
    On, GUn = O.numpy().reshape(M, H), GU.numpy().reshape(M, 2 * H)
    X64, W64 = X[rows].astype(np.float64), W.astype(np.float64)
    G64 = X64 @ W64[cols].T
    U64 = X64 @ W64[H + cols].T
    Gg, Ug = GUn[np.ix_(rows, cols)], GUn[np.ix_(rows, H + cols)]
    assert rel_l2(Gg, G64) < 2e-6 and rel_l2(Ug, U64) < 2e-6
    Og = On[np.ix_(rows, cols)]
    ref_o, _ = oracle.swiglu_fwd(np.ascontiguousarray(Gg).ravel(), np.ascontiguousarray(Ug).ravel())
    assert rel_l2(Og.ravel(), ref_o) < TOL_FWD
    closed = G64 / (1.0 + np.exp(-G64)) * U64
    assert rel_l2(Og, closed) < TOL_FWD
