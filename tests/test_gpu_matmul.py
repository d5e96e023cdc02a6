"""matmulT forward / input-grad / weight-grad on the GPU (tensor.js:34-53).

Small shapes are checked against the C oracle (the reference's own loop order,
fp32 store per +=); the isolated 2048x1024x4096 case against the fp64 closed
form (numpy), which the oracle matches at the small shapes (test_oracle.py).
"""
import ctypes

import numpy as np
import pytest

import oracle
from util import TOL_FWD, TOL_GRAD, max_rel, rel_l2

SMALL = [(3, 5, 4), (4, 5, 3), (256, 64, 128), (256, 64, 31), (256, 128, 64), (130, 70, 200), (33, 257, 129),
         (1, 1, 1), (1, 768, 5), (7, 1, 9), (2, 3, 1)]


def _run(fh, X, W, g, M, K, N, beta=0, gX0=None, gW0=None):
    DA = fh.DeviceArray
    dX, dW, dg = DA.from_numpy(X), DA.from_numpy(W), DA.from_numpy(g)
    Y = DA((M * N,))
    fh.call("matmulT_fwd", Y, dX, dW, M, K, N)
    gX = DA.from_numpy(gX0) if gX0 is not None else DA((M * K,))
    gW = DA.from_numpy(gW0) if gW0 is not None else DA((N * K,))
    fh.call("matmulT_bwd_x", gX, dg, dW, M, K, N, beta)
    fh.call("matmulT_bwd_w", gW, dg, dX, M, K, N, beta)
    return Y.numpy(), gX.numpy(), gW.numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", SMALL)
def test_matmulT_small_vs_oracle(fh, M, K, N):
    rng = oracle.RNG(2)
    X, W, g = rng.normal_f32(M * K), rng.normal_f32(N * K), rng.normal_f32(M * N)
    Y_ref = oracle.matmulT_fwd(X, W, M, K, N)
    gX_ref, gW_ref = oracle.matmulT_bwd(g, X, W, M, K, N)
    Y, gX, gW = _run(fh, X, W, g, M, K, N)
    assert rel_l2(Y, Y_ref) < TOL_FWD
    assert max_rel(gX, gX_ref) < TOL_GRAD
    assert max_rel(gW, gW_ref) < TOL_GRAD
    # accumulate (beta=1) onto existing gradients, as `grad ??=` then `+=`
    gX0, gW0 = rng.normal_f32(M * K), rng.normal_f32(N * K)
    gX_acc, gW_acc = oracle.matmulT_bwd(g, X, W, M, K, N, gX=gX0, gW=gW0)
    _, gX1, gW1 = _run(fh, X, W, g, M, K, N, beta=1, gX0=gX0, gW0=gW0)
    assert max_rel(gX1, gX_acc) < TOL_GRAD
    assert max_rel(gW1, gW_acc) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(2048, 1024, 4096), (8192, 768, 768), (1024, 2048, 768)])
def test_matmulT_large_vs_closed_form(fh, M, K, N):
    rs = np.random.default_rng(1)
    X = rs.standard_normal((M, K)).astype(np.float32)
    W = rs.standard_normal((N, K)).astype(np.float32)
    g = rs.standard_normal((M, N)).astype(np.float32)
    Y, gX, gW = _run(fh, X.ravel(), W.ravel(), g.ravel(), M, K, N)
    X64, W64, g64 = X.astype(np.float64), W.astype(np.float64), g.astype(np.float64)
    assert rel_l2(Y, X64 @ W64.T) < TOL_FWD
    assert max_rel(gX, g64 @ W64) < TOL_GRAD
    assert max_rel(gW, g64.T @ X64) < TOL_GRAD


# ───── residual fused into the GEMM epilogue (train.js:144-145, 152-153) ─────
@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(5, 7, 3), (33, 2048, 35), (100, 3072, 36), (8192, 768, 768), (8192, 3072, 768)])
def test_matmulT_fwd_resid(fh, M, K, N):
    """R + X·Wᵀ equals matmulT followed by the residual add, bit for bit
    (split-K and unaligned shapes included), and the oracle's add(R, X·Wᵀ)."""
    rng = oracle.RNG(21)
    X, W, R = rng.normal_f32(M * K), rng.normal_f32(N * K), rng.normal_f32(M * N)
    dX, dW, dR = fh.DeviceArray.from_numpy(X), fh.DeviceArray.from_numpy(W), fh.DeviceArray.from_numpy(R)
    Y, P, S = fh.DeviceArray((M * N,)), fh.DeviceArray((M * N,)), fh.DeviceArray((M * N,))
    fh.call("matmulT_fwd_resid", Y, dR, dX, dW, M, K, N)
    fh.call("matmulT_fwd", P, dX, dW, M, K, N)
    fh.call("add_fwd", S, dR, P, M * N)
    np.testing.assert_array_equal(Y.numpy(), S.numpy())
    if M * N * K <= 1 << 22:
        ref = oracle.add_fwd(R, oracle.matmulT_fwd(X, W, M, K, N))
    else:
        ref = R.astype(np.float64) + (X.reshape(M, K).astype(np.float64) @ W.reshape(N, K).T.astype(np.float64)).ravel()
    assert rel_l2(Y.numpy(), ref) < TOL_FWD


# ───── every tile configuration (128x128, 256-wide single-stage, ping-pong) ─────
# (M, K, N) chosen so the forward (NT), input-gradient (NN) and weight-gradient
# (TN) GEMMs between them hit each kernel variant, with full tiles and with
# ragged edges, with and without a K split.
CONFIGS = [(4096, 256, 2048), (4100, 200, 2050), (4096, 2048, 512), (4099, 2049, 300), (2304, 8192, 768),
           (8100, 500, 760),  # 128x192 tiles (16x16 MFMA blocks) with ragged edges, forward and dX
           # 256x256 tiles (64x128 waves, k-step 16) on 256 CUs: forward 256 tiles; forward 17 x 33 ragged
           # tiles with the tail split; dX 16 x 32 tiles; dX 17 x 33 ragged tiles with the tail split
           (4096, 256, 4096), (4100, 300, 8200), (4096, 8192, 256), (4099, 8195, 300),
           # 256x192 tiles with K split in two (768-wide outputs, K >= 2048): forward even and ragged
           (8192, 2048, 768), (8100, 3000, 760),
           # 256x256 tiles over 1-3 k-steps of 16 (the four-stage forward and weight-gradient pipeline's
           # prologue and pair barriers, the two-stage input gradient): forward K 16 / 32 / 40 (ragged),
           # input gradient over 48, weight gradient over 48 and 32
           (4096, 16, 8192), (4096, 32, 8192), (4096, 40, 8192), (4096, 8192, 48), (48, 4096, 8192),
           (32, 8192, 4096)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", CONFIGS)
def test_matmulT_tile_configs_vs_fp64(fh, M, K, N):
    """Against the fp64 product: within the path tolerances, and at fp32 level
    (rel-L2 <= 2e-6; a split that dropped a 2^-16 term would sit near 1e-5)."""
    rs = np.random.default_rng(M + K + N)
    X = rs.standard_normal((M, K)).astype(np.float32)
    W = (rs.standard_normal((N, K)) * 0.05).astype(np.float32)
    g = (rs.standard_normal((M, N)) * 1e-3).astype(np.float32)
    gX0 = rs.standard_normal((M, K)).astype(np.float32) * 1e-3
    gW0 = rs.standard_normal((N, K)).astype(np.float32) * 1e-3
    Y, gX, gW = _run(fh, X.ravel(), W.ravel(), g.ravel(), M, K, N, beta=1, gX0=gX0.ravel(), gW0=gW0.ravel())
    X64, W64, g64 = X.astype(np.float64), W.astype(np.float64), g.astype(np.float64)
    Yr, gXr, gWr = X64 @ W64.T, gX0 + g64 @ W64, gW0 + g64.T @ X64
    for got, ref in [(Y, Yr), (gX, gXr), (gW, gWr)]:
        assert rel_l2(got, ref.ravel()) < 2e-6
        assert max_rel(got, ref.ravel()) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(8192, 768, 2048), (8100, 760, 3000), (8192, 768, 32000)])
def test_matmulT_bwd_x_halves_sum_to_the_input_gradient(fh, M, K, N):
    """Shapes whose input-gradient GEMM splits K in two: the unreduced pieces
    add (fp32, in order) to exactly what fg_matmulT_bwd_x stores."""
    assert fh.lib.fg_matmulT_bwd_x_pieces(M, K, N) == 2
    rs = np.random.default_rng(M + N)
    g = rs.standard_normal(M * N).astype(np.float32)
    W = (rs.standard_normal(N * K) * 0.05).astype(np.float32)
    dg, dW = fh.DeviceArray.from_numpy(g), fh.DeviceArray.from_numpy(W)
    ref, halves = fh.DeviceArray((M * K,)), fh.DeviceArray((2 * M * K,))
    fh.call("matmulT_bwd_x", ref, dg, dW, M, K, N, 0)
    fh.call("matmulT_bwd_x_halves", halves, dg, dW, M, K, N)
    h = halves.numpy()
    np.testing.assert_array_equal(h[:M * K] + h[M * K:], ref.numpy())


@pytest.mark.gpu
def test_matmulT_bwd_x_halves_rejects_unsplit_shapes(fh):
    M, K, N = 512, 256, 384
    assert fh.lib.fg_matmulT_bwd_x_pieces(M, K, N) == 1
    DA = fh.DeviceArray
    with pytest.raises(fh.ForgeError, match="not two"):
        fh.call("matmulT_bwd_x_halves", DA((2 * M * K,)), DA((M * N,)), DA((N * K,)), M, K, N)


def _mantissa_values(rs, shape, bits):
    """Values in [1, 2) with `bits` significant bits (multiples of 2^-(bits-1)), random sign."""
    q = 1 << (bits - 1)
    v = (q + rs.integers(0, q, size=shape)) / q
    return (v * rs.choice([-1.0, 1.0], size=shape)).astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("M,R,N", [(256, 32, 256), (300, 16, 129), (4096, 32, 2048), (8192, 32, 768)])
def test_matmul_exact_sums_use_both_fp16_pieces(fh, M, R, N):
    """Known answers: one operand holds 19-bit mantissas, the other +-1, and the
    contraction length R keeps every partial sum exactly representable, so the
    GEMM must return the exact sum.  Each fp32 value needs both its hi and lo
    fp16 pieces (11 + 8 bits) for this; dropping either product with a +-1
    factor changes the result.  Checked for both operand roles and all three
    layouts (forward, input gradient, weight gradient)."""
    rs = np.random.default_rng(7)
    DA = fh.DeviceArray
    P = _mantissa_values(rs, (M, R), 19)          # precise operand
    S = rs.choice([-1.0, 1.0], size=(N, R)).astype(np.float32)  # sign operand
    exact = (P.astype(np.float64) @ S.T.astype(np.float64)).astype(np.float32)
    assert np.array_equal(exact.astype(np.float64), P.astype(np.float64) @ S.T.astype(np.float64))
    # forward: Y[M,N] = X[M,R] · W[N,R]^T with X precise, then with the roles swapped
    Y = DA((M * N,))
    fh.call("matmulT_fwd", Y, DA.from_numpy(P.ravel()), DA.from_numpy(S.ravel()), M, R, N)
    np.testing.assert_array_equal(Y.numpy(), exact.ravel())
    Yt = DA((N * M,))
    fh.call("matmulT_fwd", Yt, DA.from_numpy(S.ravel()), DA.from_numpy(P.ravel()), N, R, M)
    np.testing.assert_array_equal(Yt.numpy(), exact.T.ravel())
    # input gradient: gX[M,R'] = gY[M,N'] · W[N',R'] with the contraction over N' = R
    gY = P                                        # [M, R] plays gY with N' = R
    Wn = np.ascontiguousarray(S.T)                # [R, N] plays W[N', K'] with K' = N
    gX = DA((M * N,))
    fh.call("matmulT_bwd_x", gX, DA.from_numpy(gY.ravel()), DA.from_numpy(Wn.ravel()), M, N, R, 0)
    np.testing.assert_array_equal(gX.numpy(), exact.ravel())
    # weight gradient: gW[N',K'] = gY[M',N']^T · X[M',K'] with the contraction over M' = R
    gYt = np.ascontiguousarray(P.T)               # [R, M] = gY[M'=R, N'=M]
    Xs = np.ascontiguousarray(S.T)                # [R, N] = X[M'=R, K'=N]
    gW = DA((M * N,))
    fh.call("matmulT_bwd_w", gW, DA.from_numpy(gYt.ravel()), DA.from_numpy(Xs.ravel()), R, N, M, 0)
    np.testing.assert_array_equal(gW.numpy(), exact.ravel())


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(33, 70, 20), (8192, 768, 768), (4096, 2048, 512)])
def test_matmulT_bwd_equals_separate(fh, M, K, N):
    """fg_matmulT_bwd returns what the two separate entry points return, bit
    for bit, fresh and accumulating, and with gX and gW aliased
    (matmulT(X, X)) the weight gradient accumulates onto the input one."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(5)
    X = rs.standard_normal(M * K).astype(np.float32)
    W = rs.standard_normal(N * K).astype(np.float32)
    g = rs.standard_normal(M * N).astype(np.float32)
    gX0 = rs.standard_normal(M * K).astype(np.float32)
    gW0 = rs.standard_normal(N * K).astype(np.float32)
    dX, dW, dg = DA.from_numpy(X), DA.from_numpy(W), DA.from_numpy(g)
    for beta in (0, 1):
        a_x, a_w = DA.from_numpy(gX0), DA.from_numpy(gW0)
        b_x, b_w = DA.from_numpy(gX0), DA.from_numpy(gW0)
        fh.call("matmulT_bwd", a_x, beta, a_w, beta, dg, dX, dW, M, K, N)
        fh.call("matmulT_bwd_x", b_x, dg, dW, M, K, N, beta)
        fh.call("matmulT_bwd_w", b_w, dg, dX, M, K, N, beta)
        np.testing.assert_array_equal(a_x.numpy(), b_x.numpy())
        np.testing.assert_array_equal(a_w.numpy(), b_w.numpy())
    if M == N:  # Y = X·X^T: both gradients land in one buffer
        S = rs.standard_normal(M * K).astype(np.float32)
        dS = DA.from_numpy(S)
        a = DA((M * K,))
        fh.call("matmulT_bwd", a, 0, a, 1, dg, dS, dS, M, K, M)
        b = DA((M * K,))
        fh.call("matmulT_bwd_x", b, dg, dS, M, K, M, 0)
        fh.call("matmulT_bwd_w", b, dg, dS, M, K, M, 1)
        np.testing.assert_array_equal(a.numpy(), b.numpy())


def _grouped(fh, jobs):
    arr = (fh.WgradJob * len(jobs))()
    for i, (gW, gY, X, M, K, N, beta) in enumerate(jobs):
        arr[i] = fh.WgradJob(gW.ptr, gY.ptr, X.ptr, M, K, N, beta)
    fh.check(fh.lib.fg_matmulT_bwd_w_grouped(ctypes.cast(arr, ctypes.c_void_p), len(jobs)),
             "fg_matmulT_bwd_w_grouped")


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_vs_single_and_fp64(fh):
    """The weight gradients of several matmulTs in one grouped launch (full K,
    no split): each job against fg_matmulT_bwd_w on the same inputs (fp32
    rounding differences only: the single launch may split K) and against an
    fp64 product, fresh and accumulating, with ragged shapes (edge tiles) and
    more jobs than one launch table holds."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(9)
    shapes = [(512, 768, 2304), (512, 768, 768), (512, 768, 4096), (512, 2048, 768), (300, 200, 130),
              (64, 36, 8), (1000, 520, 1000)]
    shapes = shapes + [(96, 64, 40 + 8 * i) for i in range(50)]  # 57 jobs: two launch tables
    jobs, refs, singles, outs = [], [], [], []
    for i, (M, K, N) in enumerate(shapes):
        X = rs.standard_normal(M * K).astype(np.float32)
        g = rs.standard_normal(M * N).astype(np.float32)
        beta = i % 2
        gW0 = rs.standard_normal(N * K).astype(np.float32)
        dX, dg = DA.from_numpy(X), DA.from_numpy(g)
        out = DA.from_numpy(gW0)
        single = DA.from_numpy(gW0)
        fh.call("matmulT_bwd_w", single, dg, dX, M, K, N, beta)
        ref = g.astype(np.float64).reshape(M, N).T @ X.astype(np.float64).reshape(M, K)
        if beta:
            ref = ref + gW0.astype(np.float64).reshape(N, K)
        jobs.append((out, dg, dX, M, K, N, beta))
        refs.append(ref.ravel())
        singles.append(single)
        outs.append(out)
    _grouped(fh, jobs)
    for (M, K, N), out, single, ref in zip(shapes, outs, singles, refs):
        got = out.numpy()
        assert rel_l2(got, ref) < 2e-6, (M, K, N, rel_l2(got, ref))
        assert max_rel(got, single.numpy()) < 1e-5, (M, K, N)


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_same_output_in_order(fh):
    """Two jobs on one gW (a weight used twice in one pass: beta 0, then 1)
    inside one job list: the second accumulates onto the first, as two
    single launches would."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(11)
    M, K, N = 512, 768, 1024
    X1, X2 = rs.standard_normal(M * K).astype(np.float32), rs.standard_normal(M * K).astype(np.float32)
    g1, g2 = rs.standard_normal(M * N).astype(np.float32), rs.standard_normal(M * N).astype(np.float32)
    other = DA((N * K,))
    out = DA((N * K,))
    jobs = [(out, DA.from_numpy(g1), DA.from_numpy(X1), M, K, N, 0),
            (other, DA.from_numpy(g2), DA.from_numpy(X1), M, K, N, 0),
            (out, DA.from_numpy(g2), DA.from_numpy(X2), M, K, N, 1)]
    _grouped(fh, jobs)
    ref = (g1.astype(np.float64).reshape(M, N).T @ X1.astype(np.float64).reshape(M, K)
           + g2.astype(np.float64).reshape(M, N).T @ X2.astype(np.float64).reshape(M, K))
    assert rel_l2(out.numpy(), ref.ravel()) < 2e-6
    single = DA((N * K,))
    fh.call("matmulT_bwd_w", single, jobs[0][1], jobs[0][2], M, K, N, 0)
    fh.call("matmulT_bwd_w", single, jobs[2][1], jobs[2][2], M, K, N, 1)
    assert max_rel(out.numpy(), single.numpy()) < 1e-5


# ───── tail split: the last, at most half-full round of one-per-CU tiles is cut along K ─────
# Tile counts below are for 256 CUs (MI355X) and 128x256 ping-pong tiles.
TAIL = [
    (8192, 768, 2304),   # forward 64 x 9 = 576 tiles: 64 tail tiles in 4 pieces (the 125M qkv GEMM)
    (4196, 512, 2048),   # forward 33 x 8 = 264 tiles, ragged rows: 8 tail tiles in 4 pieces
    (1024, 2304, 4096),  # weight gradient 32 x 9 = 288 tiles: 32 tail tiles in 8 pieces
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", TAIL)
def test_matmulT_tail_split_vs_fp64(fh, M, K, N):
    """GEMMs whose last round of tiles is split along K (pieces summed by the
    tail reduction in a fixed order) against the fp64 product at fp32 level,
    accumulating (beta = 1); the residual form equals matmulT + add bit for bit."""
    rs = np.random.default_rng(M + K + N + 1)
    X = rs.standard_normal((M, K)).astype(np.float32)
    W = (rs.standard_normal((N, K)) * 0.05).astype(np.float32)
    g = (rs.standard_normal((M, N)) * 1e-3).astype(np.float32)
    gX0 = rs.standard_normal((M, K)).astype(np.float32) * 1e-3
    gW0 = rs.standard_normal((N, K)).astype(np.float32) * 1e-3
    Y, gX, gW = _run(fh, X.ravel(), W.ravel(), g.ravel(), M, K, N, beta=1, gX0=gX0.ravel(), gW0=gW0.ravel())
    X64, W64, g64 = X.astype(np.float64), W.astype(np.float64), g.astype(np.float64)
    for got, ref in [(Y, X64 @ W64.T), (gX, gX0 + g64 @ W64), (gW, gW0 + g64.T @ X64)]:
        assert rel_l2(got, ref.ravel()) < 2e-6
        assert max_rel(got, ref.ravel()) < TOL_GRAD
    DA = fh.DeviceArray
    R = rs.standard_normal(M * N).astype(np.float32)
    dX, dW, dR = DA.from_numpy(X.ravel()), DA.from_numpy(W.ravel()), DA.from_numpy(R)
    Yr, P, S = DA((M * N,)), DA((M * N,)), DA((M * N,))
    fh.call("matmulT_fwd_resid", Yr, dR, dX, dW, M, K, N)
    fh.call("matmulT_fwd", P, dX, dW, M, K, N)
    fh.call("add_fwd", S, dR, P, M * N)
    np.testing.assert_array_equal(Yr.numpy(), S.numpy())


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_tail_split(fh):
    """A grouped launch of 2 x 128 + 8 tiles (256 CUs): the 8 tail tiles are cut
    into 8 K pieces each; every job against fp64, fresh and accumulating."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(13)
    shapes = [(1024, 2048, 2048), (1024, 2048, 2048), (1024, 256, 1024)]  # (M, K, N): 128, 128, 8 tiles
    jobs, refs, outs = [], [], []
    for i, (M, K, N) in enumerate(shapes):
        X = rs.standard_normal(M * K).astype(np.float32)
        g = rs.standard_normal(M * N).astype(np.float32)
        beta = (i + 1) % 2  # the tail job accumulates
        gW0 = rs.standard_normal(N * K).astype(np.float32)
        out = DA.from_numpy(gW0)
        ref = g.astype(np.float64).reshape(M, N).T @ X.astype(np.float64).reshape(M, K)
        if beta:
            ref = ref + gW0.astype(np.float64).reshape(N, K)
        jobs.append((out, DA.from_numpy(g), DA.from_numpy(X), M, K, N, beta))
        refs.append(ref.ravel())
        outs.append(out)
    _grouped(fh, jobs)
    for (M, K, N), out, ref in zip(shapes, outs, refs):
        got = out.numpy()
        assert rel_l2(got, ref) < 2e-6, (M, K, N, rel_l2(got, ref))
        assert max_rel(got, ref) < TOL_GRAD


def _grouped_vs_fp64(fh, shapes, seed, single=False):
    DA = fh.DeviceArray
    rs = np.random.default_rng(seed)
    jobs, refs, outs, singles = [], [], [], []
    for i, (M, K, N) in enumerate(shapes):
        X = rs.standard_normal(M * K).astype(np.float32)
        g = rs.standard_normal(M * N).astype(np.float32)
        beta = i % 2
        gW0 = rs.standard_normal(N * K).astype(np.float32)
        dX, dg = DA.from_numpy(X), DA.from_numpy(g)
        out = DA.from_numpy(gW0)
        if single:
            one = DA.from_numpy(gW0)
            fh.call("matmulT_bwd_w", one, dg, dX, M, K, N, beta)
            singles.append(one)
        ref = g.astype(np.float64).reshape(M, N).T @ X.astype(np.float64).reshape(M, K)
        if beta:
            ref = ref + gW0.astype(np.float64).reshape(N, K)
        jobs.append((out, dg, dX, M, K, N, beta))
        refs.append(ref.ravel())
        outs.append(out)
    _grouped(fh, jobs)
    for i, ((M, K, N), out, ref) in enumerate(zip(shapes, outs, refs)):
        got = out.numpy()
        assert rel_l2(got, ref) < 2e-6, (M, K, N, rel_l2(got, ref))
        assert max_rel(got, ref) < TOL_GRAD, (M, K, N)
        if single:
            assert max_rel(got, singles[i].numpy()) < 1e-5, (M, K, N)


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_wide_tiles(fh):
    """A grouped launch of 256 + 272 + 2 tiles of 256x256 (>= two rounds of 256
    CUs: the wide kernel), full and ragged tiles, fresh and accumulating,
    against fp64 and the single launch."""
    _grouped_vs_fp64(fh, [(256, 4096, 4096), (256, 4100, 4000), (64, 300, 260)], 17, single=True)


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_wide_tail_split(fh):
    """256 + 256 + 8 tiles of 256x256: the 8 tail tiles are cut into 8 K pieces
    each (summed in order by the tail reduction)."""
    _grouped_vs_fp64(fh, [(1024, 4096, 4096), (1024, 4096, 4096), (1024, 512, 1024)], 19)


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_wide_split_of_a_fuller_last_round(fh):
    """256 + 256 + 160 tiles of 256x256 over K = 2048: the last round (160 of
    256 CUs) is cut into 3 K pieces per tile (3 x 160 pieces = two rounds of a
    third), summed in order by the tail reduction."""
    _grouped_vs_fp64(fh, [(2048, 4096, 4096), (2048, 4096, 4096), (2048, 4096, 2560)], 23)


@pytest.mark.gpu
def test_matmulT_bwd_w_grouped_rejects_bad_jobs(fh):
    DA = fh.DeviceArray
    a = DA((16,))
    with pytest.raises(fh.ForgeError, match="bad shape"):
        _grouped(fh, [(a, a, a, 4, 0, 4, 0)])
    _grouped(fh, [])  # nothing to do


@pytest.mark.gpu
def test_non_finite_operand_divergence_is_as_documented(fh):
    """The documented divergence for non-finite operands: the split of ±inf
    into fp16 pieces forms inf - inf = NaN, so an output that the
    reference's fp64 sums make ±inf comes out NaN here, and the reference's
    skip of gY == 0 entries (tensor.js:44) has no counterpart (0 · inf =
    NaN).  Every output that does not touch the non-finite element matches
    the oracle."""
    M, K, N = 64, 96, 80
    rs = np.random.default_rng(21)
    X = (rs.standard_normal((M, K)) + 3.0).astype(np.float32)  # nonzero: no inf * 0 in the reference
    W = rs.standard_normal((N, K)).astype(np.float32)
    W[3, 5] = np.inf
    gY = rs.standard_normal((M, N)).astype(np.float32)
    gY[:, 3] = 0.0  # the reference skips these entries
    dX, dW, dg = (fh.DeviceArray.from_numpy(a.ravel()) for a in (X, W, gY))
    Y = fh.DeviceArray((M * N,))
    fh.call("matmulT_fwd", Y, dX, dW, M, K, N)
    gX = fh.DeviceArray((M * K,))
    fh.call("matmulT_bwd_x", gX, dg, dW, M, K, N, 0)
    Yn, gXn = Y.numpy().reshape(M, N), gX.numpy().reshape(M, K)
    Yr = oracle.matmulT_fwd(X.ravel(), W.ravel(), M, K, N).reshape(M, N)
    gXr, _ = oracle.matmulT_bwd(gY.ravel(), X.ravel(), W.ravel(), M, K, N)
    gXr = gXr.reshape(M, K)
    assert np.all(np.isinf(Yr[:, 3])) and np.all(np.isnan(Yn[:, 3]))
    assert np.all(np.isfinite(gXr[:, 5])) and np.all(np.isnan(gXn[:, 5]))
    keep = [n for n in range(N) if n != 3]
    assert rel_l2(Yn[:, keep], Yr[:, keep]) < TOL_FWD
    keepk = [k for k in range(K) if k != 5]
    assert max_rel(gXn[:, keepk], gXr[:, keepk]) < TOL_GRAD


# ───── operand maxima: the *_p forms fill them once and reuse them ─────
@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(8192, 768, 2304), (300, 200, 130), (2048, 1024, 4096)])
def test_matmulT_p_forms_reuse_operand_maxima(fh, M, K, N):
    """The forward fills the maxima of X and W, the input gradient those of gY
    and reuses W's, the weight gradient (single and grouped) reuses gY's and
    X's: every result is the plain entry point's, bit for bit, and each filled
    buffer's largest partial is the operand's largest magnitude."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(31)
    X = rs.standard_normal(M * K).astype(np.float32)
    W = (rs.standard_normal(N * K) * 0.02).astype(np.float32)
    g = (rs.standard_normal(M * N) * 1e-4).astype(np.float32)
    dX, dW, dg = DA.from_numpy(X), DA.from_numpy(W), DA.from_numpy(g)
    xpx, xpw, xpg = DA((256,)), DA((256,)), DA((256,))
    Y, Yp = DA((M * N,)), DA((M * N,))
    fh.call("matmulT_fwd", Y, dX, dW, M, K, N)
    fh.call("matmulT_fwd_p", Yp, dX, dW, M, K, N, xpx, xpw, 0)
    np.testing.assert_array_equal(Yp.numpy(), Y.numpy())
    for buf, arr in ((xpx, X), (xpw, W)):
        assert buf.numpy().max() == np.abs(arr).max()
    gX, gXp = DA((M * K,)), DA((M * K,))
    fh.call("matmulT_bwd_x", gX, dg, dW, M, K, N, 0)
    fh.call("matmulT_bwd_x_p", gXp, dg, dW, M, K, N, 0, xpg, xpw, 2)
    np.testing.assert_array_equal(gXp.numpy(), gX.numpy())
    assert xpg.numpy().max() == np.abs(g).max()
    gW, gWp = DA((N * K,)), DA((N * K,))
    fh.call("matmulT_bwd_w", gW, dg, dX, M, K, N, 0)
    fh.call("matmulT_bwd_w_p", gWp, dg, dX, M, K, N, 0, xpg, xpx, 3)
    np.testing.assert_array_equal(gWp.numpy(), gW.numpy())
    # both gradients in one call, every maximum given, and none given
    gX2, gW2 = DA((M * K,)), DA((N * K,))
    fh.call("matmulT_bwd_p", gX2, 0, gW2, 0, dg, dX, dW, M, K, N, xpg, xpx, xpw, 7)
    np.testing.assert_array_equal(gX2.numpy(), gX.numpy())
    np.testing.assert_array_equal(gW2.numpy(), gW.numpy())
    gX3, gW3 = DA((M * K,)), DA((N * K,))
    fh.call("matmulT_bwd_p", gX3, 0, gW3, 0, dg, dX, dW, M, K, N, None, None, None, 0)
    np.testing.assert_array_equal(gX3.numpy(), gX.numpy())
    np.testing.assert_array_equal(gW3.numpy(), gW.numpy())
    # grouped: one job with the maxima, one computing them
    out1, out2 = DA((N * K,)), DA((N * K,))
    arr = (fh.WgradJob * 2)()
    arr[0] = fh.WgradJob(out1.ptr, dg.ptr, dX.ptr, M, K, N, 0, xpg.ptr, xpx.ptr)
    arr[1] = fh.WgradJob(out2.ptr, dg.ptr, dX.ptr, M, K, N, 0, None, None)
    fh.check(fh.lib.fg_matmulT_bwd_w_grouped(ctypes.cast(arr, ctypes.c_void_p), 2), "fg_matmulT_bwd_w_grouped")
    np.testing.assert_array_equal(out1.numpy(), out2.numpy())
    assert max_rel(out1.numpy(), gW.numpy()) < 1e-5  # one K range against the single launch's pieces


@pytest.mark.gpu
def test_matmulT_operand_scale_is_per_operand(fh):
    """Operands far outside fp16's range (|x| ~ 1e30 against 1e-30, and
    gradients of 1e-20) come out as their fp64 products: each operand's power
    of two brings it into range, and the sum is scaled back exactly."""
    DA = fh.DeviceArray
    rs = np.random.default_rng(33)
    M, K, N = 256, 384, 320
    for sx, sw in ((1e30, 1e-30), (1e-20, 1e-18), (3e4, 7e4)):
        X = (rs.standard_normal(M * K) * sx).astype(np.float32)
        W = (rs.standard_normal(N * K) * sw).astype(np.float32)
        Y = DA((M * N,))
        fh.call("matmulT_fwd", Y, DA.from_numpy(X), DA.from_numpy(W), M, K, N)
        ref = X.astype(np.float64).reshape(M, K) @ W.astype(np.float64).reshape(N, K).T
        assert rel_l2(Y.numpy(), ref.ravel()) < 2e-6, (sx, sw)
