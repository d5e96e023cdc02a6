"""Device vector-level autograd ops, single-row attention and rmsnormInto
(fg_vec_*, fg_row_attention, fg_row_rmsnorm) against the oracle
(oracle/vector_oracle.c) through the C ABI.

The device evaluates the reference's expressions in the same fp64 order
with one fp32 rounding per store, so results are bit-exact; where an fp64
exp enters (silu, softmaxVec, the attention weights) the device library's
exp may differ from glibc's in the last fp64 ulp, which can move an fp32
result by one ulp: those compare within 1 ulp.
"""
import numpy as np
import pytest

import oracle


def up(fh, a):
    return fh.DeviceArray.from_numpy(np.ascontiguousarray(a))


def f32(rs, n, s=1.0):
    return (rs.standard_normal(n) * s).astype(np.float32)


def ulps(a, b):
    a = np.asarray(a, np.float32).ravel().view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).ravel().view(np.int32).astype(np.int64)
    assert a.size == b.size
    return int(np.max(np.abs(a - b))) if a.size else 0


SIZES = [1, 7, 256, 1000, 70001]


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("scalar_b", [False, True])
@pytest.mark.parametrize("beta", [0, 1])
def test_vec_mul(fh, n, scalar_b, beta):
    rs = np.random.default_rng(n + 10 * scalar_b + 100 * beta)
    a, g = f32(rs, n), f32(rs, n)
    b = f32(rs, 1 if scalar_b else n)
    ga0 = f32(rs, n) if beta else None
    gb0 = f32(rs, b.size) if beta else None
    y_ref = oracle.vec_mul_fwd(a, b)
    ga_ref, gb_ref = oracle.vec_mul_bwd(g, a, b, ga=ga0, gb=gb0)
    da, db, dg = up(fh, a), up(fh, b), up(fh, g)
    y = fh.DeviceArray((n,))
    fh.call("vec_mul_fwd", y, da, db, n, b.size)
    ga = up(fh, ga0) if beta else fh.DeviceArray((n,))
    gb = up(fh, gb0) if beta else fh.DeviceArray((b.size,))
    fh.call("vec_mul_bwd", ga, beta, gb, beta, dg, da, db, n, b.size)
    assert np.array_equal(y.numpy(), y_ref)
    assert np.array_equal(ga.numpy(), ga_ref)
    assert np.array_equal(gb.numpy(), gb_ref)


@pytest.mark.gpu
def test_vec_mul_empty_a_scalar_b_writes_zero_gradient(fh):
    # n = 0 against a one-element b: a fresh gb (beta 0) is the empty sum, 0;
    # an accumulated one keeps its value
    one = up(fh, np.ones(1, np.float32))
    gb = up(fh, np.full(1, np.nan, np.float32))  # stands for uninitialised memory
    ga = fh.DeviceArray((1,))
    fh.call("vec_mul_bwd", ga, 0, gb, 0, one, one, one, 0, 1)
    assert gb.numpy()[0] == 0.0
    gb2 = up(fh, np.full(1, 2.5, np.float32))
    fh.call("vec_mul_bwd", ga, 0, gb2, 1, one, one, one, 0, 1)
    assert gb2.numpy()[0] == np.float32(2.5)


@pytest.mark.gpu
def test_vec_mul_and_dot_of_one_tensor_with_itself(fh):
    # mul(x, x) and dot(x, x): both gradient updates land in x's one buffer,
    # in the reference's order (the ga loop, then the gb loop; autograd.js:73-77, :142-144)
    rs = np.random.default_rng(5)
    n = 4099
    x, g = f32(rs, n), f32(rs, n)
    ga_ref, _ = oracle.vec_mul_bwd(g, x, x)
    _, both_ref = oracle.vec_mul_bwd(g, x, x, gb=ga_ref)
    dx, dg = up(fh, x), up(fh, g)
    gx = fh.DeviceArray((n,))
    fh.call("vec_mul_bwd", gx, 0, gx, 1, dg, dx, dx, n, n)
    assert np.array_equal(gx.numpy(), both_ref)
    k = np.float32(0.37)
    ga_ref, gb_ref = oracle.vec_dot_bwd(k, x, x)
    # the dot loop interleaves ga[i] and gb[i]: one buffer takes both per element
    both = ((ga_ref.astype(np.float64) + np.float64(k) * x.astype(np.float64)).astype(np.float32))
    gx2 = fh.DeviceArray((n,))
    fh.call("vec_dot_bwd", gx2, 0, gx2, 1, up(fh, np.array([k], np.float32)), dx, dx, n)
    assert np.array_equal(gx2.numpy(), both)


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("beta", [0, 1])
def test_vec_silu(fh, n, beta):
    rs = np.random.default_rng(n + beta)
    x, g = f32(rs, n, 4.0), f32(rs, n)
    gx0 = f32(rs, n) if beta else None
    y_ref, s_ref = oracle.vec_silu_fwd(x)
    dx = up(fh, x)
    y, s = fh.DeviceArray((n,)), fh.DeviceArray((n,))
    fh.call("vec_silu_fwd", y, s, dx, n)
    assert ulps(s.numpy(), s_ref) <= 1 and ulps(y.numpy(), y_ref) <= 1
    # backward from the oracle's saved sigma: bit-exact
    gx_ref = oracle.vec_silu_bwd(g, x, s_ref, gx=gx0)
    gx = up(fh, gx0) if beta else fh.DeviceArray((n,))
    fh.call("vec_silu_bwd", gx, beta, up(fh, g), dx, up(fh, s_ref), n)
    assert np.array_equal(gx.numpy(), gx_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [0] + SIZES)
def test_vec_dot_and_scale(fh, n):
    rs = np.random.default_rng(n + 3)
    a, b, g = f32(rs, n), f32(rs, n), f32(rs, n)
    da, db = up(fh, a if n else np.zeros(1, np.float32)), up(fh, b if n else np.zeros(1, np.float32))
    out = fh.DeviceArray((1,))
    fh.call("vec_dot_fwd", out, da, db, n)
    assert out.numpy()[0] == oracle.vec_dot_fwd(a, b)
    if n == 0:
        return
    k = np.float32(-1.25)
    ga_ref, gb_ref = oracle.vec_dot_bwd(k, a, b)
    ga, gb = fh.DeviceArray((n,)), fh.DeviceArray((n,))
    fh.call("vec_dot_bwd", ga, 0, gb, 0, up(fh, np.array([k], np.float32)), da, db, n)
    assert np.array_equal(ga.numpy(), ga_ref) and np.array_equal(gb.numpy(), gb_ref)
    s = 0.1 * (n % 7) - 0.33
    y = fh.DeviceArray((n,))
    fh.call("vec_scale_fwd", y, da, s, n)
    assert np.array_equal(y.numpy(), oracle.vec_scale_fwd(a, s))
    gx0 = f32(rs, n)
    gx = up(fh, gx0)
    fh.call("vec_scale_bwd", gx, 1, up(fh, g), s, n)
    assert np.array_equal(gx.numpy(), oracle.vec_scale_bwd(g, s, gx=gx0))


@pytest.mark.gpu
@pytest.mark.parametrize("n,dH", [(16, 16), (130, 64), (9, 7), (8, 0), (4096, 128)])
@pytest.mark.parametrize("beta", [0, 1])
def test_vec_rope(fh, n, dH, beta):
    rs = np.random.default_rng(n + dH + beta)
    half = (dH + 1) // 2
    ang = 3.0 * 10000.0 ** (-(2 * np.arange(half)) / max(dH, 1))
    c, s = np.cos(ang), np.sin(ang)
    x, g = f32(rs, n), f32(rs, n)
    gx0 = f32(rs, n) if beta else None
    y_ref = oracle.vec_rope_fwd(x, c, s, dH)
    gx_ref = oracle.vec_rope_bwd(g, c, s, dH, gx=gx0 if beta else np.zeros(n, np.float32))
    ct = up(fh, c if half else np.zeros(1))
    st = up(fh, s if half else np.zeros(1))
    y = fh.DeviceArray((n,))
    fh.call("vec_rope_fwd", y, up(fh, x), ct, st, n, dH)
    gx = up(fh, gx0) if beta else fh.DeviceArray((n,))
    fh.call("vec_rope_bwd", gx, beta, up(fh, g), ct, st, n, dH)
    assert np.array_equal(y.numpy(), y_ref)
    assert np.array_equal(gx.numpy(), gx_ref)


@pytest.mark.gpu
def test_vec_rope_rejects_pairs_past_the_vector(fh):
    x = up(fh, np.zeros(8, np.float32))
    t = up(fh, np.zeros(8))
    y = fh.DeviceArray((8,))
    with pytest.raises(fh.ForgeError):
        fh.call("vec_rope_fwd", y, x, t, t, 8, 9)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 7, 256, 1000, 5003])
@pytest.mark.parametrize("beta", [0, 1])
def test_vec_softmax(fh, n, beta):
    rs = np.random.default_rng(n + beta)
    x, g = f32(rs, n, 3.0), f32(rs, n)
    gx0 = f32(rs, n) if beta else None
    y_ref, p_ref = oracle.vec_softmax_fwd(x)
    y, p = fh.DeviceArray((n,)), fh.DeviceArray((n,))
    fh.call("vec_softmax_fwd", y, p, up(fh, x), n)
    assert ulps(p.numpy(), p_ref) <= 1 and np.array_equal(y.numpy(), p.numpy())
    gx_ref = oracle.vec_softmax_bwd(g, p_ref, gx=gx0)
    gx = up(fh, gx0) if beta else fh.DeviceArray((n,))
    fh.call("vec_softmax_bwd", gx, beta, up(fh, g), up(fh, p_ref), n)
    assert np.array_equal(gx.numpy(), gx_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("beta", [0, 1])
def test_vec_softmax_bwd_long_vector(fh, beta):
    # past 65536 elements the backward takes the O(n) form p_i (g_i - g.p):
    # against its fp64 closed form, within one fp32 ulp
    n = 200003
    rs = np.random.default_rng(beta)
    x, g = f32(rs, n, 3.0), f32(rs, n)
    gx0 = f32(rs, n) if beta else np.zeros(n, np.float32)
    _, p = oracle.vec_softmax_fwd(x)
    p64, g64 = p.astype(np.float64), g.astype(np.float64)
    ref = (gx0.astype(np.float64) + p64 * (g64 - np.dot(g64, p64))).astype(np.float32)
    gx = up(fh, gx0) if beta else fh.DeviceArray((n,))
    fh.call("vec_softmax_bwd", gx, beta, up(fh, g), up(fh, p), n)
    assert ulps(gx.numpy(), ref) <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("n,d,causal,qOff", [(64, 16, True, 63), (40, 24, True, 17), (33, 8, False, 0),
                                             (300, 64, True, 250), (1, 4, True, 0), (64, 16, True, -1),
                                             (0, 8, True, 0), (1030, 300, False, 0)])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_row_attention_vs_oracle(fh, n, d, causal, qOff, mode):
    rs = np.random.default_rng(n * 7 + d + mode)
    q, K, V = f32(rs, d), f32(rs, max(n, 1) * d), f32(rs, max(n, 1) * d)
    scale = 1 / np.sqrt(d)
    block = 16
    sc = None
    if mode == 0:
        ref, sc_ref = oracle.attention_decode(q, K, V, n, d, scale, causal, qOff)
    elif mode == 1:
        ref = oracle.attention_naive(q, K, V, n, d, scale, causal, qOff)
    else:
        ref = oracle.flash_attention(q, K, V, n, d, scale, causal, qOff, block)
    out = fh.DeviceArray((d,))
    if mode == 0:
        sc = fh.DeviceArray((max(n, 1),))
    fh.call("row_attention", out, up(fh, q), up(fh, K), up(fh, V), n, d, float(scale), int(causal), qOff, mode,
            block, sc)
    o = out.numpy()
    if np.all(np.isnan(ref)):  # every key masked in the naive variant: 0/0 as in the reference
        assert np.all(np.isnan(o))
    else:
        assert ulps(o, ref) <= 1, (np.max(np.abs(o - ref)))
    if mode == 0 and n > 0:
        assert np.array_equal(sc.numpy()[:n], sc_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 64, 768, 4096, 5000])
def test_row_rmsnorm_vs_oracle(fh, n):
    rs = np.random.default_rng(n)
    x, w = f32(rs, n, 2.0), f32(rs, n)
    out = fh.DeviceArray((n,))
    fh.call("row_rmsnorm", out, up(fh, x), up(fh, w), n, 1e-5)
    assert np.array_equal(out.numpy(), oracle.row_rmsnorm(x, w, 1e-5))
