"""crossEntropyMean fwd/bwd on the GPU vs the oracle (tensor.js:393-417)."""
import numpy as np
import pytest

import oracle
from util import TOL_FWD, TOL_GRAD, max_rel, rel_l2


@pytest.mark.gpu
@pytest.mark.parametrize("rows,V,scale", [(3, 6, 1.0), (256, 31, 1.0), (7, 1001, 3.0), (2048, 32000, 2.0), (1, 1, 1.0),
                                          (2, 2, 1.0), (3, 50000, 2.0)])
def test_ce_parity(fh, rows, V, scale):
    DA = fh.DeviceArray
    rng = oracle.RNG(1)
    logits = rng.normal_f32(rows * V, scale)
    targets = rng.ints(rows, V)
    loss_ref, probs = oracle.ce_fwd(logits, targets, rows, V)
    gl_ref = oracle.ce_bwd(1.0, probs, targets, rows, V)

    L, T = DA.from_numpy(logits), DA.from_numpy(targets)
    loss, lse = DA((1,)), DA((rows,))
    g1 = DA.from_numpy(np.ones(1, np.float32))
    gl = DA((rows * V,))
    fh.call("ce_fwd", loss, lse, L, T, rows, V)
    fh.call("ce_bwd", gl, L, lse, T, g1, rows, V, 0)
    got_loss = loss.numpy()[0]
    assert rel_l2([got_loss], [loss_ref]) < TOL_FWD, (got_loss, loss_ref)
    assert max_rel(gl.numpy(), gl_ref) < TOL_GRAD
    # beta=1 accumulates onto the existing gradient
    fh.call("ce_bwd", gl, L, lse, T, g1, rows, V, 1)
    assert max_rel(gl.numpy(), 2.0 * gl_ref.astype(np.float64)) < TOL_GRAD


@pytest.mark.gpu
@pytest.mark.parametrize("rows,V,scale", [(3, 6, 1.0), (7, 1001, 3.0), (256, 31, 1.0), (4, 4, 1.0), (33, 1000, 1.0),
                                          (2048, 32000, 2.0), (5, 32768, 3.0),
                                          (3, 32772, 1.0), (64, 40000, 2.0), (5, 65536, 2.0), (3, 131072, 1.0),
                                          (4, 128256, 2.0), (2, 131076, 1.0), (3, 50001, 1.0)])
# rows of 128 KB to 512 KB take the kernel holding the row in registers and LDS;
# longer or unaligned ones the kernel reading each row twice
def test_ce_fwd_bwd_equals_fwd_then_bwd(fh, rows, V, scale):
    """fg_ce_fwd_bwd (one pass over the logits) = fg_ce_fwd then fg_ce_bwd with
    a seed gradient of 1 and beta 0, bit for bit: loss, lse and dlogits."""
    DA = fh.DeviceArray
    rng = oracle.RNG(2)
    logits = rng.normal_f32(rows * V, scale)
    targets = rng.ints(rows, V)
    L, T = DA.from_numpy(logits), DA.from_numpy(targets)
    g1 = DA.from_numpy(np.ones(1, np.float32))
    loss1, lse1, gl1 = DA((1,)), DA((rows,)), DA((rows * V,))
    fh.call("ce_fwd", loss1, lse1, L, T, rows, V)
    fh.call("ce_bwd", gl1, L, lse1, T, g1, rows, V, 0)
    loss2, lse2, gl2 = DA((1,)), DA((rows,)), DA((rows * V,))
    fh.call("ce_fwd_bwd", loss2, lse2, gl2, L, T, rows, V)
    np.testing.assert_array_equal(loss2.numpy(), loss1.numpy())
    np.testing.assert_array_equal(lse2.numpy(), lse1.numpy())
    np.testing.assert_array_equal(gl2.numpy(), gl1.numpy())
    with pytest.raises(fh.ForgeError, match="alias"):
        fh.call("ce_fwd_bwd", loss2, lse2, L, L, T, rows, V)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,V", [(3, 6), (2048, 32000), (4, 128256)])
def test_ce_fwd_bwd_p_bounds_the_gradient(fh, rows, V):
    """fg_ce_fwd_bwd_p writes what fg_ce_fwd_bwd writes, and fills the
    gradient's operand maxima with the bound 1/rows, which every entry of the
    seed-1 gradient (softmax - onehot) / rows respects."""
    DA = fh.DeviceArray
    rng = oracle.RNG(5)
    logits = rng.normal_f32(rows * V, 2.0)
    targets = rng.ints(rows, V)
    L, T = DA.from_numpy(logits), DA.from_numpy(targets)
    outs = []
    for p in (False, True):
        loss, lse, gl = DA((1,)), DA((rows,)), DA((rows * V,))
        if p:
            xp = DA((256,))
            fh.call("ce_fwd_bwd_p", loss, lse, gl, L, T, rows, V, xp)
        else:
            fh.call("ce_fwd_bwd", loss, lse, gl, L, T, rows, V)
        outs.append((loss.numpy(), lse.numpy(), gl.numpy()))
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a, b)
    bound = xp.numpy()
    assert np.all(bound == np.float32(1.0 / rows))
    assert np.abs(outs[1][2]).max() <= bound.max() * (1 + 2 ** -23)
