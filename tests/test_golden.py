"""The committed golden fixtures (tests/golden/golden_ops.npz, fp64 closed
forms) against the C oracle (CPU) and against the GPU kernels (GPU)."""
import os

import numpy as np
import pytest

import oracle
from util import TOL_FWD, TOL_GRAD, max_rel, rel_l2

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_ops.npz"), allow_pickle=False)


def test_oracle_vs_golden():
    Y = oracle.matmulT_fwd(G["mm_X"], G["mm_W"], 5, 7, 3)
    gX, gW = oracle.matmulT_bwd(G["mm_G"], G["mm_X"], G["mm_W"], 5, 7, 3)
    assert rel_l2(Y, G["mm_Y"]) < 1e-7 and max_rel(gX, G["mm_gX"]) < 1e-6 and max_rel(gW, G["mm_gW"]) < 1e-6
    Y, inv = oracle.rmsnorm_fwd(G["rn_X"], G["rn_w"], 3, 6, 1e-5)
    gX, gw = oracle.rmsnorm_bwd(G["rn_G"], G["rn_X"], G["rn_w"], inv, 3, 6)
    assert rel_l2(Y, G["rn_Y"]) < 1e-7 and max_rel(gX, G["rn_gX"]) < 1e-6 and max_rel(gw, G["rn_gw"]) < 1e-6
    assert rel_l2(oracle.rope_fwd(G["rp_X"], 5, 2, 8, 3, 1e4, 0), G["rp_Y"]) < 1e-7
    assert rel_l2(oracle.rope_bwd(G["rp_G"], 5, 2, 8, 3, 1e4, 0), G["rp_gX"]) < 1e-7
    O, P = oracle.attn_fwd(G["at_Q"], G["at_K"], G["at_V"], 2, 5, 4, 2, 8)
    dQ, dK, dV = oracle.attn_bwd(G["at_G"], P, G["at_Q"], G["at_K"], G["at_V"], 2, 5, 4, 2, 8)
    assert rel_l2(O, G["at_O"]) < 1e-6
    for a, b in [(dQ, "at_dQ"), (dK, "at_dK"), (dV, "at_dV")]:
        assert max_rel(a, G[b]) < 1e-5
    O, sig = oracle.swiglu_fwd(G["sw_G"], G["sw_U"])
    gG, gU = oracle.swiglu_bwd(G["sw_D"], sig, G["sw_G"], G["sw_U"])
    assert rel_l2(O, G["sw_O"]) < 1e-7 and max_rel(gG, G["sw_gG"]) < 1e-6 and max_rel(gU, G["sw_gU"]) < 1e-6
    loss, probs = oracle.ce_fwd(G["ce_L"], G["ce_tg"], 4, 9)
    assert abs(loss - G["ce_loss"][0]) < 1e-6
    assert max_rel(oracle.ce_bwd(1.0, probs, G["ce_tg"], 4, 9), G["ce_gL"]) < 1e-6
    np.testing.assert_array_equal(oracle.embed_bwd(np.arange(1, 10, dtype=np.float32), G["em_ids"], 4, 3),
                                  G["em_gE"].ravel())
    p, g = [np.ones(1, np.float32)], [np.ones(1, np.float32)]
    oracle.adam_step(p, g, [np.zeros(1, np.float32)], [np.zeros(1, np.float32)], 1, lr=0.1, total=100)
    assert abs(1 - p[0][0] - G["adam_known_dw"][0]) < 1e-7


@pytest.mark.gpu
def test_gpu_vs_golden(fh):
    DA = fh.DeviceArray
    up = DA.from_numpy
    Y, gX, gW = DA((15,)), DA((35,)), DA((21,))
    fh.call("matmulT_fwd", Y, up(G["mm_X"]), up(G["mm_W"]), 5, 7, 3)
    fh.call("matmulT_bwd_x", gX, up(G["mm_G"]), up(G["mm_W"]), 5, 7, 3, 0)
    fh.call("matmulT_bwd_w", gW, up(G["mm_G"]), up(G["mm_X"]), 5, 7, 3, 0)
    assert rel_l2(Y.numpy(), G["mm_Y"]) < TOL_FWD
    assert max_rel(gX.numpy(), G["mm_gX"]) < TOL_GRAD and max_rel(gW.numpy(), G["mm_gW"]) < TOL_GRAD
    Y, inv, gX, gw = DA((18,)), DA((3,)), DA((18,)), DA((6,))
    fh.call("rmsnorm_fwd", Y, inv, up(G["rn_X"]), up(G["rn_w"]), 3, 6, 1e-5)
    fh.call("rmsnorm_bwd", gX, 0, gw, 0, up(G["rn_G"]), up(G["rn_X"]), up(G["rn_w"]), inv, 3, 6)
    assert rel_l2(Y.numpy(), G["rn_Y"]) < TOL_FWD
    assert max_rel(gX.numpy(), G["rn_gX"]) < TOL_GRAD and max_rel(gw.numpy(), G["rn_gw"]) < TOL_GRAD
    c, s = oracle.rope_table(8, 8, 1e4)
    Y, gX = DA((80,)), DA((80,))
    fh.call("rope_fwd", Y, up(G["rp_X"]), up(c), up(s), 8, 5, 2, 8, 3, 0)
    fh.call("rope_bwd", gX, up(G["rp_G"]), up(c), up(s), 8, 5, 2, 8, 3, 0, 0)
    assert rel_l2(Y.numpy(), G["rp_Y"]) < TOL_FWD and rel_l2(gX.numpy(), G["rp_gX"]) < TOL_FWD
    O, lse = DA((320,)), DA((40,))
    dQ, dK, dV = DA((320,)), DA((160,)), DA((160,))
    Q, K, V = up(G["at_Q"]), up(G["at_K"]), up(G["at_V"])
    fh.call("attn_fwd", O, lse, Q, K, V, 2, 5, 4, 2, 8)
    fh.call("attn_bwd", dQ, 0, dK, 0, dV, 0, up(G["at_G"]), Q, K, V, O, lse, 2, 5, 4, 2, 8)
    assert rel_l2(O.numpy(), G["at_O"]) < TOL_FWD
    for a, b in [(dQ, "at_dQ"), (dK, "at_dK"), (dV, "at_dV")]:
        assert max_rel(a.numpy(), G[b]) < TOL_GRAD
    O, gG, gU = DA((12,)), DA((12,)), DA((12,))
    fh.call("swiglu_fwd", O, up(G["sw_G"]), up(G["sw_U"]), 12)
    fh.call("swiglu_bwd", gG, 0, gU, 0, up(G["sw_D"]), up(G["sw_G"]), up(G["sw_U"]), 12)
    assert rel_l2(O.numpy(), G["sw_O"]) < TOL_FWD
    assert max_rel(gG.numpy(), G["sw_gG"]) < TOL_GRAD and max_rel(gU.numpy(), G["sw_gU"]) < TOL_GRAD
    loss, lse, gL = DA((1,)), DA((4,)), DA((36,))
    L, tg = up(G["ce_L"]), up(G["ce_tg"])
    fh.call("ce_fwd", loss, lse, L, tg, 4, 9)
    fh.call("ce_bwd", gL, L, lse, tg, up(np.ones(1, np.float32)), 4, 9, 0)
    assert abs(loss.numpy()[0] - G["ce_loss"][0]) < 1e-5 * abs(G["ce_loss"][0])
    assert max_rel(gL.numpy(), G["ce_gL"]) < TOL_GRAD
