"""Writes tests/golden/golden_ops.npz: small inputs and their fp64 closed-form
outputs for every op of the training path (from oracle/np_ref.py), plus the
reference's own known answers.  The C oracle (CPU) and the GPU kernels (GPU)
are both checked against this file, so a change to either restatement cannot
silently move the target.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import np_ref  # noqa: E402


def f32(rs, *shape, s=1.0):
    return (rs.standard_normal(shape) * s).astype(np.float32)


def main():
    rs = np.random.default_rng(20260101)
    out = {}
    # matmulT  M=5 K=7 N=3
    X, W, G = f32(rs, 5, 7), f32(rs, 3, 7), f32(rs, 5, 3)
    out.update(mm_X=X, mm_W=W, mm_G=G, mm_Y=np_ref.matmulT(X.astype(float), W.astype(float)))
    gX, gW = np_ref.matmulT_grads(G.astype(float), X.astype(float), W.astype(float))
    out.update(mm_gX=gX, mm_gW=gW)
    # rmsNorm  T=3 D=6 eps=1e-5
    X, w, G = f32(rs, 3, 6), f32(rs, 6, s=0.5) + 1, f32(rs, 3, 6)
    Y, inv = np_ref.rmsnorm(X.astype(float), w.astype(float), 1e-5)
    gX, gw = np_ref.rmsnorm_grads(G.astype(float), X.astype(float), w.astype(float), 1e-5)
    out.update(rn_X=X, rn_w=w, rn_G=G, rn_Y=Y, rn_inv=inv, rn_gX=gX, rn_gw=gw)
    # ropeRows  T=5 nH=2 dH=8 pos0=3 theta=1e4 (and the backward)
    X, G = f32(rs, 5, 16), f32(rs, 5, 16)
    out.update(rp_X=X, rp_G=G, rp_Y=np_ref.rope(X.astype(float), 2, 8, 3, 1e4, 0),
               rp_gX=np_ref.rope(G.astype(float), 2, 8, 3, 1e4, 0, inverse=True))
    # attention  B=2 T=5 nH=4 nKV=2 dH=8
    Q, K, V, G = f32(rs, 10, 32), f32(rs, 10, 16), f32(rs, 10, 16), f32(rs, 10, 32)
    O, grads = np_ref.attention(Q.astype(float), K.astype(float), V.astype(float), 2, 5, 4, 2, 8)
    dQ, dK, dV = grads(G.astype(float))
    out.update(at_Q=Q, at_K=K, at_V=V, at_G=G, at_O=O, at_dQ=dQ, at_dK=dK, at_dV=dV)
    # swiglu  n=12
    Gt, U, D = f32(rs, 12, s=2), f32(rs, 12), f32(rs, 12)
    gG, gU = np_ref.swiglu_grads(D.astype(float), Gt.astype(float), U.astype(float))
    out.update(sw_G=Gt, sw_U=U, sw_D=D, sw_O=np_ref.swiglu(Gt.astype(float), U.astype(float)), sw_gG=gG, sw_gU=gU)
    # crossEntropyMean  T=4 V=9
    L = f32(rs, 4, 9, s=2)
    tg = np.array([0, 8, 3, 3], np.int32)
    loss, gL = np_ref.ce(L.astype(float), tg)
    out.update(ce_L=L, ce_tg=tg, ce_loss=np.array([loss]), ce_gL=gL)
    # Adam known answer (l2-l6.test.js:205-211): lr 0.1, g 1, total 100
    out["adam_known_dw"] = np.array([0.1 * 0.5 * (1 + np.cos(np.pi / 100)) / (1 + 1e-8)])
    # embed scatter-add known answer (l2-l6.test.js:158-173)
    E = (np.arange(12) * 0.1).astype(np.float32)
    ids = np.array([0, 2, 2], np.int32)
    want = np.zeros((4, 3))
    np.add.at(want, ids, np.arange(1, 10, dtype=np.float64).reshape(3, 3))
    out.update(em_E=E, em_ids=ids, em_gE=want)
    np.savez_compressed(os.path.join(HERE, "golden_ops.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
