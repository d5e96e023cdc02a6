"""Isolated-op measurements (one MI355X).

    python forge-llm_amd/bench/configs.py [--reps N]

Workloads: matmulT X[2048x1024]·W[4096x1024]^T forward + input gradient +
weight gradient; crossEntropyMean over 2048x32000 logits ~ N(0, 2^2),
forward + backward; Adam over 2^26 parameters (p, g ~ N(0, 1), clip 1);
causalAttnBatch B 8, nH 16, nKV 4, T 2048, dH 64, forward and backward;
the same at B 8, T 1024, d_model 768 for other head sizes (dH 80: the dH 96
MFMA kernels on head-padded copies; dH 96: its own; dH 256: batched GEMM
launches).  Each line gives the mean time over N launches (HIP events on the
library stream), the algorithmic work and its fraction of the kernel's
roofline: HBM 8 TB/s, or for the split-fp16 contractions the dense fp16 MFMA
peak / 3 (2500 / 3 TFLOP/s, three fp16 products per fp32 product), with the
fraction of the fp32 MFMA peak (157.3 TFLOP/s) beside it.  Prints one JSON
object.
"""
import argparse
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402

PEAK_SPLIT_TFS = 2500.0 / 3
PEAK_HBM_GBS = 8000.0


def timed(fn, reps):
    fn()
    fh.sync()
    e0, e1 = fh.Event(), fh.Event()
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    return e0.elapsed_ms(e1) / reps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=10)
    a = ap.parse_args()
    fh.init(0)
    DA = fh.DeviceArray
    rs = np.random.default_rng(1)
    out = []

    def up(x):
        return DA.from_numpy(np.ascontiguousarray(x, dtype=np.float32).ravel())

    def line(workload, op, ms, work, unit):
        if unit == "TFLOP/s":
            ach = work / (ms * 1e-3) / 1e12
            peak = PEAK_SPLIT_TFS
        else:
            ach = work / (ms * 1e-3) / 1e9
            peak = PEAK_HBM_GBS
        r = {"workload": workload, "op": op, "ms": round(ms, 4), "achieved": round(ach, 1), "unit": unit,
             "peak": round(peak, 1), "frac": round(ach / peak, 4)}
        if unit == "TFLOP/s":
            r["frac_fp32_mfma"] = round(ach / 157.3, 4)
        out.append(r)
        print("%-26s %-22s %9.3f ms  %8.1f %s  (%.1f%% of %.1f)" % (workload, op, ms, ach, unit, 100 * ach / peak, peak),
              file=sys.stderr, flush=True)

    # ── matmulT 2048x1024x4096 ──
    M, K, N = 2048, 1024, 4096
    X, W, G = up(rs.standard_normal((M, K))), up(rs.standard_normal((N, K))), up(rs.standard_normal((M, N)))
    Y, gX, gW = DA((M * N,)), DA((M * K,)), DA((N * K,))
    fl = 2.0 * M * N * K
    line("matmulT 2048x1024x4096", "matmulT fwd", timed(lambda: fh.call("matmulT_fwd", Y, X, W, M, K, N), a.reps), fl, "TFLOP/s")
    line("matmulT 2048x1024x4096", "matmulT bwd dX", timed(lambda: fh.call("matmulT_bwd_x", gX, G, W, M, K, N, 0), a.reps), fl, "TFLOP/s")
    line("matmulT 2048x1024x4096", "matmulT bwd dW", timed(lambda: fh.call("matmulT_bwd_w", gW, G, X, M, K, N, 0), a.reps), fl, "TFLOP/s")
    line("matmulT 2048x1024x4096", "matmulT bwd dX+dW (one call)",
         timed(lambda: fh.call("matmulT_bwd", gX, 0, gW, 0, G, X, W, M, K, N), a.reps), 2 * fl, "TFLOP/s")
    for t in (X, W, G, Y, gX, gW):
        t.free()

    # ── crossEntropyMean 2048x32000 ──
    R, V = 2048, 32000
    L = up(2.0 * rs.standard_normal((R, V)))
    tg = DA.from_numpy(rs.integers(0, V, R).astype(np.int32))
    loss, lse, gL = DA((1,)), DA((R,)), DA((R * V,))
    one = up(np.ones(1))
    line("CE 2048x32000", "crossEntropyMean fwd", timed(lambda: fh.call("ce_fwd", loss, lse, L, tg, R, V), a.reps),
         4.0 * R * V + 8.0 * R, "GB/s")
    line("CE 2048x32000", "crossEntropyMean bwd", timed(lambda: fh.call("ce_bwd", gL, L, lse, tg, one, R, V, 0), a.reps),
         8.0 * R * V, "GB/s")
    for t in (L, gL):
        t.free()

    # ── Adam over 2^26 parameters (one tensor) ──
    n = 1 << 26
    p, g = up(rs.standard_normal(n)), up(rs.standard_normal(n))
    m, v = DA.zeros((n,)), DA.zeros((n,))
    line("Adam 2^26", "Adam step (clip 1)", timed(lambda: fh.adam_step([(p, g, m, v)], 3e-4, 0.9, 0.999, 1e-8, 0.0, 1.0,
                                                            0.1, 0.001), a.reps), 32.0 * n, "GB/s")
    for t in (p, g, m, v):
        t.free()

    # ── causal attention B8 T2048 nH16 nKV4 dH64 ──
    B, T, nH, nKV, dH = 8, 2048, 16, 4, 64
    Q, Kt, Vt = up(rs.standard_normal(B * T * nH * dH)), up(rs.standard_normal(B * T * nKV * dH)), \
        up(rs.standard_normal(B * T * nKV * dH))
    dO = up(rs.standard_normal(B * T * nH * dH))
    O, LS = DA((B * T * nH * dH,)), DA((B * nH * T,))
    dQ, dK, dV = DA((B * T * nH * dH,)), DA((B * T * nKV * dH,)), DA((B * T * nKV * dH,))
    P = T * (T + 1) / 2.0
    line("attn B8 T2048 nH16/nKV4", "causalAttnBatch fwd", timed(lambda: fh.call("attn_fwd", O, LS, Q, Kt, Vt, B, T, nH, nKV, dH), a.reps),
         4.0 * dH * P * B * nH, "TFLOP/s")
    line("attn B8 T2048 nH16/nKV4", "causalAttnBatch bwd", timed(lambda: fh.call("attn_bwd", dQ, 0, dK, 0, dV, 0, dO, Q, Kt, Vt, O, LS, B, T,
                                                           nH, nKV, dH), a.reps), 8.0 * dH * P * B * nH, "TFLOP/s")
    for t in (Q, Kt, Vt, dO, O, LS, dQ, dK, dV):
        t.free()

    # ── head sizes without a kernel of their own: B8 T1024, d_model 768 ──
    for nH, dH in ((12, 80), (8, 96), (3, 256)):
        B, T = 8, 1024
        Q, Kt, Vt = (up(rs.standard_normal(B * T * nH * dH)) for _ in range(3))
        dO = up(rs.standard_normal(B * T * nH * dH))
        O, LS = DA((B * T * nH * dH,)), DA((B * nH * T,))
        dQ, dK, dV = (DA((B * T * nH * dH,)) for _ in range(3))
        P = T * (T + 1) / 2.0
        wl = "attn B8 T1024 nH%d dH%d" % (nH, dH)
        line(wl, "causalAttnBatch fwd", timed(lambda: fh.call("attn_fwd", O, LS, Q, Kt, Vt, B, T, nH, nH, dH), a.reps),
             4.0 * dH * P * B * nH, "TFLOP/s")
        line(wl, "causalAttnBatch bwd", timed(lambda: fh.call("attn_bwd", dQ, 0, dK, 0, dV, 0, dO, Q, Kt, Vt, O, LS, B,
                                                              T, nH, nH, dH), a.reps), 8.0 * dH * P * B * nH, "TFLOP/s")
        for t in (Q, Kt, Vt, dO, O, LS, dQ, dK, dV):
            t.free()
    print(json.dumps({"ops": out}))


if __name__ == "__main__":
    main()
