"""Times one matmulT shape on the device, for profiler and counter runs.

    python forge-llm_amd/bench/gemm_shape.py [M N K] [reps] [fwd|bwd_x|bwd_w]

Runs `reps` launches of fg_matmulT_fwd (Y[M,N] = X[M,K]·W[N,K]^T, default), of
fg_matmulT_bwd_x or of fg_matmulT_bwd_w over N(0,1) activations and N(0,0.02)
weights (random operands: the MFMA clock under load depends on the data) and
prints the mean device time per launch and the fp32 TFLOP/s.
"""
import ctypes
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402


def main():
    a = sys.argv[1:]
    M, N, K = (int(a[0]), int(a[1]), int(a[2])) if len(a) >= 3 else (8192, 4096, 768)
    reps = int(a[3]) if len(a) >= 4 else 20
    mode = a[4] if len(a) >= 5 else "fwd"
    fh.init(0)
    rs = np.random.default_rng(0)
    vp = ctypes.c_void_p
    if mode == "fwd":     # Y[M,N] = X[M,K] W[N,K]^T
        X = fh.DeviceArray.from_numpy(rs.standard_normal(M * K).astype(np.float32))
        W = fh.DeviceArray.from_numpy((rs.standard_normal(N * K) * 0.02).astype(np.float32))
        Y = fh.DeviceArray((M * N,))
        run = lambda: fh.lib.fg_matmulT_fwd(vp(Y.ptr), vp(X.ptr), vp(W.ptr), M, K, N)  # noqa: E731
    elif mode == "bwd_x":  # gX[M,K] = gY[M,N] W[N,K]
        G = fh.DeviceArray.from_numpy(rs.standard_normal(M * N).astype(np.float32))
        W = fh.DeviceArray.from_numpy((rs.standard_normal(N * K) * 0.02).astype(np.float32))
        Y = fh.DeviceArray((M * K,))
        run = lambda: fh.lib.fg_matmulT_bwd_x(vp(Y.ptr), vp(G.ptr), vp(W.ptr), M, K, N, 0)  # noqa: E731
    else:                  # gW[N,K] = gY[M,N]^T X[M,K]
        G = fh.DeviceArray.from_numpy(rs.standard_normal(M * N).astype(np.float32))
        X = fh.DeviceArray.from_numpy(rs.standard_normal(M * K).astype(np.float32))
        Y = fh.DeviceArray((N * K,))
        run = lambda: fh.lib.fg_matmulT_bwd_w(vp(Y.ptr), vp(G.ptr), vp(X.ptr), M, K, N, 0)  # noqa: E731
    for _ in range(3):
        fh.check(run(), mode)
    e0, e1 = fh.Event(), fh.Event()
    e0.record()
    for _ in range(reps):
        fh.check(run(), mode)
    e1.record()
    fh.sync()
    us = e0.elapsed_ms(e1) * 1e3 / reps
    print("matmulT %s M=%d N=%d K=%d: %.1f us per launch, %.1f TFLOP/s" % (mode, M, N, K, us,
                                                                       2.0 * M * N * K / us / 1e6))


if __name__ == "__main__":
    main()
