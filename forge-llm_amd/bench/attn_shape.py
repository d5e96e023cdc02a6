"""Times causal attention forward and backward at one shape, for profiler and
counter runs.

    python forge-llm_amd/bench/attn_shape.py [B T nH nKV dH] [reps]

Q, K, V, dO ~ N(0,1); `reps` launches each of fg_attn_fwd and fg_attn_bwd;
prints the mean device time per launch and the algorithmic fp32 TFLOP/s
(forward 4·dH per causal pair, backward 8·dH per pair).
"""
import ctypes
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402


def main():
    a = sys.argv[1:]
    B, T, nH, nKV, dH = (int(x) for x in a[:5]) if len(a) >= 5 else (8, 1024, 12, 12, 64)
    reps = int(a[5]) if len(a) >= 6 else 20
    fh.init(0)
    rs = np.random.default_rng(0)
    vp = ctypes.c_void_p
    arr = lambda n: fh.DeviceArray.from_numpy(rs.standard_normal(n).astype(np.float32))  # noqa: E731
    Q, dO = arr(B * T * nH * dH), arr(B * T * nH * dH)
    K, V = arr(B * T * nKV * dH), arr(B * T * nKV * dH)
    O, dQ = fh.DeviceArray((B * T * nH * dH,)), fh.DeviceArray((B * T * nH * dH,))
    dK, dV = fh.DeviceArray((B * T * nKV * dH,)), fh.DeviceArray((B * T * nKV * dH,))
    lse = fh.DeviceArray((B * nH * T,))
    fwd = lambda: fh.lib.fg_attn_fwd(vp(O.ptr), vp(lse.ptr), vp(Q.ptr), vp(K.ptr), vp(V.ptr), B, T, nH, nKV, dH)  # noqa: E731
    bwd = lambda: fh.lib.fg_attn_bwd(vp(dQ.ptr), 0, vp(dK.ptr), 0, vp(dV.ptr), 0, vp(dO.ptr), vp(Q.ptr),  # noqa: E731
                                     vp(K.ptr), vp(V.ptr), vp(O.ptr), vp(lse.ptr), B, T, nH, nKV, dH)
    pairs = T * (T + 1) / 2.0
    for name, f, flop in (("fwd", fwd, 4.0 * dH * pairs * B * nH), ("bwd", bwd, 8.0 * dH * pairs * B * nH)):
        for _ in range(3):
            fh.check(f(), name)
        e0, e1 = fh.Event(), fh.Event()
        e0.record()
        for _ in range(reps):
            fh.check(f(), name)
        e1.record()
        fh.sync()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        print("attention %s B=%d T=%d nH=%d nKV=%d dH=%d: %.1f us per launch, %.1f TFLOP/s" % (
            name, B, T, nH, nKV, dH, us, flop / us / 1e6))


if __name__ == "__main__":
    main()
