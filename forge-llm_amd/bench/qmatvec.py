"""Times fg_qmatvec (QuantLinear.forward on the device) per ggml type at the
matrix shapes of a Llama-3-8B layer and its LM head, batch 1.

Each launch reads one of several copies of the weight matrix in turn (copies
enough to span > 768 MiB, three times the 256 MiB MALL), so every launch
streams its weights from HBM.  Achieved bandwidth counts the algorithmic
bytes of one launch: N rows of rowBytes(type, K) plus x (4K) and y (4N).

    python forge-llm_amd/bench/qmatvec.py [types] [reps]
    e.g. python forge-llm_amd/bench/qmatvec.py 0,1,8,12,13,14 200

Prints one JSON line per (type, shape).
"""
import ctypes
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402

SHAPES = {"wqkv": (6144, 4096), "wo": (4096, 4096), "gate_up": (14336, 4096), "down": (4096, 14336),
          "head": (128256, 4096)}
HBM_PEAK = 8.0e12


def row_bytes(t, k):
    b = ctypes.c_int64()
    fh.check(fh.lib.fg_qrow_bytes(t, k, ctypes.byref(b)), "fg_qrow_bytes")
    return b.value


def main():
    types = [int(t) for t in (sys.argv[1] if len(sys.argv) > 1 else "0,1,8,12,13,14").split(",")]
    reps = int(sys.argv[2]) if len(sys.argv) > 2 else 200
    fh.init(0)
    rs = np.random.default_rng(0)
    for name, (N, K) in SHAPES.items():
        x = fh.DeviceArray.from_numpy(rs.standard_normal(K).astype(np.float32))
        y = fh.DeviceArray((N,))
        for t in types:
            wbytes = row_bytes(t, K) * N
            copies = max(2, -(-768 * 2 ** 20 // wbytes))
            # weights: arbitrary bytes with small, finite scales are enough for timing;
            # quantize a normal matrix once on the device and replicate it
            src = fh.DeviceArray.from_numpy((rs.standard_normal(N * K) * 0.02).astype(np.float32))
            ws = [fh.DeviceArray((wbytes,), np.uint8) for _ in range(copies)]
            fh.check(fh.lib.fg_quantize(t, ctypes.c_void_p(ws[0].ptr), ctypes.c_void_p(src.ptr), N * K), "fg_quantize")
            src.free()
            for w in ws[1:]:
                fh.check(fh.lib.fg_d2d(ctypes.c_void_p(w.ptr), ctypes.c_void_p(ws[0].ptr), wbytes), "fg_d2d")
            launch = lambda i: fh.check(fh.lib.fg_qmatvec(  # noqa: E731
                t, ctypes.c_void_p(y.ptr), ctypes.c_void_p(ws[i % copies].ptr), ctypes.c_void_p(x.ptr), N, K),
                "fg_qmatvec")
            for i in range(10):
                launch(i)
            e0, e1 = fh.Event(), fh.Event()
            e0.record()
            for i in range(reps):
                launch(i)
            e1.record()
            fh.sync()
            us = e0.elapsed_ms(e1) * 1e3 / reps
            alg = wbytes + 4 * K + 4 * N
            print(json.dumps({"type": t, "matrix": name, "N": N, "K": K, "copies": copies, "us": round(us, 2),
                              "weight_bytes": wbytes, "GBps": round(alg / us / 1e3, 1),
                              "hbm_frac": round(alg / (us * 1e-6) / HBM_PEAK, 3)}), flush=True)
            for w in ws:
                w.free()


if __name__ == "__main__":
    main()
