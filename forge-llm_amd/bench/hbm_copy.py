"""Measures the practical HBM stream bandwidth on this GPU: device-to-device
copies (hipMemcpy through fg_d2d, and the library's slice kernel over the full
width) of 64 MiB, 256 MiB and 1 GiB buffers.  Copies larger than the 256 MiB
Infinity Cache (MALL) run from HBM; smaller ones partly from the cache.

    python forge-llm_amd/bench/hbm_copy.py

Prints read+write GB/s per size and method.
"""
import ctypes
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402


def main():
    fh.init(0)
    for n in (1 << 24, 1 << 26, 1 << 28):
        x, y = fh.DeviceArray((n,)), fh.DeviceArray((n,))
        fh.call("zero", x, n * 4)
        rows, cols = n // 4096, 4096
        for name, run in (("slice kernel", lambda: fh.call("slice_cols_fwd", y, x, rows, cols, 0, cols)),
                          ("hipMemcpy d2d", lambda: fh.check(fh.lib.fg_d2d(ctypes.c_void_p(y.ptr),
                                                                            ctypes.c_void_p(x.ptr), n * 4), "d2d"))):
            for _ in range(3):
                run()
            e0, e1 = fh.Event(), fh.Event()
            reps = 20
            e0.record()
            for _ in range(reps):
                run()
            e1.record()
            fh.sync()
            us = e0.elapsed_ms(e1) * 1e3 / reps
            print("%-14s %5d MiB: %8.1f us, %6.0f GB/s read+write" % (name, 4 * n >> 20, us, 8 * n / us / 1e3))
        x.free()
        y.free()


if __name__ == "__main__":
    main()
