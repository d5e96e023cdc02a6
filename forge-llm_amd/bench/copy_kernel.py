"""Copy-kernel calibration for HBM traffic counters.

Runs the library's sliceCols kernel over the full width (a plain,
cached stream copy Y[i] = X[i], the load/store kind the GEMMs use) over N
fp32 elements, REPS times, so a `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE`
run over it gives the counter reading for a known number of bytes (4*N read,
4*N written per dispatch).

    python forge-llm_amd/bench/copy_kernel.py [N] [REPS]
"""
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), ".."))
import forge_hip as fh  # noqa: E402


def main():
    n = int(sys.argv[1]) if len(sys.argv) > 1 else 1 << 26
    reps = int(sys.argv[2]) if len(sys.argv) > 2 else 5
    fh.init(0)
    x, y = fh.DeviceArray((n,)), fh.DeviceArray((n,))
    fh.call("zero", x, n * 4)
    rows, cols = n // 4096, 4096
    for _ in range(reps):
        fh.call("slice_cols_fwd", y, x, rows, cols, 0, cols)
    fh.sync()
    print("copied %d x %d bytes" % (reps, 4 * n))


if __name__ == "__main__":
    main()
