"""Copy-kernel calibration for HBM traffic counters.

Runs the library's accumulate kernel with beta = 0 (a plain stream copy,
Y[i] = X[i]) over N fp32 elements, REPS times, so a `rocprofv3 --pmc
FETCH_SIZE` / `WRITE_SIZE` run over it gives the counter reading for a known
number of bytes (4*N read, 4*N written per dispatch).

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
    for _ in range(reps):
        fh.call("accum", y, x, n, 0)
    fh.sync()
    print("copied %d x %d bytes" % (reps, 4 * n))


if __name__ == "__main__":
    main()
