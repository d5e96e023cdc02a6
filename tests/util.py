"""Error metrics used by the parity tests (the reference's own definitions)."""
import numpy as np


def rel_l2(got, ref):
    """numeric.js:152-156 relL2, in fp64."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    den = float(np.sum(ref * ref)) or 1.0
    return float(np.sqrt(np.sum((got - ref) ** 2) / den))


def max_rel(got, ref):
    """max|got-ref| / max|ref| per tensor (verify.js:138-161 gradient-scale metric)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    scale = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    return float(np.max(np.abs(got - ref))) / scale if ref.size else 0.0


# Tolerances stated for this path: forward outputs relative-L2, gradients
# max-relative (to the tensor's max |value|), Adam state relative.
TOL_FWD = 1e-5
TOL_GRAD = 1e-4
TOL_ADAM = 1e-6
