"""Shared helpers for the parity tests."""
import math

import numpy as np

# Tolerances from the north-star parity bar, relative to the output RMS.
TOL_F32 = 1e-5
TOL_16 = 2e-3


def rel_err(got, ref) -> float:
    """max |got - ref| / rms(ref)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = math.sqrt(float(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref))) / max(rms, 1e-30)


def normal(rng, shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(np.float32).astype(dtype)


def log(*args):
    print(*args, flush=True)
