"""Shared helpers for the parity tests."""
import math

import numpy as np

# Tolerances from the north-star parity bar, relative to the output RMS.
TOL_F32 = 1e-5
TOL_16 = 2e-3

# The reference's fp32 attention (crates/qx-runtime/src/lib.rs:484-548) sums
# the softmax denominator and every output element as sequential binary32
# folds over the positions.  Its own distance from exact attention grows with
# the context: at most 6.9e-6 x RMS at 1000 positions but up to 1.6e-5 at
# 4096 (tests/test_oracle_attention.py pins both), so up to this length the
# 1e-5 bar against the oracle holds for any accurate summation order, and
# beyond it only for the reference's own order.
FP32_ORACLE_BAR_MAX_LENGTH = 1024


def rel_err(got, ref) -> float:
    """max |got - ref| / rms(ref)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = math.sqrt(float(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref))) / max(rms, 1e-30)


def row_rel_err(got, ref) -> float:
    """The bar per attention output: max over rows of max |got - ref| / rms(ref
    row), rows along the first axis.  A prefill row is the decode output at
    its position (the reference runs a prompt as repeated decode), held to
    the bar of its own RMS as every decode output is; one RMS over rows of
    very different lengths would let the long rows' small outputs set the
    scale for the short rows' large ones."""
    got = np.asarray(got, dtype=np.float64).reshape(np.shape(got)[0], -1)
    ref = np.asarray(ref, dtype=np.float64).reshape(got.shape)
    rms = np.sqrt(np.mean(ref * ref, axis=1))
    return float(np.max(np.max(np.abs(got - ref), axis=1) / np.maximum(rms, 1e-30)))


def attend64(q, keys, values, scale):
    """float64 GQA attention: q [Hq][D], keys/values [L][Hkv][D]."""
    out = np.zeros(q.shape)
    g = q.shape[0] // keys.shape[1]
    for h in range(q.shape[0]):
        sc = keys[:, h // g, :].astype(np.float64) @ q[h].astype(np.float64) * scale
        w = np.exp(sc - sc.max())
        out[h] = (w / w.sum()) @ values[:, h // g, :].astype(np.float64)
    return out


def check_fp32_bar(got, oracle_out, exact, length):
    """The fp32 parity bar for GPU attention over values the cache holds
    exactly.  Always: within TOL_F32 / 2 of exact (float64) attention.  Up to
    FP32_ORACLE_BAR_MAX_LENGTH positions: within TOL_F32 of the oracle.
    Returns (error vs oracle, error vs exact, oracle's error vs exact)."""
    e, e_gpu, e_ora = rel_err(got, oracle_out), rel_err(got, exact), rel_err(oracle_out, exact)
    assert e_gpu <= TOL_F32 / 2, (e, e_gpu, e_ora)
    if length <= FP32_ORACLE_BAR_MAX_LENGTH:
        assert e <= TOL_F32, (e, e_gpu, e_ora)
    return e, e_gpu, e_ora


def normal(rng, shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(np.float32).astype(dtype)


def log(*args):
    print(*args, flush=True)
