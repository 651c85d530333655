"""Pins of the oracle's tiered value cache (oracle.tiered_quantize,
tiered_dequantize, TieredValueCache).  The reference only proposes this
format (docs/qx-structural-memory-2026-08-25.md:69-74); the definition is
this build's (include/qx_hip.h, QXH_I8_TIERED), so the pins are mathematical:

- quantiser: a block of exactly representable multiples returns the
  multiples; every code is the brute-force nearest of the 255 codes (ties to
  even); the scale is within half a binary16 ulp of max|v| / 127; the clamp
  case (subnormal scale), the zero block and a scale that rounds to zero;
- tier model: the boundary bounds (length - window <= boundary <= length),
  every row at or past the boundary is the binary16 value last appended there
  and every row before it the quantisation of that value, and the state does
  not depend on how appends are chunked.
"""
import numpy as np
import pytest

from oracle import oracle as O


def f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16)


def test_exact_multiples_round_trip():
    k = np.array(list(range(-127, -95)) , dtype=np.float32)
    k[5] = 127.0
    v = f16(k / 16.0)
    codes, scale = O.tiered_quantize(v)
    assert scale[0] == np.float16(1.0 / 16)
    assert np.array_equal(codes, k.astype(np.int8))
    assert np.array_equal(O.tiered_dequantize(codes, scale), v.astype(np.float32))


@pytest.mark.parametrize("mag", [1e-3, 0.3, 7.0, 900.0])
def test_codes_are_brute_force_nearest(mag):
    rng = np.random.default_rng(int(mag * 1000) + 1)
    v = f16(mag * rng.standard_normal((64, 32)))
    codes, scales = O.tiered_quantize(v)
    cand = np.arange(-127, 128, dtype=np.float64)
    for row in range(64):
        s = float(scales[row, 0])
        amax = float(np.max(np.abs(v[row].astype(np.float64))))
        ulp = float(np.spacing(np.float16(amax / 127)))
        assert abs(s - amax / 127) <= 0.5 * ulp * (1 + 2.0 ** -10)
        for j in range(32):
            x = float(v[row, j])
            d = np.abs(cand * s - x)
            best = cand[d == d.min()]
            want = best[0] if len(best) == 1 else best[np.argmin(np.abs(best) % 2)]
            assert codes[row, j] == want, (row, j, x, s)


def test_round_half_to_even_and_error_bound():
    v = np.zeros(32, np.float32)
    v[:6] = [127.0, 2.5, 3.5, -2.5, 0.5, -1.5]
    codes, scale = O.tiered_quantize(f16(v))
    assert scale[0] == np.float16(1.0)
    assert list(codes[:6]) == [127, 2, 4, -2, 0, -2]
    rng = np.random.default_rng(3)
    w = f16(rng.standard_normal((100, 64)))
    c, s = O.tiered_quantize(w)
    err = np.abs(O.tiered_dequantize(c, s) - w.astype(np.float32)).reshape(100, 2, 32)
    assert np.all(err <= s.astype(np.float32)[..., None] / 2 * (1 + 1e-6))


def test_clamp_zero_and_vanishing_scale():
    # max|v| / 127 = 1.4 x 2^-24 rounds to the smallest subnormal 2^-24, so
    # max|v| / scale = 177.8 and the code clamps to 127
    v = np.zeros(32, np.float32)
    v[0] = 127 * 1.4 * 2.0 ** -24
    v[1] = -v[0]
    c, s = O.tiered_quantize(f16(v))
    assert s[0] == np.float16(2.0 ** -24) and c[0] == 127 and c[1] == -127
    c, s = O.tiered_quantize(np.zeros(32, np.float16))
    assert s[0] == 0 and not c.any()
    v = np.zeros(32, np.float32)
    v[3] = 2.0 ** -24  # / 127 is below half the smallest subnormal: scale 0
    c, s = O.tiered_quantize(f16(v))
    assert s[0] == 0 and not c.any()


def expected_rows(m: O.TieredValueCache):
    half = m.half[: m.length]
    out = half.astype(np.float32)
    b = m.boundary
    out[:b] = O.tiered_dequantize(*O.tiered_quantize(half[:b]))
    return out


def test_tier_model_invariants_under_appends_and_rollbacks():
    rng = np.random.default_rng(5)
    W = 32
    m = O.TieredValueCache(W, 2, 64)
    for step in range(200):
        if m.length and rng.random() < 0.25:
            m.rollback(int(rng.integers(0, m.length + 1)))
        else:
            t = int(rng.integers(1, 2 * W + 2))
            m.append(rng.standard_normal((t, 2, 64)))
        assert m.length - W <= m.boundary <= m.length
        assert np.array_equal(m.rows(), expected_rows(m)), step


def test_tier_model_is_chunking_independent():
    rng = np.random.default_rng(6)
    rows = rng.standard_normal((300, 2, 64))
    whole = O.TieredValueCache(64, 2, 64)
    whole.append(rows)
    ones = O.TieredValueCache(64, 2, 64)
    for r in rows:
        ones.append(r[None])
    mixed = O.TieredValueCache(64, 2, 64)
    i = 0
    for t in (5, 70, 1, 100, 124):
        mixed.append(rows[i:i + t])
        i += t
    for m in (ones, mixed):
        assert m.boundary == whole.boundary == 300 - 64
        assert np.array_equal(m.rows(), whole.rows())
