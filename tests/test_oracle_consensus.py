"""Pins for the oracle's consensus math (crates/qx-consensus-math/src/lib.rs).

The golden bits below are the reference's own known answers
(lib.rs:267-295 and :314-330); the error bounds are its own tests
(lib.rs:217-264, :298-311).  A changed constant, a dropped fmaf or a wrong
rounding rule fails at least one of them.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def bits(x):
    return O.f32_bits(x)


def test_exp_golden_bits():
    # lib.rs:267-281
    cases = [-87.0, -10.0, -1.0, 0.0, 1.0, 10.0, 88.0]
    expected = [0x00B33687, 0x383E6BCE, 0x3EBC5AB2, 0x3F800000, 0x402DF854, 0x46AC14EF, 0x7EF882B7]
    assert [bits(O.exp_f32(c)) for c in cases] == expected


def test_rsqrt_golden_bits():
    # lib.rs:283-294
    cases = [1.0e-6, 0.25, 1.0, 2.0, 1024.0]
    expected = [0x447A0000, 0x3FFFFFFF, 0x3F7FFFFF, 0x3F3504F3, 0x3CFFFFFF]
    got = [bits(O.rsqrt_f32(np.float32(c))) for c in cases]
    assert got == expected


def test_rope_sin_cos_golden_bits():
    # lib.rs:314-330
    cases = [(0, 0), (1, 1), (4095, 0), (4095, 31)]
    expected = [(0x00000000, 0x3F800000), (0x3F2E7ACE, 0x3F3B54B0),
                (0xBF7F7136, 0xBD871E5E), (0x3F04F364, 0x3F5AC4FF)]
    got = [tuple(bits(v) for v in O.granite_rope_sin_cos(p, i)) for p, i in cases]
    assert got == expected


def test_exp_error_bound_over_model_domain():
    # lib.rs:217-236: relative error <= 3e-6 on [-87, 88] step 1e-3
    worst = 0.0
    for step in range(-87_000, 88_001, 7):  # every 7th point keeps the CPU suite fast
        x = np.float32(step / 1000.0)
        got = O.exp_f32(x)
        ref = math.exp(float(x))
        worst = max(worst, abs(got - ref) / ref)
    assert worst <= 3.0e-6, worst


def test_rsqrt_error_bound():
    # lib.rs:239-254
    worst = 0.0
    for e in range(-20, 21):
        for m in range(1, 1001, 3):
            x = np.float32(np.float32(m / 1000.0) * np.float32(2.0 ** e))
            got = O.rsqrt_f32(x)
            ref = 1.0 / math.sqrt(float(x))
            worst = max(worst, abs(got - ref) / ref)
    assert worst <= 3.0e-7, worst


def test_special_values():
    # lib.rs:257-264
    assert O.exp_f32(-100.0) == 0.0
    assert O.exp_f32(100.0) == np.finfo(np.float32).max
    assert O.exp_f32(float("nan")) is None
    assert O.exp_f32(float("inf")) is None
    assert O.rsqrt_f32(0.0) is None
    assert O.rsqrt_f32(-1.0) is None
    assert O.sin_cos_f32(4097.0) is None
    assert O.sin_cos_f32(float("nan")) is None
    assert O.granite_rope_sin_cos(0, 32) is None


def test_rope_close_to_native_over_registered_context():
    # lib.rs:298-311: |err| <= 3e-4 against native sin/cos over 4096 x 32
    inv = np.array([O.lib().qxo_granite_inverse_frequency_bits(i) for i in range(32)], np.uint32).view(np.float32)
    worst = 0.0
    for pos in range(0, 4096, 3):
        for pair in range(32):
            angle = np.float32(np.float32(pos) * inv[pair])
            s, c = O.granite_rope_sin_cos(pos, pair)
            worst = max(worst, abs(s - math.sin(float(angle))), abs(c - math.cos(float(angle))))
    assert worst <= 3.0e-4, worst


def test_inverse_frequency_table_is_theta_1e4():
    # The pinned bits are 10000^(-2i/64) rounded to binary32 (lib.rs:24-27).
    inv = np.array([O.lib().qxo_granite_inverse_frequency_bits(i) for i in range(32)], np.uint32).view(np.float32)
    ref = (10000.0 ** (-np.arange(32) * 2.0 / 64.0)).astype(np.float32)
    assert np.max(np.abs(inv.view(np.int32) - ref.view(np.int32))) <= 1


def test_rope_pair_closed_forms():
    # position 0: sin = +0, cos = 1 exactly -> fma(-r, 0, l) = l, fma(r, 1, 0*l) = r
    rng = np.random.default_rng(5)
    for left, right in rng.standard_normal((64, 2)).astype(np.float32):
        f, g = O.granite_rope_pair(0, 3, left, right)
        assert bits(f) == bits(left) and bits(g) == bits(right)
    # rotation preserves the pair norm to within the sin/cos error bound
    for pos in (1, 17, 511, 4095):
        for pair in (0, 5, 31):
            l, r = np.float32(0.75), np.float32(-1.25)
            f, g = O.granite_rope_pair(pos, pair, l, r)
            s, c = O.granite_rope_sin_cos(pos, pair)
            assert abs(f - (l * c - r * s)) < 1e-6 and abs(g - (r * c + l * s)) < 1e-6
            assert abs(math.hypot(f, g) - math.hypot(l, r)) < 1e-3
    assert O.granite_rope_pair(3, 0, float("inf"), 1.0) is None


def test_f16_conversion_matches_numpy_rne():
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(30.0),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, 5.96e-8, 2.98e-8, 1e5, -1e5,
                  np.float32(1.0) + np.float32(2.0 ** -11), np.float32(1.0) + np.float32(3 * 2.0 ** -11)], np.float32),
        (rng.standard_normal(500) * 1e-5).astype(np.float32),  # subnormal halves
    ])
    mine = np.array([O.lib().qxo_f32_to_f16(float(v)) for v in vals], np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, ref)
    back = np.array([O.lib().qxo_f16_to_f32(int(b)) for b in ref], np.float32)
    assert np.array_equal(back.view(np.uint32), ref.view(np.float16).astype(np.float32).view(np.uint32))


def test_bf16_conversion_matches_torch_rne():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(12)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * np.float32(100.0),
                           np.array([0.0, -0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.4e38], np.float32)])
    mine = np.array([O.lib().qxo_f32_to_bf16(float(v)) for v in vals], np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, ref)
    assert np.array_equal(O.f32_to_bf16_bits(vals), ref)
