"""Pins of the oracle's group-32 Q4 restatement (crates/qx-quant/src/lib.rs)
and of the 256-thread RMS order (crates/qx-runtime/src/lib.rs:2416-2432).

What pins what:
- the reference's own Q4 test (storage size, round-trip error bound);
- closed forms: exact multiples of an f16 scale give codes k + 7 and decode
  exactly; one nonzero input column returns that column of the dequantized
  matrix bit for bit (nibble order, code offset, scale index);
- Rust's round-half-away-from-zero against the banker's rounding a C port
  could slip into;
- the 32-lane tree and the fold orders, by inputs where every other order
  gives a different float32 result.  The expected sums follow the tree the
  reference spells out (reduce_simd32, crates/qx-runtime/src/lib.rs:2298-2305;
  "(((0+16)+(8+24))+...)", kernels/q4_dense.metal:4-5);
- float64 brute force for everything else.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

HID, QH, KVH, D = 1024, 16, 8, 64
BIG = np.float32(2.0 ** 24)  # 2^24 + 1 rounds to 2^24 (ties to even), 2^24 + 2 is exact


def rng(seed):
    return np.random.default_rng(seed)


def decode_numpy(m: O.Q4Matrix):
    """Dequantize straight from the bytes: value i of group g of row r is the
    low (i even) or high (i odd) nibble of byte r*cols/2 + g*16 + i/2."""
    lo = (m.packed & 0xF).astype(np.int32)
    hi = (m.packed >> 4).astype(np.int32)
    codes = np.empty((m.rows, m.cols), np.int32)
    codes[:, 0::2], codes[:, 1::2] = lo, hi
    scale = np.repeat(m.scales.view(np.float16).astype(np.float32), 32, axis=1)
    return (codes - 7).astype(np.float32) * scale


def one_group(codes, scale_bits=0x3C00, groups=1, rows=1):
    """A Q4 matrix from explicit codes [rows][cols] and one f16 scale (1.0)."""
    codes = np.asarray(codes, np.uint8).reshape(rows, 32 * groups)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scales = np.full((rows, groups), scale_bits, np.uint16)
    return O.Q4Matrix(packed, scales, rows, 32 * groups)


def test_reference_round_trip_q4():
    # crates/qx-quant/src/lib.rs:1492-1511 (the Q4 case)
    x = ((np.arange(32, dtype=np.float32) - 16.0) / 7.0)[None]
    m = O.q4_quantize(x)
    assert m.packed.nbytes == 16 and m.scales.size == 1
    deq = O.q4_dequantize(m)
    rel = math.sqrt(float(np.sum((x - deq) ** 2))) / math.sqrt(float(np.sum(x * x)))
    assert rel < 0.6


def test_tail_groups_are_rejected():
    # group tails (crates/qx-quant/src/lib.rs:1556-1561) are outside the GPU layout
    with pytest.raises(O.OracleError):
        O.q4_quantize(np.arange(37, dtype=np.float32)[None])


def test_exact_multiples_give_offset_codes():
    s = np.float32(0.25)
    ks = np.array([7, -7, 3, -1, 0, 5, -6, 2] * 4, np.int32)
    x = (ks.astype(np.float32) * s)[None]
    m = O.q4_quantize(x)
    assert m.scales[0, 0] == 0x3400  # f16 0.25 = max_abs / 7
    codes = (ks + 7).astype(np.uint8)
    assert np.array_equal(m.packed[0], codes[0::2] | (codes[1::2] << 4))
    assert np.array_equal(O.q4_dequantize(m), x)


def test_rounding_is_half_away_from_zero():
    s = np.float32(0.25)
    x = np.zeros(32, np.float32)
    x[:5] = [7 * s, 2.5 * s, -2.5 * s, 0.5 * s, -0.5 * s]
    m = O.q4_quantize(x[None])
    codes = decode_numpy(m)[0] / s
    assert list(codes[:5]) == [7, 3, -3, 1, -1]  # rint would give 2, -2, 0, 0


def test_scale_is_the_f16_rounding_of_max_abs_over_7():
    r = rng(1)
    w = (0.02 * r.standard_normal((16, 256))).astype(np.float32)
    m = O.q4_quantize(w)
    mx = np.max(np.abs(w.reshape(16, 8, 32)), axis=2)
    expect = (mx / np.float32(7.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(m.scales, expect)
    assert np.array_equal(O.q4_dequantize(m), decode_numpy(m))
    assert np.max(np.abs(O.q4_dequantize(m) - w)) <= np.max(mx) / 7 * 0.5 * 1.01


def test_single_column_returns_that_column_exactly():
    r = rng(2)
    m = O.q4_quantize((0.05 * r.standard_normal((8, 128))).astype(np.float32))
    deq = decode_numpy(m)
    for c in (0, 1, 2, 31, 32, 33, 77, 127):
        e = np.zeros(128, np.float32)
        e[c] = 1.0
        assert np.array_equal(O.q4_mat_vec_simd32(m, e), deq[:, c]), c


def test_lane_tree_order():
    # lane partials {0: 2^24, 8: 1, 24: 1}: the reference tree adds 8 + 24
    # first (offset 16), then 0 + 2 (offset 8) = 2^24 + 2.  A left fold or the
    # reversed offsets lose both ones.
    codes = np.full(32, 7, np.uint8)
    codes[[0, 8, 24]] = 8  # weight 1.0
    x = np.zeros(32, np.float32)
    x[0], x[8], x[24] = BIG, 1.0, 1.0
    assert O.q4_mat_vec_simd32(one_group(codes), x)[0] == np.float32(16777218.0)


def test_lane_fold_is_ascending_fma():
    # lane 0 folds columns 0, 32, 64 in order: fma(1, 1, 2^24) rounds back to
    # 2^24 twice.  Summing the two ones first would give 2^24 + 2.
    codes = np.full(96, 7, np.uint8)
    codes[[0, 32, 64]] = 8
    x = np.zeros(96, np.float32)
    x[0], x[32], x[64] = BIG, 1.0, 1.0
    assert O.q4_mat_vec_simd32(one_group(codes, groups=3), x)[0] == BIG


def test_mat_vec_against_float64_and_multiplier():
    r = rng(3)
    m = O.q4_quantize((0.02 * r.standard_normal((64, HID))).astype(np.float32))
    x = r.standard_normal(HID).astype(np.float32)
    got = O.q4_mat_vec_simd32(m, x)
    deq = decode_numpy(m).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    bound = 40 * 2.0 ** -24 * (np.abs(deq) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - ref) <= bound)
    assert np.array_equal(O.q4_mat_vec_simd32(m, x, 0.5), got * np.float32(0.5))
    # a transposed matrix would be caught
    assert not np.allclose(O.q4_mat_vec_simd32(m, x)[:32], (deq[:32, :32].T @ x[:32]), atol=1e-3)


def test_rms_simd_all_ones():
    x = np.ones(HID, np.float32)
    out, total, inv = O.granite_rms_norm_simd(x, np.full(HID, 2.0, np.float32))
    assert total == np.float32(1024.0)
    assert inv == np.float32(O.rsqrt_f32(np.float32(1.0) + np.float32(1e-6)))
    assert abs(float(inv) - 1 / math.sqrt(1.000001)) <= 3e-7
    assert np.all(out == np.float32(inv) * np.float32(2.0))


@pytest.mark.parametrize("small", [[8, 24], [256, 512], [64, 192]])
def test_rms_simd_reduction_order(small):
    # [8, 24]: threads 8 and 24 meet first in group 0's tree -> 2^24 + 2.
    # [256, 512]: thread 0 folds x[0], x[256], x[512] in order -> 2^24.
    # [64, 192]: groups 2 and 6 meet first in the final tree -> 2^24 + 2.
    x = np.zeros(HID, np.float32)
    x[0] = 4096.0  # square 2^24
    x[small] = 1.0
    _, total, _ = O.granite_rms_norm_simd(x)
    expect = BIG if small == [256, 512] else np.float32(16777218.0)
    assert total == expect


def test_rms_simd_against_float64():
    r = rng(4)
    h = r.standard_normal(HID).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(HID)).astype(np.float32)
    y, _, inv = O.granite_rms_norm_simd(h, w)
    ref_inv = 1 / math.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-6)
    assert abs(float(inv) - ref_inv) <= 1e-6 * ref_inv
    assert np.max(np.abs(y - h.astype(np.float64) * ref_inv * w)) <= 2e-6 * np.max(np.abs(y))


def test_hierarchical_attention_closed_forms():
    r = rng(5)
    c = O.KvCache(512)
    k = r.standard_normal((1, KVH, D)).astype(np.float32)
    v = r.standard_normal((1, KVH, D)).astype(np.float32)
    c.extend(k, v)
    q = r.standard_normal(HID).astype(np.float32)
    out = O.granite_attend_simd(q, c, 1).reshape(QH, D)
    for qh in range(QH):
        assert np.array_equal(out[qh], v[0, qh // 2])  # L = 1: weight 1 exactly
    # GQA mapping (crates/qx-runtime/src/lib.rs:2872-2892) over two 32-position
    # chunks: q = k = 0, V_h = h + 1; weights 1/64 and every partial are exact
    c2 = O.KvCache(64)
    vals = np.broadcast_to(np.arange(1, KVH + 1, dtype=np.float32)[None, :, None], (64, KVH, D)).copy()
    c2.extend(np.zeros((64, KVH, D), np.float32), vals)
    out = O.granite_attend_simd(np.zeros(HID, np.float32), c2, 64).reshape(QH, D)
    for qh in range(QH):
        assert np.all(out[qh] == np.float32(qh // 2 + 1))
    with pytest.raises(O.OracleError):
        c3 = O.KvCache(600)
        c3.extend(r.standard_normal((513, KVH, D)).astype(np.float32),
                  r.standard_normal((513, KVH, D)).astype(np.float32))
        O.granite_attend_simd(q, c3, 513)


def test_hierarchical_attention_matches_sequential_form():
    r = rng(6)
    for L in (31, 32, 33, 300, 512):
        c = O.KvCache(512)
        c.extend(r.standard_normal((L, KVH, D)).astype(np.float32), r.standard_normal((L, KVH, D)).astype(np.float32))
        q = r.standard_normal(HID).astype(np.float32)
        a, b = O.granite_attend_simd(q, c, L), O.granite_attend(q, c, L)
        # same math, different summation orders: binary32 rounding only
        assert np.max(np.abs(a - b)) <= 4e-6 * math.sqrt(np.mean(b.astype(np.float64) ** 2)), L


def q4_weights(r):
    nw = (1.0 + 0.05 * r.standard_normal(HID)).astype(np.float32)
    mats = [O.q4_quantize((0.02 * r.standard_normal(shape)).astype(np.float32))
            for shape in ((HID, HID), (512, HID), (512, HID), (HID, HID))]
    return nw, mats


def test_q4_block_composes_the_reference_stages():
    r = rng(7)
    nw, (wq, wk, wv, wo) = q4_weights(r)
    c1, c2 = O.KvCache(8), O.KvCache(8)
    for pos in range(4):
        h = r.standard_normal(HID).astype(np.float32)
        got, qrot, att, inv = O.granite_q4_attention_block(h, nw, wq, wk, wv, wo, pos, c1)
        x, _, _ = O.granite_rms_norm_simd(h, nw)
        q, k, v = (O.q4_mat_vec_simd32(m, x) for m in (wq, wk, wv))
        qr, kr = O.apply_granite_rope(q, k, pos)
        c2.append(pos, kr, v)
        a = O.granite_attend_simd(qr, c2, pos + 1)
        assert np.array_equal(qrot, qr) and np.array_equal(att, a)
        proj = O.q4_mat_vec_simd32(wo, a)
        ref = (np.float64(np.float32(0.22)) * proj.astype(np.float64) + h.astype(np.float64)).astype(np.float32)
        assert np.max(np.abs(got.view(np.int32) - ref.view(np.int32))) <= 1
        assert np.array_equal(got, O.granite_residual(h, proj))
        assert inv == O.granite_rms_norm_simd(got)[2]
    assert np.array_equal(c1.keys(), c2.keys()) and np.array_equal(c1.values(), c2.values())


def test_q4_block_against_float64():
    r = rng(8)
    nw, mats = q4_weights(r)
    deq = [decode_numpy(m).astype(np.float64) for m in mats]
    inv_freq = np.array([O.lib().qxo_granite_inverse_frequency_bits(i) for i in range(32)], np.uint32).view(np.float32)

    def rope(x, pos, heads):
        ang = (np.float32(pos) * inv_freq).astype(np.float64)
        s, c = np.sin(ang), np.cos(ang)
        x = x.reshape(heads, D)
        lft, rgt = x[:, :32], x[:, 32:]
        return np.concatenate([lft * c - rgt * s, rgt * c + lft * s], axis=1)

    cache = O.KvCache(16)
    keys, values = [], []
    for pos in range(12):
        h = r.standard_normal(HID).astype(np.float32)
        got, _, _, _ = O.granite_q4_attention_block(h, nw, *mats, pos, cache)
        h64 = h.astype(np.float64)
        n = h64 / math.sqrt(np.mean(h64 ** 2) + 1e-6) * nw
        q, k, v = deq[0] @ n, deq[1] @ n, deq[2] @ n
        keys.append(rope(k, pos, KVH))
        values.append(v.reshape(KVH, D))
        qr = rope(q, pos, QH)
        K, V = np.stack(keys), np.stack(values)
        att = np.zeros((QH, D))
        for qh in range(QH):
            s = K[:, qh // 2, :] @ qr[qh] * 0.015625
            w = np.exp(s - s.max())
            att[qh] = (w / w.sum()) @ V[:, qh // 2, :]
        delta = 0.22 * (deq[3] @ att.reshape(-1))
        err = np.max(np.abs((got.astype(np.float64) - h64) - delta))
        # binary32 rounding plus the <= 3e-4 consensus sin/cos error
        assert err <= 2e-3 * math.sqrt(np.mean(delta ** 2)), pos
