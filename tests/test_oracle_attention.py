"""Pins for the oracle's GQA attention (crates/qx-runtime/src/lib.rs:349-552,
:592-638, :2406-2453; tools/qx-qwen-parity/src/main.rs:1170-1258).

Each check is chosen so that a plausible slip fails it: the reference's own
GQA-mapping and cursor tests, exact special cases (L=1, q=0 at a power-of-two
length), an independent float64 restatement, and torch's float64
scaled_dot_product_attention with enable_gqa.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

QH, KVH, D, HID = 16, 8, 64, 1024


def rng(seed):
    return np.random.default_rng(seed)


def test_grouped_query_attention_uses_matching_kv_head():
    # crates/qx-runtime/src/lib.rs:2872-2892
    cache = O.KvCache(4)
    value = np.zeros((KVH, D), np.float32)
    for h in range(KVH):
        value[h] = h + 1.0
    out = O.granite_attention_decode(np.zeros(HID), np.zeros(KVH * D), value.ravel(), 0, cache)
    assert len(cache) == 1
    for qh in range(QH):
        assert np.all(out[qh * D:(qh + 1) * D] == qh // 2 + 1.0)


def test_kv_cache_rejects_non_sequential_positions():
    # crates/qx-runtime/src/lib.rs:2894-2901 and append rules :382-405
    cache = O.KvCache(2)
    z = np.zeros(HID)
    with pytest.raises(O.OracleError, match="does not follow"):
        O.granite_attention_decode(z, z[:512], z[:512], 1, cache)
    O.granite_attention_decode(z, z[:512], z[:512], 0, cache)
    O.granite_attention_decode(z, z[:512], z[:512], 1, cache)
    with pytest.raises(O.OracleError, match="exceeds context"):
        O.granite_attention_decode(z, z[:512], z[:512], 2, cache)
    assert len(cache) == 2
    cache.reset()
    assert len(cache) == 0


def test_length_one_returns_value_exactly():
    r = rng(1)
    cache = O.KvCache(8)
    q, k, v = (r.standard_normal(n).astype(np.float32) for n in (HID, 512, 512))
    out = O.granite_attention_decode(q, k, v, 0, cache)
    vv = v.reshape(KVH, D)
    for qh in range(QH):
        assert np.array_equal(out[qh * D:(qh + 1) * D], vv[qh // 2])


def test_cache_holds_rotated_key_and_raw_value_position_major():
    r = rng(2)
    cache = O.KvCache(16)
    for pos in range(5):
        q, k, v = (r.standard_normal(n).astype(np.float32) for n in (HID, 512, 512))
        O.granite_attention_decode(q, k, v, pos, cache)
        _, krot = O.apply_granite_rope(q, k, pos)
        assert np.array_equal(cache.keys()[pos].ravel(), krot)
        assert np.array_equal(cache.values()[pos].ravel(), v)


def test_uniform_scores_average_values_exactly():
    # q = 0 -> every score 0 -> exp 1 -> normalizer = L; for L = 4 each weight is
    # exactly 0.25, and with dyadic values every fma is exact.
    cache = O.KvCache(8)
    vals = []
    for pos in range(4):
        v = (np.arange(512, dtype=np.float32) % 7 + pos).astype(np.float32)
        vals.append(v)
        out = O.granite_attention_decode(np.zeros(HID), np.ones(512), v, pos, cache)
    mean = np.mean(np.stack(vals), axis=0).reshape(KVH, D)
    for qh in range(QH):
        assert np.array_equal(out[qh * D:(qh + 1) * D], mean[qh // 2])


def _rope64(x, pos, heads):
    """float64 rotate-half RoPE with the pinned inverse frequencies."""
    inv = np.array([O.lib().qxo_granite_inverse_frequency_bits(i) for i in range(32)], np.uint32).view(np.float32)
    ang = np.float32(pos) * inv  # one binary32 rounding, as the reference
    s, c = np.sin(ang.astype(np.float64)), np.cos(ang.astype(np.float64))
    x = x.reshape(heads, D).astype(np.float64)
    l, rr = x[:, :32], x[:, 32:]
    return np.concatenate([l * c - rr * s, rr * c + l * s], axis=1)


def _attend64(q, keys, values, scale):
    """float64 GQA softmax attention; q [QH][D], keys/values [L][KVH][D]."""
    out = np.zeros((q.shape[0], keys.shape[2]))
    g = q.shape[0] // keys.shape[1]
    for qh in range(q.shape[0]):
        kvh = qh // g
        s = keys[:, kvh, :].astype(np.float64) @ q[qh].astype(np.float64) * scale
        w = np.exp(s - s.max())
        out[qh] = (w / w.sum()) @ values[:, kvh, :].astype(np.float64)
    return out


def test_decode_sequence_matches_float64_restatement():
    r = rng(3)
    cache = O.KvCache(64)
    keys, values = [], []
    for pos in range(40):
        q, k, v = (r.standard_normal(n).astype(np.float32) for n in (HID, 512, 512))
        out = O.granite_attention_decode(q, k, v, pos, cache)
        keys.append(_rope64(k, pos, KVH))
        values.append(v.reshape(KVH, D))
        ref = _attend64(_rope64(q, pos, QH), np.stack(keys), np.stack(values), 0.015625)
        rms = math.sqrt(np.mean(ref ** 2))
        # the only differences are binary32 rounding and the <=3e-4 consensus
        # sin/cos error (lib.rs:298-311)
        assert np.max(np.abs(out.reshape(QH, D) - ref)) <= 2e-3 * rms


def test_attend_matches_torch_sdpa_float64():
    torch = pytest.importorskip("torch")
    r = rng(4)
    L = 300
    cache = O.KvCache(512)
    kr = r.standard_normal((L, KVH, D)).astype(np.float32)
    vr = r.standard_normal((L, KVH, D)).astype(np.float32)
    cache.extend(kr, vr)
    q = r.standard_normal(HID).astype(np.float32)
    out = O.granite_attend(q, cache, L).reshape(QH, D)
    qt = torch.from_numpy(q.reshape(1, QH, 1, D)).double()
    kt = torch.from_numpy(kr.transpose(1, 0, 2).copy()).double().unsqueeze(0)
    vt = torch.from_numpy(vr.transpose(1, 0, 2).copy()).double().unsqueeze(0)
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=0.015625, enable_gqa=True)
    ref = ref[0, :, 0, :].numpy()
    rms = math.sqrt(np.mean(ref ** 2))
    assert np.max(np.abs(out - ref)) <= 1e-5 * rms


def test_fp16_store_rounds_key_after_rope():
    # kernels/v2_decode.metal:478-485: K = half(fma(...)), V = half(v)
    r = rng(6)
    c32, c16 = O.KvCache(8), O.KvCache(8, O.F16, O.F16)
    q, k, v = (r.standard_normal(n).astype(np.float32) for n in (HID, 512, 512))
    O.granite_attention_decode(q, k, v, 3 - 3, c32)
    O.granite_attention_decode(q, k, v, 0, c16)
    assert np.array_equal(c16.keys(), c32.keys().astype(np.float16).astype(np.float32))
    assert np.array_equal(c16.values(), c32.values().astype(np.float16).astype(np.float32))


def test_prefill_rows_equal_repeated_decode():
    r = rng(7)
    T = 24
    q = r.standard_normal((T, HID)).astype(np.float32)
    k = r.standard_normal((T, 512)).astype(np.float32)
    v = r.standard_normal((T, 512)).astype(np.float32)
    dec = O.KvCache(T)
    outs = np.stack([O.granite_attention_decode(q[t], k[t], v[t], t, dec) for t in range(T)])
    pre = O.KvCache(T)
    qrot = np.zeros_like(q)
    for t in range(T):
        qrot[t], krot = O.apply_granite_rope(q[t], k[t], t)
        pre.append(t, krot, v[t])
    rows = np.arange(T)
    assert np.array_equal(O.granite_prefill_rows(qrot, pre, 0, rows), outs)


def test_rms_norm_and_dense_against_float64():
    r = rng(8)
    h = r.standard_normal(HID).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(HID)).astype(np.float32)
    y = O.granite_rms_norm(h, w)
    ref = h.astype(np.float64) / math.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(y - ref)) <= 1e-6 * np.max(np.abs(ref))
    m = (0.02 * r.standard_normal((512, HID))).astype(np.float32)
    d = O.dense_apply(m, h)
    ref = m.astype(np.float64) @ h.astype(np.float64)
    assert np.max(np.abs(d - ref)) <= 1e-5 * math.sqrt(np.mean(ref ** 2))
    # a transposed operand would be caught here
    assert not np.allclose(O.dense_apply(m[:, :512].T.copy(), h[:512]), ref[:512], atol=1e-3)


def test_attention_block_composes_the_reference_stages():
    r = rng(9)
    wq = (0.02 * r.standard_normal((HID, HID))).astype(np.float32)
    wk = (0.02 * r.standard_normal((512, HID))).astype(np.float32)
    wv = (0.02 * r.standard_normal((512, HID))).astype(np.float32)
    wo = (0.02 * r.standard_normal((HID, HID))).astype(np.float32)
    nw = np.ones(HID, np.float32)
    c1, c2 = O.KvCache(4), O.KvCache(4)
    for pos in range(3):
        h = r.standard_normal(HID).astype(np.float32)
        got = O.granite_attention_block(h, nw, wq, wk, wv, wo, pos, c1)
        x = O.granite_rms_norm(h, nw)
        att = O.granite_attention_decode(O.dense_apply(wq, x), O.dense_apply(wk, x), O.dense_apply(wv, x), pos, c2)
        proj = O.dense_apply(wo, att)
        # fma(0.22, proj, h): the float32 product is exact in float64, so one
        # float64 add then a float32 rounding differs from fma by at most 1 ulp
        ref = (np.float64(np.float32(0.22)) * proj.astype(np.float64) + h.astype(np.float64)).astype(np.float32)
        assert np.max(np.abs(got.view(np.int32) - ref.view(np.int32))) <= 1


# --- Qwen -----------------------------------------------------------------------

def test_qwen_gqa_attention_matches_float64():
    r = rng(10)
    ctx = 97
    q = r.standard_normal(32 * 128).astype(np.float16)
    kc = r.standard_normal(ctx * 512).astype(np.float16)
    vc = r.standard_normal(ctx * 512).astype(np.float16)
    bits, f = O.qwen_gqa_attention(q.view(np.uint16), kc.view(np.uint16), vc.view(np.uint16), O.F16, want_f32=True)
    ref = _attend64(q.astype(np.float64).reshape(32, 128), kc.astype(np.float64).reshape(ctx, 4, 128),
                    vc.astype(np.float64).reshape(ctx, 4, 128), 1.0 / math.sqrt(128.0))
    rms = math.sqrt(np.mean(ref ** 2))
    assert np.max(np.abs(f.reshape(32, 128) - ref)) <= 1e-5 * rms
    assert np.array_equal(bits, f.astype(np.float16).view(np.uint16))
    # head mapping: kv head = q head // 8 (main.rs:1225)
    vc2 = np.zeros((ctx, 4, 128), np.float16)
    for h in range(4):
        vc2[:, h, :] = h + 1
    out = O.qwen_gqa_attention(q.view(np.uint16), kc.view(np.uint16), vc2.ravel().view(np.uint16))
    got = out.view(np.float16).reshape(32, 128)
    for qh in range(32):
        assert np.all(got[qh] == qh // 8 + 1)


def test_qwen_qk_norm_rope_matches_float64():
    r = rng(11)
    for fmt, npdt in ((O.F16, np.float16), (O.BF16, None)):
        qf = r.standard_normal(32 * 128).astype(np.float32)
        kf = r.standard_normal(4 * 128).astype(np.float32)
        qb, kb = O.to_bits16(qf, fmt), O.to_bits16(kf, fmt)
        qn = np.ones(128, np.float32)
        kn = (1 + 0.1 * r.standard_normal(128)).astype(np.float32)
        pos = 1234
        qo, ko = O.qwen_qk_norm_rope(qb, kb, qn, kn, pos, fmt)

        def ref(bits_, heads, norm):
            x = O.from_bits16(bits_, fmt).astype(np.float64).reshape(heads, 128)
            inv = 1.0 / np.sqrt(np.mean(x ** 2, axis=1, keepdims=True) + 1e-6)
            y = x * inv * norm
            # binary32 angle, as the reference forms it (pos as f32 * powf(...))
            freq = (1e6 ** (-np.arange(64) / 64.0)).astype(np.float32)
            ang = (np.float32(pos) * freq).astype(np.float64)
            s, c = np.sin(ang), np.cos(ang)
            lft, rgt = y[:, :64], y[:, 64:]
            return np.concatenate([lft * c - rgt * s, rgt * c + lft * s], axis=1)

        for got, bits_, heads, norm in ((qo, qb, 32, qn), (ko, kb, 4, kn)):
            g = O.from_bits16(got, fmt).reshape(heads, 128)
            rr = ref(bits_, heads, norm)
            half_ulp = 2.0 ** -11 if fmt == O.F16 else 2.0 ** -8
            # one RNE rounding of the output, plus binary32 arithmetic noise
            assert np.all(np.abs(g - rr) <= half_ulp * np.abs(rr) * 1.01 + 1e-5)


def test_qwen_prefill_rows_equal_decode():
    r = rng(12)
    T = 9
    q = r.standard_normal((T, 4096)).astype(np.float16).view(np.uint16)
    kc = r.standard_normal((T, 512)).astype(np.float16).view(np.uint16)
    vc = r.standard_normal((T, 512)).astype(np.float16).view(np.uint16)
    rows = [0, 3, 8]
    bits, _ = O.qwen_prefill_rows(q, kc, vc, 0, rows)
    for i, t in enumerate(rows):
        assert np.array_equal(bits[i], O.qwen_gqa_attention(q[t], kc[:t + 1], vc[:t + 1]))
    # rows dealt over threads come back in order, bit for bit
    many = [8, 0, 5, 3, 3, 7, 1]
    b1, f1 = O.qwen_prefill_rows(q, kc, vc, 0, many)
    b4, f4 = O.qwen_prefill_rows(q, kc, vc, 0, many, workers=4)
    assert np.array_equal(b1, b4) and np.array_equal(f1, f4)
    assert np.array_equal(b1[1], bits[0]) and np.array_equal(b1[3], bits[1]) and np.array_equal(b1[0], bits[2])


def test_oracle_rounding_against_exact_attention_grows_past_the_fp32_bar():
    """The reference's attention sums its softmax denominator and each output
    element as sequential binary32 folds (crates/qx-runtime/src/lib.rs:517,
    :540-548), so its own distance from exact attention grows with the
    context.  On twelve seeded N(0,1) caches it stays below 7e-6 x RMS at
    1000 positions (the fp32 bar of 1e-5 against it is then met by any
    accurate summation order) and passes 1e-5 at 4096 positions (only the
    reference's own order can meet the bar against it there)."""
    from tests.helpers import attend64, rel_err

    worst = {}
    for L in (1000, 4096):
        errs = []
        for seed in range(12):
            g = rng(1000 + seed)
            k = g.standard_normal((L, KVH, D), dtype=np.float32)
            v = g.standard_normal((L, KVH, D), dtype=np.float32)
            q = g.standard_normal((QH, D), dtype=np.float32)
            cache = O.KvCache(L)
            cache.extend(k, v)
            errs.append(rel_err(O.granite_attend(q.ravel(), cache, L), attend64(q, k, v, 0.015625).ravel()))
        worst[L] = max(errs)
    assert 3e-6 < worst[1000] < 7e-6, worst
    assert worst[4096] > 1e-5, worst
