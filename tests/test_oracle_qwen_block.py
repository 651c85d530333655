"""Pins of the oracle's Qwen attention-half pieces: QuantizedTensor::mat_vec
(crates/qx-quant/src/lib.rs:851-891), the parity tool's rms_norm
(tools/qx-qwen-parity/src/main.rs:1157-1168) and the stage composition the
parity tool checks (main.rs:124-240).

- mat_vec: one nonzero column returns that column exactly; inputs where the
  sequential fma chain and the 32-lane tree give different float32 sums pin
  the sequential order; float64 bound.
- rms_norm: an input whose left-fold sum of squares differs from any tree
  order in float32 pins the fold; float64 bound.
- the block: a float64 restatement of the whole attention half (dequantised
  weights, per-head RMSNorm, RoPE with theta = 1e6, GQA softmax, residual,
  post-attention norm) within the reference's own relative-L2 bar of 0.01
  (main.rs:23-24), the f16 roundings between stages being the difference.
"""
import math

import numpy as np

from oracle import oracle as O
from tests.test_oracle_q4 import BIG, decode_numpy, one_group

HID = 2048


def rng(seed):
    return np.random.default_rng(seed)


def test_mat_vec_single_column_and_sequential_order():
    r = rng(1)
    m = O.q4_quantize((0.05 * r.standard_normal((6, 96))).astype(np.float32))
    deq = decode_numpy(m)
    for c in (0, 1, 31, 32, 95):
        e = np.zeros(96, np.float32)
        e[c] = 1.0
        assert np.array_equal(O.q4_mat_vec(m, e), deq[:, c])
    codes = np.full(32, 7, np.uint8)
    codes[[0, 8, 24]] = 8
    x = np.zeros(32, np.float32)
    x[0], x[8], x[24] = BIG, 1.0, 1.0
    g = one_group(codes)
    # sequential: 2^24 + 1 -> 2^24, twice; the 32-lane tree adds 1 + 1 first
    assert O.q4_mat_vec(g, x)[0] == BIG
    assert O.q4_mat_vec_simd32(g, x)[0] == np.float32(16777218.0)


def test_mat_vec_against_float64():
    r = rng(2)
    m = O.q4_quantize((0.02 * r.standard_normal((32, HID))).astype(np.float32))
    x = r.standard_normal(HID).astype(np.float32)
    deq = decode_numpy(m).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    bound = HID * 2.0 ** -24 * (np.abs(deq) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(O.q4_mat_vec(m, x) - ref) <= bound)


def test_rms_norm_left_fold_and_float64():
    # [4096, 1, 1, 0]: the left fold gives 2^24 exactly (each +1 is lost), so
    # the mean is 2^22 and the inverse 1/2048; a tree would add 1 + 1 first.
    x = np.array([4096.0, 1.0, 1.0, 0.0], np.float32)
    out = O.qwen_rms_norm(x, np.ones(4, np.float32))
    assert out[0] == np.float32(2.0) and out[1] == np.float32(1.0 / 2048)
    r = rng(3)
    h = r.standard_normal(HID).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(HID)).astype(np.float32)
    got = O.qwen_rms_norm(h, w)
    ref = h.astype(np.float64) / math.sqrt(np.mean(h.astype(np.float64) ** 2) + 1e-6) * w
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(ref))


def qwen_weights(r):
    mats = [O.q4_quantize((0.02 * r.standard_normal(s)).astype(np.float32))
            for s in ((4096, HID), (512, HID), (512, HID), (HID, 4096))]
    norms = [(1 + 0.05 * r.standard_normal(n)).astype(np.float32) for n in (HID, 128, 128, HID)]
    return mats, norms


def block64(h, mats, norms, pos, kc, vc):
    """float64 attention half; kc, vc: [pos][4][128] earlier rows (float64)."""
    wq, wk, wv, wo = (decode_numpy(m).astype(np.float64) for m in mats)
    in_norm, qn, kn, post = (n.astype(np.float64) for n in norms)

    def rms(v, w):
        return v / math.sqrt(np.mean(v ** 2) + 1e-6) * w

    a = rms(h, in_norm)
    q, k, v = (wq @ a).reshape(32, 128), (wk @ a).reshape(4, 128), (wv @ a).reshape(4, 128)
    freq = (1e6 ** (-np.arange(64) / 64.0)).astype(np.float32)
    ang = (np.float32(pos) * freq).astype(np.float64)
    s, c = np.sin(ang), np.cos(ang)

    def norm_rope(x, w):
        y = x / np.sqrt(np.mean(x ** 2, axis=1, keepdims=True) + 1e-6) * w
        lft, rgt = y[:, :64], y[:, 64:]
        return np.concatenate([lft * c - rgt * s, rgt * c + lft * s], axis=1)

    q, k = norm_rope(q, qn), norm_rope(k, kn)
    K = np.concatenate([kc, k[None]]) if pos else k[None]
    V = np.concatenate([vc, v[None]]) if pos else v[None]
    att = np.zeros((32, 128))
    for hq in range(32):
        sc = K[:, hq // 8, :] @ q[hq] / math.sqrt(128.0)
        wgt = np.exp(sc - sc.max())
        att[hq] = (wgt / wgt.sum()) @ V[:, hq // 8, :]
    after = h + wo @ att.ravel()
    return after, rms(after, post)


def test_qwen_block_matches_float64():
    r = rng(4)
    mats, norms = qwen_weights(r)
    pos = 37
    kc = r.standard_normal((pos, 4, 128)).astype(np.float16)
    vc = r.standard_normal((pos, 4, 128)).astype(np.float16)
    h = r.standard_normal(HID).astype(np.float16)
    st = O.qwen_attention_block(h.view(np.uint16), norms[0], *mats[:3], norms[1], norms[2], mats[3], norms[3], pos,
                                kc.view(np.uint16), vc.view(np.uint16))
    after, moe = block64(h.astype(np.float64), mats, norms, pos, kc.astype(np.float64), vc.astype(np.float64))
    for got, ref in ((st["hidden_after_attention"], after), (st["moe_input"], moe)):
        g = got.astype(np.float64)
        assert np.linalg.norm(g - ref) <= 0.01 * np.linalg.norm(ref)
    # the update itself (after - hidden), which the hidden state would mask
    upd, ref_upd = st["projection"].astype(np.float64), after - h.astype(np.float64)
    assert np.linalg.norm(upd - ref_upd) <= 0.01 * np.linalg.norm(ref_upd)
    # the stored key row is the rotated key, the value row the raw projection
    assert st["key_rotated"].shape == (512,) and st["value"].shape == (512,)
