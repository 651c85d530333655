"""The oracle's row loops (the CPU baseline of the prompt front ends) equal
its per-token functions bit for bit."""
import numpy as np

from oracle import oracle as O


def test_granite_rope_rows_equal_per_token_calls():
    g = np.random.default_rng(1)
    q = g.standard_normal((7, 1024), dtype=np.float32)
    k = g.standard_normal((7, 512), dtype=np.float32)
    qr, kr = O.apply_granite_rope_rows(q, k, 4090)
    for t in range(7):
        a, b = O.apply_granite_rope(q[t], k[t], 4090 + t)
        assert np.array_equal(qr[t].view(np.uint32), a.view(np.uint32))
        assert np.array_equal(kr[t].view(np.uint32), b.view(np.uint32))


def test_qwen_norm_rope_rows_equal_per_token_calls():
    g = np.random.default_rng(2)
    for fmt in (O.F16, O.BF16):
        qb = O.to_bits16(g.standard_normal((5, 4096)), fmt)
        kb = O.to_bits16(g.standard_normal((5, 512)), fmt)
        qn = (1 + 0.1 * g.standard_normal(128)).astype(np.float32)
        kn = (1 + 0.1 * g.standard_normal(128)).astype(np.float32)
        qo, ko = O.qwen_qk_norm_rope_rows(qb, kb, qn, kn, 32760, fmt)
        for t in range(5):
            a, b = O.qwen_qk_norm_rope(qb[t], kb[t], qn, kn, 32760 + t, fmt)
            assert np.array_equal(qo[t], a) and np.array_equal(ko[t], b)
