"""GPU parity for caches whose K and V dtypes differ: the reference's Granite
KV plans Fp32KFp16V (the canonical default) and Fp16KFp32V
(KvPrecision, crates/qx-format/src/lib.rs:136-141; kernels
qx_v2_rope_kv_simd_kf32_vf16 and qx_v2_attention_v_partial_gqa_f16,
kernels/v2_decode.metal), plus their bf16 twins, and causal rows (the K-wide
verifier) on fp32 and mixed caches.

All attention math runs in fp32 on values the cache holds exactly, so the
fp32 bar (1e-5 x output RMS) applies against the oracle fed the same rounded
rows.  Cache rows and digests compare bit for bit.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_16, TOL_F32, attend64, check_fp32_bar, log, rel_err

pytestmark = pytest.mark.gpu

MIXED = [(abi.F32, abi.F16), (abi.F32, abi.BF16), (abi.F16, abi.F32), (abi.BF16, abi.F32)]
FMT = {abi.F32: O.F32, abi.F16: O.F16, abi.BF16: O.BF16}


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("kdt,vdt", MIXED)
@pytest.mark.parametrize("length", [1, 300, 4096])
def test_mixed_decode_matches_oracle(ctx, kdt, vdt, length):
    log("mixed decode", kdt, vdt, length)
    rng = np.random.default_rng(7 * length + 3 * kdt + vdt)
    S = 2
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, 4096, kdt, vdt)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=length + kdt, length=length)
    q = dev(rng.standard_normal((S, 16, 64), dtype=np.float32))
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, q, length)
    for s in range(S):
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 0, s, 0, length)
        assert kk.dtype == rt.torch_dtype(kdt) and vv.dtype == rt.torch_dtype(vdt)
        kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
        ref_cache = O.KvCache(4096)
        ref_cache.extend(kf, vf)
        qs = q[s].cpu().numpy()
        ref = O.granite_attend(qs.ravel(), ref_cache, length)
        e, _, _ = check_fp32_bar(out[s].cpu().numpy().ravel(), ref, attend64(qs, kf, vf, 0.015625).ravel(), length)
        log(f"  seq {s}: {e:.2e}")


@pytest.mark.parametrize("kdt,vdt", [(abi.F32, abi.F16), (abi.F16, abi.F32)])
@pytest.mark.parametrize("start", [0, 700, 1500])
def test_mixed_decode_step(ctx, kdt, vdt, start):
    """One-dispatch step (and the two-call path past 1024): appended rows
    rounded per dtype, bit-identical to the oracle's append."""
    log("mixed decode step", kdt, vdt, start)
    rng = np.random.default_rng(start + kdt)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 2048, kdt, vdt)
    if start:
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=4, length=start)
            kk, vv = arena.gather(g, 0, 0, 0, start)
    ref = O.KvCache(2048, FMT[kdt], FMT[vdt])
    if start:
        ref.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
    for step in range(3):
        p = start + step
        q, k, v = (rng.standard_normal(n, dtype=np.float32) for n in ((16, 64), (8, 64), (8, 64)))
        with rt.Graph(ctx) as g:
            qo = torch.empty((16, 64), device="cuda:0")  # past 1024 positions the step needs it
            out = rt.decode_step(g, arena, 0, p, dev(q), dev(k), dev(v), query_out=qo)
            kk, vv = arena.gather(g, 0, 0, p, 1)
        r = O.granite_attention_decode(q.ravel(), k.ravel(), v.ravel(), p, ref)
        assert np.array_equal(kk.float().cpu().numpy(), ref.keys()[p:p + 1])
        assert np.array_equal(vv.float().cpu().numpy(), ref.values()[p:p + 1])
        e = rel_err(out.cpu().numpy().ravel(), r)
        assert e <= TOL_F32, (p, e)


@pytest.mark.parametrize("kdt,vdt", [(abi.F32, abi.F32), (abi.F32, abi.F16), (abi.F16, abi.F32)])
@pytest.mark.parametrize("start,tokens", [(300, 4), (0, 64), (1000, 3)])
def test_causal_rows_on_fp32_and_mixed_caches(ctx, kdt, vdt, start, tokens):
    """K-wide verifier rows (encode_attention_batch_with_plan,
    crates/qx-metal/src/lib.rs:8206-8267) on caches the MFMA prefill does not
    take: row t attends [0, start + t], as granite_prefill_rows."""
    log("causal rows", kdt, vdt, start, tokens)
    rng = np.random.default_rng(start + tokens + kdt)
    cap = 1200
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, kdt, vdt)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=11, length=start + tokens)
        kk, vv = arena.gather(g, 0, 0, 0, start + tokens)
    ref = O.KvCache(cap)
    ref.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
    q = rng.standard_normal((tokens, 16, 64), dtype=np.float32)
    with rt.Graph(ctx) as g:
        out = rt.prefill_attention(g, arena, 0, start, dev(q))
    r = O.granite_prefill_rows(q.reshape(tokens, -1), ref, start, np.arange(tokens))
    e = rel_err(out.cpu().numpy().reshape(tokens, -1), r)
    log(f"  causal rows max-abs/rms {e:.2e}")
    assert e <= TOL_F32


def test_qwen_causal_rows_on_fp32_cache(ctx):
    """Qwen shape (D = 128, G = 8) through the same path, against float64."""
    rng = np.random.default_rng(5)
    start, tokens = 200, 5
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, 512, abi.F32)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=12, length=start + tokens)
        kk, vv = arena.gather(g, 0, 0, 0, start + tokens)
    kf, vf = kk.cpu().numpy(), vv.cpu().numpy()
    q = rng.standard_normal((tokens, 32, 128), dtype=np.float32)
    with rt.Graph(ctx) as g:
        out = rt.prefill_attention(g, arena, 0, start, dev(q)).cpu().numpy()
    for t in range(tokens):
        exact = attend64(q[t], kf[:start + t + 1], vf[:start + t + 1], 1 / np.sqrt(128))
        assert rel_err(out[t], exact) <= TOL_F32, t


def granite_weights(rng):
    nw = (1.0 + 0.05 * rng.standard_normal(1024)).astype(np.float32)
    ws = [(0.02 * rng.standard_normal(s)).astype(np.float32) for s in ((1024, 1024), (512, 1024), (512, 1024),
                                                                       (1024, 1024))]
    return nw, ws


def test_granite_block_on_fp32k_fp16v_cache(ctx):
    """The fp32-weight attention block on the canonical KV plan: K rows fp32,
    V rows fp16, against the oracle cache with the same store rounding."""
    rng = np.random.default_rng(61)
    nw, ws = granite_weights(rng)
    layer = rt.GraniteLayer(dev(nw), *[dev(w) for w in ws])
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 32, abi.F32, abi.F16)
    ref = O.KvCache(32, O.F32, O.F16)
    wsp = torch.empty(rt.granite_block_workspace_bytes(arena, 32), dtype=torch.uint8, device="cuda:0")
    for p in range(12):
        h = rng.standard_normal(1024, dtype=np.float32)
        out = torch.empty(1024, device="cuda:0")
        with rt.Graph(ctx) as g:
            rt.granite_attention_block(g, arena, 0, p, layer, dev(h), out, wsp)
        r = O.granite_attention_block(h, nw, *ws, p, ref)
        assert rel_err(out.cpu().numpy(), r) <= TOL_F32, p
    with rt.Graph(ctx) as g:
        kk, vv = arena.gather(g, 0, 0, 0, 12)
    assert vv.dtype == torch.float16
    assert rel_err(kk.cpu().numpy(), ref.keys()) <= TOL_F32
    # the fp32 projections differ from the oracle's left fold in the last bits,
    # which can move a value across an fp16 rounding boundary: the fp16 bar
    assert rel_err(vv.float().cpu().numpy(), ref.values()) <= TOL_16


# The fp32-weight block on equal 16-bit caches runs its attention on the MFMA
# decode: one chunk at 701 positions, split past 768 (1001 and 2501).
@pytest.mark.parametrize("kdt,position", [(abi.F16, 700), (abi.F16, 1000), (abi.BF16, 2500)])
def test_granite_block_on_16bit_cache(ctx, kdt, position):
    """The block output against the oracle's block over a cache with the same
    store rounding, and its attention (the workspace's merged attention for
    its own rotated query) against granite_attend over the rows the cache
    holds, at the 16-bit bar."""
    log("granite block on a 16-bit cache", kdt, position)
    rng = np.random.default_rng(63 + position)
    nw, ws = granite_weights(rng)
    layer = rt.GraniteLayer(dev(nw), *[dev(w) for w in ws])
    L = position + 1
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, L, kdt)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=position, length=position)
    h = rng.standard_normal(1024, dtype=np.float32)
    out = torch.empty(1024, device="cuda:0")
    wsp = torch.zeros(rt.granite_block_workspace_bytes(arena, L), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.granite_attention_block(g, arena, 0, position, layer, dev(h), out, wsp)
        kk, vv = arena.gather(g, 0, 0, 0, L)
    kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
    fmt = O.F16 if kdt == abi.F16 else O.BF16
    ref = O.KvCache(L, fmt, fmt)
    ref.extend(kf[:position], vf[:position])
    r = O.granite_attention_block(h, nw, *ws, position, ref)
    assert rel_err(out.cpu().numpy(), r) <= TOL_16
    w = wsp[:2 * 1024 * 4].view(torch.float32).cpu().numpy()
    q_rot, att = w[:1024], w[1024:]
    held = O.KvCache(L, fmt, fmt)
    held.extend(kf, vf)
    e = rel_err(att, O.granite_attend(q_rot, held, L))
    log(f"  attention vs oracle {e:.3e}")
    assert e <= TOL_16


def test_q4_block_on_fp32k_fp16v_cache(ctx):
    """The Q4 attention block on the canonical KV plan: K rows (norm, Q4
    projection, RoPE) and fp16-rounded V rows bit for bit."""
    rng = np.random.default_rng(62)
    nw = (1.0 + 0.05 * rng.standard_normal(1024)).astype(np.float32)
    mats = [O.q4_quantize((0.02 * rng.standard_normal(s)).astype(np.float32))
            for s in ((1024, 1024), (512, 1024), (512, 1024), (1024, 1024))]
    layer = rt.GraniteQ4Layer(dev(nw), *[rt.Q4Matrix(dev(m.packed), dev(m.scales.view(np.int16)), m.rows, m.cols)
                                         for m in mats])
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 32, abi.F32, abi.F16)
    ref = O.KvCache(32, O.F32, O.F16)
    wsp = torch.empty(rt.granite_block_workspace_bytes(arena, 32), dtype=torch.uint8, device="cuda:0")
    for p in range(12):
        h = rng.standard_normal(1024, dtype=np.float32)
        out = torch.empty(1024, device="cuda:0")
        with rt.Graph(ctx) as g:
            rt.granite_attention_block_q4(g, arena, 0, p, layer, dev(h), out, wsp)
        r, _, _, _ = O.granite_q4_attention_block(h, nw, *mats, p, ref)
        assert rel_err(out.cpu().numpy(), r) <= TOL_F32, p
    with rt.Graph(ctx) as g:
        kk, vv = arena.gather(g, 0, 0, 0, 12)
    assert np.array_equal(kk.cpu().numpy(), ref.keys())
    assert np.array_equal(vv.float().cpu().numpy(), ref.values())


def row_bytes(t):
    return t.contiguous().cpu().view(torch.uint8).numpy().tobytes()


@pytest.mark.parametrize("shape,kdt,vdt", [(abi.SHAPE_GRANITE, abi.F32, abi.F16), (abi.SHAPE_GRANITE, abi.F16, abi.F32),
                                           (abi.SHAPE_QWEN3, abi.F32, abi.BF16)])
def test_mixed_kv_leaf_and_verification_hashes(ctx, shape, kdt, vdt):
    """kv_leaf_hash_v1 over the stored K and V row bytes (2048 and 1024 bytes:
    eight and four chunks), and the per-token verification digests."""
    log("mixed hashes", shape, kdt, vdt)
    layers, cap, seqs = 3, 80, 2
    arena = rt.KvArena(ctx, shape, layers, seqs, cap, kdt, vdt)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=21, length=cap)
        got = arena.leaf_hashes(g, 2, 9, 45, first_sequence=0, sequences=2).cpu().numpy()
        rows = [arena.gather(g, 2, s, 9, 45) for s in range(seqs)]
    for s, (kk, vv) in enumerate(rows):
        for i in range(45):
            assert got[s, i].tobytes() == O.kv_leaf_hash_v1(2, 9 + i, row_bytes(kk[i]), row_bytes(vv[i])), (s, i)
    stride, token = 4096, 33
    res = torch.randint(0, 256, ((layers + 1) * stride,), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        dig = arena.verification_hashes(g, res, stride, token, layers, 2, sequence=1)
        vrows = [arena.gather(g, l, 1, token, 1) for l in range(layers)]
    ref = O.verification_hashes(res.cpu().numpy().tobytes(), stride, [row_bytes(k[0]) for k, _ in vrows],
                                [row_bytes(v[0]) for _, v in vrows], token, layers, 2)
    assert dig.cpu().numpy().tobytes() == ref


@pytest.mark.parametrize("kdt,vdt", [(abi.F32, abi.F32)] + MIXED)
def test_short_single_sequence_attention(ctx, kdt, vdt):
    """One sequence at contexts up to 320 positions takes the one-dispatch
    attention (one workgroup per kv head, 4 or 8 waves by length), longer
    ones the split path: every length class and both sides of the 320
    boundary against the oracle at the fp32 bar, a 16-bit query and a bf16
    output once each, and the split path (the same sequence inside a
    two-sequence call) within the bar of it."""
    rng = np.random.default_rng(100 + 5 * kdt + vdt)
    for length in (1, 37, 128, 129, 320, 321, 500, 1024):
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 2, 1024, kdt, vdt)
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=length, length=length)
            kk, vv = arena.gather(g, 0, 0, 0, length)
        kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
        ref_cache = O.KvCache(1024)
        ref_cache.extend(kf, vf)
        qn = rng.standard_normal((16, 64), dtype=np.float32)
        q16 = length == 129
        qt = dev(qn).half() if q16 else dev(qn)
        qf = qt.float().cpu().numpy()
        out_dt = torch.bfloat16 if length == 500 else torch.float32
        out = torch.empty((1, 16, 64), dtype=out_dt, device="cuda:0")
        with rt.Graph(ctx) as g:
            rt.attention(g, arena, 0, qt[None], length, out=out)
        ref = O.granite_attend(qf.ravel(), ref_cache, length)
        got = out.float().cpu().numpy().ravel()
        if out_dt == torch.bfloat16:
            want = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
            assert np.max(np.abs(got - want)) <= 2.0 ** -8 * np.max(np.abs(want)) + 1e-6, length
        else:
            e, _, _ = check_fp32_bar(got, ref, attend64(qf, kf, vf, 0.015625).ravel(), length)
            log(f"short attention {kdt}/{vdt} L={length}: {e:.2e}")
        # sequence 0 again inside a two-sequence call, which takes the split path
        two = torch.empty((2, 16, 64), device="cuda:0")
        q2 = torch.stack([qt.float(), qt.float()])
        with rt.Graph(ctx) as g:
            rt.attention(g, arena, 0, q2, length, out=two)
        if out_dt == torch.float32:
            assert rel_err(two[0].cpu().numpy().ravel(), got) <= TOL_F32
