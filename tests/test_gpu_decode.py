"""GPU parity: split-K decode attention against the oracle.

Granite fp32 KV: max-abs error <= 1e-5 x output RMS against
granite_attention_decode (crates/qx-runtime/src/lib.rs:444-552).
fp16/bf16 KV: <= 2e-3 x RMS against the fp32 oracle on the same (rounded)
cache contents.  Qwen: against cpu_gqa_attention
(tools/qx-qwen-parity/src/main.rs:1218-1258).
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi, api
from qx_amd import runtime as rt
from tests.helpers import FP32_ORACLE_BAR_MAX_LENGTH, TOL_16, TOL_F32, attend64, check_fp32_bar, log, rel_err

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "granite_cfg1.npz")


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0").to(dtype)


def test_grouped_query_attention_uses_matching_kv_head():
    # crates/qx-runtime/src/lib.rs:2872-2892, through the reference-shaped API
    cache = api.KvCache(4)
    value = np.zeros((8, 64), np.float32)
    for h in range(8):
        value[h] = h + 1.0
    out = api.granite_attention_decode(np.zeros(1024), np.zeros(512), value.ravel(), 0, cache)
    assert len(cache) == 1
    for qh in range(16):
        assert np.all(out[qh * 64:(qh + 1) * 64] == qh // 2 + 1.0)


def test_kv_cache_rejects_non_sequential_positions():
    # crates/qx-runtime/src/lib.rs:2894-2901
    cache = api.KvCache(2)
    z = np.zeros(1024)
    with pytest.raises(abi.QxhError):
        api.granite_attention_decode(z, z[:512], z[:512], 1, cache)


def test_cfg1_positions_0_to_511_fp32(ctx):
    """Config 1: one Granite layer, positions 0..511 appended one at a time
    into an fp32 cache of capacity 512; every step's [16,64] output."""
    log("cfg1 decode 0..511")
    gold = np.load(GOLDEN)
    rng = np.random.default_rng(int(gold["seed"]))
    P = 512
    q = rng.standard_normal((P, 1024), dtype=np.float32)
    k = rng.standard_normal((P, 512), dtype=np.float32)
    v = rng.standard_normal((P, 512), dtype=np.float32)
    cache = api.KvCache(512)
    ref = O.KvCache(512)
    worst = 0.0
    checkpoints = list(gold["checkpoints"])
    for p in range(P):
        out = api.granite_attention_decode(q[p], k[p], v[p], p, cache)
        r = O.granite_attention_decode(q[p], k[p], v[p], p, ref)
        e = rel_err(out, r)
        worst = max(worst, e)
        assert e <= TOL_F32, (p, e)
        if p in checkpoints:
            i = checkpoints.index(p)
            assert np.array_equal(r, gold["outputs"][i])  # the oracle still reproduces the fixture
            assert rel_err(out, gold["outputs"][i]) <= TOL_F32
    log(f"cfg1 worst max-abs/rms = {worst:.3e}")
    kk, vv = cache.token_rows()
    assert np.array_equal(kk, ref.keys()) and np.array_equal(vv, ref.values())


@pytest.mark.parametrize("kdt,length", [(abi.F32, 1), (abi.F32, 4096), (abi.F16, 37), (abi.F16, 4096),
                                        (abi.BF16, 2049), (abi.F32, 1000)])
def test_granite_decode_lengths_and_dtypes(ctx, kdt, length):
    log("granite decode", kdt, length)
    rng = np.random.default_rng(100 + length + kdt)
    S = 3
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 2, S, 4096, kdt)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=length * 7 + kdt, length=length)
    q = dev(rng.standard_normal((S, 16, 64), dtype=np.float32))
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 1, q, length)
    tol = TOL_F32 if kdt == abi.F32 else TOL_16
    for s in range(S):
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 1, s, 0, length)
        kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
        ref_cache = O.KvCache(4096)
        ref_cache.extend(kf, vf)
        qs = q[s].cpu().numpy()
        r = O.granite_attend(qs.ravel(), ref_cache, length)
        got = out[s].cpu().numpy().ravel()
        e = rel_err(got, r)
        exact = attend64(qs, kf, vf, 0.015625).ravel()
        e_gpu, e_ora = rel_err(got, exact), rel_err(r, exact)
        log(f"seq {s}: gpu-oracle {e:.3e}  gpu-f64 {e_gpu:.3e}  oracle-f64 {e_ora:.3e}")
        if kdt == abi.F32:
            check_fp32_bar(got, r, exact, length)
        else:
            assert e <= tol, (s, e)


# The MFMA decode plan's boundaries (16-bit caches): Granite keeps one chunk
# per head up to 768 positions, or up to 2048 once the heads make 128 or more
# workgroups; Qwen up to 256, or 512 from 64 workgroups; past that the split
# count is at most 256 workgroups' worth, rounded down (3 sequences = 24
# Granite units: 7 splits at 769 positions, 8 at 4096; 16 sequences = 128
# units: 2 at 2049; Qwen, one sequence = 4 units: 3 at 257; 16 sequences = 64
# units: 3 at 513; 3 sequences = 12 units: 19 at 16384).  Each case against
# the oracle, and the plan's shape read from its workspace size (zero for
# one chunk).
@pytest.mark.parametrize("shape,kdt,S,L,single", [
    (abi.SHAPE_GRANITE, abi.F16, 3, 768, True), (abi.SHAPE_GRANITE, abi.F16, 3, 769, False),
    (abi.SHAPE_GRANITE, abi.BF16, 3, 4096, False), (abi.SHAPE_GRANITE, abi.F16, 16, 2048, True),
    (abi.SHAPE_GRANITE, abi.BF16, 16, 2049, False), (abi.SHAPE_QWEN3, abi.BF16, 1, 256, True),
    (abi.SHAPE_QWEN3, abi.F16, 1, 257, False), (abi.SHAPE_QWEN3, abi.BF16, 16, 512, True),
    (abi.SHAPE_QWEN3, abi.BF16, 16, 513, False), (abi.SHAPE_QWEN3, abi.BF16, 3, 16384, False)])
def test_mfma_decode_plan_boundaries(ctx, shape, kdt, S, L, single):
    log("mfma decode plan boundary", shape, kdt, S, L)
    info = rt.shape_info(shape)
    arena = rt.KvArena(ctx, shape, 1, S, L, kdt)
    dt = rt.torch_dtype(kdt)
    q = torch.empty((S, info.q_heads, info.head_dim), dtype=dt, device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=S * 131 + L, length=L)
        rt.fill_normal(g, q, seed=L + 5)
    ws = rt.attention_workspace_bytes(arena, S, L)
    units = S * info.kv_heads
    partial = units * (info.q_heads // info.kv_heads) * (info.head_dim + 2) * 4
    if single:
        assert ws == 0
    else:
        assert ws > 0 and ws % partial == 0
        splits = ws // partial
        assert splits >= 2 and units * splits <= 256, splits
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, q, L, out_dtype=torch.float32)
    tobits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().ravel().view(np.uint16)
    worst = 0.0
    for s in range(S):
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 0, s, 0, L)
        if shape == abi.SHAPE_GRANITE:
            ref_cache = O.KvCache(L)
            ref_cache.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
            r = O.granite_attend(q[s].float().cpu().numpy().ravel(), ref_cache, L)
        else:
            _, r = O.qwen_gqa_attention(tobits(q[s]), tobits(kk), tobits(vv), O.F16 if kdt == abi.F16 else O.BF16,
                                        want_f32=True)
        e = rel_err(out[s].cpu().numpy().ravel(), r)
        worst = max(worst, e)
        assert e <= TOL_16, (s, e)
    log(f"  workspace {ws} B, worst max-abs/rms {worst:.3e} over {S} sequences")


def fp32_cases(ctx, S, L, seed):
    """GPU decode of S fp32 sequences at length L; per sequence (gpu, oracle, exact)."""
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, L, abi.F32)
    q = torch.empty((S, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=seed, length=L)
        rt.fill_normal(g, q, seed=seed + 1)
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, q, L)
    for s in range(S):
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 0, s, 0, L)
        kf, vf = kk.cpu().numpy(), vv.cpu().numpy()
        ref_cache = O.KvCache(L)
        ref_cache.extend(kf, vf)
        qs = q[s].cpu().numpy()
        yield (out[s].cpu().numpy().ravel(), O.granite_attend(qs.ravel(), ref_cache, L),
               attend64(qs, kf, vf, 0.015625).ravel())


@pytest.mark.parametrize("S,L", [(1, 1), (256, 1), (1, 1000), (256, 1000)])
def test_fp32_decode_strict_bar_single_and_batched(ctx, S, L):
    """The north-star fp32 bar, unconditionally: every sequence of a single
    and a 256-sequence batch within 1e-5 x RMS of the oracle (split-K with a
    combine for one sequence, one split per unit for the batch)."""
    log("fp32 strict bar", S, L)
    assert L <= FP32_ORACLE_BAR_MAX_LENGTH
    worst = 0.0
    for got, r, exact in fp32_cases(ctx, S, L, seed=17 * L + S):
        e = rel_err(got, r)
        worst = max(worst, e)
        assert e <= TOL_F32, e
        assert rel_err(got, exact) <= TOL_F32 / 2
        if L == 1:
            assert np.array_equal(got, r)  # one position: out = v exactly
    log(f"  worst gpu-oracle {worst:.2e}")


@pytest.mark.parametrize("S", [1, 256])
def test_fp32_decode_at_4096_against_exact_attention(ctx, S):
    """At 4096 positions the reference's own sequential binary32 sums are up
    to 1.6e-5 x RMS from exact attention (pinned on the CPU by
    tests/test_oracle_attention.py), so there the bar is applied to exact
    (float64) attention at half its width, for every sequence; the distance
    to the oracle is logged."""
    log("fp32 at 4096", S)
    eg, eo, ef = [], [], []
    for got, r, exact in fp32_cases(ctx, S, 4096, seed=4096 + S):
        e, e_gpu, e_ora = check_fp32_bar(got, r, exact, 4096)
        eo.append(e), eg.append(e_gpu), ef.append(e_ora)
    log(f"  gpu-f64 max {max(eg):.2e}; gpu-oracle max {max(eo):.2e}; oracle-f64 max {max(ef):.2e}")


def test_cfg4_batched_fp16_decode_full_size(ctx):
    """Config 4 shape: 256 sequences x 4096 positions of fp16 KV (one layer here);
    sampled sequences against the oracle."""
    log("cfg4 256x4096 fp16")
    S, L = 256, 4096
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, L, abi.F16)
    q = torch.empty((S, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=4, length=L)
        rt.fill_normal(g, q, seed=44)
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, q, L)
    assert torch.isfinite(out).all()
    worst = 0.0
    for s in (0, 1, 128, 255):
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 0, s, 0, L)
        ref_cache = O.KvCache(L)
        ref_cache.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
        r = O.granite_attend(q[s].cpu().numpy().ravel(), ref_cache, L)
        e = rel_err(out[s].cpu().numpy().ravel(), r)
        worst = max(worst, e)
        assert e <= TOL_16
    log(f"  cfg4 worst max-abs/rms {worst:.3e} over sequences 0, 1, 128, 255")


def test_split_and_unsplit_agree(ctx):
    """Size-independent property: the same cache attended as 1 sequence
    (many splits) and inside a 256-sequence batch (one split) agree."""
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 256, 2048, abi.F32)
    q = torch.empty((256, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=9, length=2048)
        rt.fill_normal(g, q, seed=99)
        batched = rt.attention(g, arena, 0, q, 2048)
        single = rt.attention(g, arena, 0, q[7:8].contiguous(), 2048, first_sequence=7)
    assert rt.attention_workspace_bytes(arena, 1, 2048) > 0 == rt.attention_workspace_bytes(arena, 256, 2048)
    assert rel_err(single[0].cpu().numpy(), batched[7].cpu().numpy()) <= TOL_F32


def test_attention_length_beyond_cursor_is_rejected(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 64, abi.F32)
    arena.set_len(10)
    q = torch.zeros((1, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="exceeds committed length"):
            rt.attention(g, arena, 0, q, 11)


@pytest.mark.parametrize("fmt,ctxlen", [(abi.F16, 97), (abi.F16, 4096), (abi.BF16, 5000), (abi.BF16, 32768)])
def test_qwen_decode_matches_cpu_gqa_attention(ctx, fmt, ctxlen):
    log("qwen decode", fmt, ctxlen)
    dt = torch.float16 if fmt == abi.F16 else torch.bfloat16
    ofmt = O.F16 if fmt == abi.F16 else O.BF16
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, ctxlen, fmt)
    q = torch.empty((1, 32, 128), dtype=dt, device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=ctxlen + fmt, length=ctxlen)
        rt.fill_normal(g, q, seed=3)
        out32 = rt.attention(g, arena, 0, q, ctxlen, out_dtype=torch.float32)
        out16 = rt.attention(g, arena, 0, q, ctxlen)
        kk, vv = arena.gather(g, 0, 0, 0, ctxlen)
    tobits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().ravel().view(np.uint16)
    ref_bits, ref = O.qwen_gqa_attention(tobits(q), tobits(kk), tobits(vv), ofmt, want_f32=True)
    got = out32.cpu().numpy().ravel()
    e = rel_err(got, ref)
    log(f"qwen {fmt} {ctxlen}: fp32 output max-abs/rms {e:.3e}")
    # the tolerance applies to the attention arithmetic (fp32 output); the
    # 16-bit output is the RNE rounding of that same value
    assert e <= TOL_16
    assert np.array_equal(tobits(out16), O.to_bits16(got, ofmt))


def test_run_qwen_gqa_attention_mirror():
    rng = np.random.default_rng(21)
    n = 300
    q = O.to_bits16(rng.standard_normal(4096), O.F16)
    kc = O.to_bits16(rng.standard_normal(n * 512), O.F16)
    vc = O.to_bits16(rng.standard_normal(n * 512), O.F16)
    got = api.run_qwen_gqa_attention(q, kc, vc)
    _, ref = O.qwen_gqa_attention(q, kc, vc, O.F16, want_f32=True)
    assert rel_err(O.from_bits16(got, O.F16), ref) <= TOL_16


@pytest.mark.parametrize("kdt,start", [(abi.F32, 0), (abi.F32, 700), (abi.F16, 300), (abi.BF16, 1023),
                                       (abi.F32, 1500), (abi.F16, 2047)])
def test_decode_step_matches_the_two_call_path(ctx, kdt, start):
    """qxh_encode_decode_step_for_layer (one dispatch up to 1024 positions, the
    two-call path beyond) against qxh_encode_rope_kv_for_layer + attention on
    a twin cache: bit-identical appended K/V and rotated q, outputs within the
    dtype's tolerance of each other and of the oracle."""
    log("decode step", kdt, start)
    rng = np.random.default_rng(start + 10 * kdt)
    cap = 2048 + 8
    a1 = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, kdt)
    a2 = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, kdt)
    if start:
        with rt.Graph(ctx) as g:
            a1.fill_normal(g, seed=3, length=start)
            a2.fill_normal(g, seed=3, length=start)
    tol = TOL_F32 if kdt == abi.F32 else TOL_16
    for step in range(3):
        p = start + step
        q = dev(rng.standard_normal((16, 64), dtype=np.float32))
        k = dev(rng.standard_normal((8, 64), dtype=np.float32))
        v = dev(rng.standard_normal((8, 64), dtype=np.float32))
        qo1 = torch.empty_like(q)
        qo2 = torch.empty((1, 1, 16, 64), device="cuda:0")
        with rt.Graph(ctx) as g:
            out1 = rt.decode_step(g, a1, 0, p, q, k, v, query_out=qo1)
            rt.rope_kv_batch(g, a2, 0, p, q.view(1, 1, 16, 64), k.view(1, 1, 8, 64), v.view(1, 1, 8, 64),
                             query_out=qo2)
            out2 = rt.attention(g, a2, 0, qo2.view(1, 16, 64), p + 1)
            k1, v1 = a1.gather(g, 0, 0, 0, p + 1)
            k2, v2 = a2.gather(g, 0, 0, 0, p + 1)
        assert a1.len() == p + 1
        assert torch.equal(qo1, qo2.view(16, 64))
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
        e = rel_err(out1.cpu().numpy(), out2[0].cpu().numpy())
        ref = attend64(qo1.cpu().numpy(), k1.float().cpu().numpy(), v1.float().cpu().numpy(), 0.015625)
        e64 = rel_err(out1.cpu().numpy(), ref)
        log(f"decode step {kdt} p={p}: vs two-call {e:.2e}, vs float64 {e64:.2e}")
        assert e <= tol and e64 <= tol


def test_decode_step_rejects_out_of_order_positions(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 16, abi.F32)
    z = torch.zeros((16, 64), device="cuda:0")
    zk = torch.zeros((8, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="does not follow cache length"):
            rt.decode_step(g, arena, 0, 1, z, zk, zk)
