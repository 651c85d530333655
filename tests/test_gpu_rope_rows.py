"""GPU parity: the prompt front ends (RoPE + KV append of many token rows).

Calls of 16 rows or more (tokens x sequences) take the row kernels of
rope_append.hip: one wave per token row, 16-byte slices, sin/cos evaluated
once per row.  Granite rows must equal the oracle's apply_granite_rope
(crates/qx-runtime/src/lib.rs:434-441) bit for bit in every input, query and
cache dtype, like the per-head kernel; Qwen rows must equal the per-head
kernel bit for bit and stay within one unit in the last place of
cpu_qk_norm_rope (tools/qx-qwen-parity/src/main.rs:1170-1210) on at most 2%
of elements, values copied bit for bit
(the reference counterparts are encode_rope_kv_batch,
crates/qx-metal/src/lib.rs:8105-8174, and qx_qwen_qk_norm_rope,
kernels/qwen_attention.metal:138-177).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import log

pytestmark = pytest.mark.gpu

TORCH = {abi.F32: torch.float32, abi.F16: torch.float16, abi.BF16: torch.bfloat16}


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def rounded(a, dt):
    """float32 values rounded to `dt` (RNE) and widened back, on the CPU."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(TORCH[dt]).float().numpy()


def bits(t):
    t = t.detach().cpu()
    return t.view(torch.int32).numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy()


@pytest.mark.parametrize("idt", [abi.F32, abi.F16, abi.BF16])
@pytest.mark.parametrize("kdt,vdt", [(abi.F32, abi.F32), (abi.F16, abi.F16), (abi.BF16, abi.BF16),
                                     (abi.F32, abi.F16)])
def test_granite_rows_match_oracle_bits(ctx, idt, kdt, vdt):
    S, T, start, cap = 2, 40, 5, 64
    log(f"granite rows in={idt} k={kdt} v={vdt}")
    rng = np.random.default_rng(100 + 10 * idt + 3 * kdt + vdt)
    q = rounded(rng.standard_normal((S, T, 16, 64)), idt)
    k = rounded(rng.standard_normal((S, T, 8, 64)), idt)
    v = rounded(rng.standard_normal((S, T, 8, 64)), idt)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, cap, kdt, vdt)
    arena.set_len(start)
    qo = torch.empty((S, T, 16, 64), dtype=TORCH[idt], device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.rope_kv_batch(g, arena, 0, start, *(torch.from_numpy(a).cuda().to(TORCH[idt]) for a in (q, k, v)),
                         query_out=qo)
    qo = qo.float().cpu().numpy()
    for s in range(S):
        assert arena.len(0, s) == start + T
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 0, s, start, T)
        kk, vv = kk.float().cpu().numpy(), vv.float().cpu().numpy()
        for t in range(T):
            qr, kr = O.apply_granite_rope(q[s, t].ravel(), k[s, t].ravel(), start + t)
            assert np.array_equal(qo[s, t].ravel().view(np.uint32), rounded(qr, idt).view(np.uint32)), (s, t)
            assert np.array_equal(kk[t].ravel().view(np.uint32), rounded(kr, kdt).view(np.uint32)), (s, t)
            assert np.array_equal(vv[t].ravel().view(np.uint32), rounded(v[s, t].ravel(), vdt).view(np.uint32))


def test_granite_rows_without_query_and_misaligned_query(ctx):
    """No query: the cache rows alone, bit for bit as with a query.  A query
    that does not start on a 16-byte boundary takes the per-head kernel, with
    the same bits."""
    S, T = 1, 24
    rng = np.random.default_rng(7)
    q = rng.standard_normal((S, T, 16, 64)).astype(np.float32)
    k = rng.standard_normal((S, T, 8, 64)).astype(np.float32)
    v = rng.standard_normal((S, T, 8, 64)).astype(np.float32)
    qd = torch.from_numpy(q).cuda().half()
    kd, vd = torch.from_numpy(k).cuda().half(), torch.from_numpy(v).cuda().half()
    rows = []
    outs = []
    for case in ("aligned", "no-query", "misaligned"):
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, 32, abi.F16)
        if case == "misaligned":
            buf = torch.empty(qd.numel() + 1, dtype=torch.float16, device="cuda:0")
            qin = buf[1:].view(qd.shape)
            qin.copy_(qd)
            obuf = torch.empty_like(buf)
            qout = obuf[1:].view(qd.shape)
        else:
            qin, qout = (qd, torch.empty_like(qd)) if case == "aligned" else (None, None)
        with rt.Graph(ctx) as g:
            rt.rope_kv_batch(g, arena, 0, 0, qin, kd, vd, query_out=qout)
            rows.append(arena.gather(g, 0, 0, 0, T))
        if qout is not None:
            outs.append(qout.clone())
    for kk, vv in rows[1:]:
        assert torch.equal(kk, rows[0][0]) and torch.equal(vv, rows[0][1])
    assert torch.equal(outs[0], outs[1])
    for t in range(T):
        qr, kr = O.apply_granite_rope(q[0, t].ravel().astype(np.float16).astype(np.float32),
                                      k[0, t].ravel().astype(np.float16).astype(np.float32), t)
        assert np.array_equal(outs[0][0, t].cpu().numpy().ravel(), qr.astype(np.float16))


@pytest.mark.parametrize("fmt", [abi.F16, abi.BF16])
def test_qwen_rows_match_oracle(ctx, fmt):
    """Rows near the end of a 40,000-position cache and from position 0, two
    sequences; each row against cpu_qk_norm_rope, and the whole call against
    one-token calls of the per-head kernel, bit for bit (the row kernel sums
    the squares in the per-head kernel's tree).  Against the oracle: at most
    one unit in the last place on elements of at least 1/8 of the row RMS and
    on at most 2% of all elements; smaller elements (where the rotation
    cancels, so one unit of fp32 rounding in the inverse RMS is several units
    of a tiny 16-bit result) within 2^-10 (f16) or 2^-7 (bf16) of the row
    RMS."""
    log("qwen rows", fmt)
    rng = np.random.default_rng(17 + fmt)
    dt = TORCH[fmt]
    ofmt = O.F16 if fmt == abi.F16 else O.BF16
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    S, T, cap = 2, 24, 40000
    worst, mism, total, worst_abs = 0, 0, 0, 0.0
    for start in (0, cap - T):
        qb = O.to_bits16(rng.standard_normal((S, T, 32, 128)), ofmt)
        kb = O.to_bits16(rng.standard_normal((S, T, 4, 128)), ofmt)
        vb = O.to_bits16(rng.standard_normal((S, T, 4, 128)), ofmt)
        qt, kt, vt = (torch.from_numpy(b.view(np.int16).copy()).cuda().view(dt) for b in (qb, kb, vb))
        arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, S, cap, fmt)
        arena.set_len(start)
        qo = torch.empty_like(qt)
        qnd, knd = torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda()
        with rt.Graph(ctx) as g:
            rt.rope_kv_batch(g, arena, 0, start, qt, kt, vt, query_out=qo, query_norm=qnd, key_norm=knd)
        # the per-head kernel, one token at a time
        single = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, cap, fmt)
        single.set_len(start)
        qo1 = torch.empty_like(qt)
        with rt.Graph(ctx) as g:
            for t in range(T):
                rt.rope_kv_batch(g, single, 0, start + t, qt[:1, t:t + 1], kt[:1, t:t + 1], vt[:1, t:t + 1],
                                 query_out=qo1[:1, t:t + 1], query_norm=qnd, key_norm=knd)
        gq = bits(qo).view(np.uint16).reshape(S, T, -1)
        gq1 = bits(qo1).view(np.uint16).reshape(S, T, -1)
        assert np.array_equal(gq[0], gq1[0])
        with rt.Graph(ctx) as g:
            k1, v1 = single.gather(g, 0, 0, start, T)
        for s in range(S):
            with rt.Graph(ctx) as g:
                kk, vv = arena.gather(g, 0, s, start, T)
            gk = bits(kk).view(np.uint16).reshape(T, -1)
            gv = bits(vv).view(np.uint16).reshape(T, -1)
            assert np.array_equal(gv, vb[s].reshape(T, -1))
            if s == 0:
                assert np.array_equal(gk, bits(k1).view(np.uint16).reshape(T, -1))
            for t in range(T):
                rq, rk = O.qwen_qk_norm_rope(qb[s, t].ravel(), kb[s, t].ravel(), qn, kn, start + t, ofmt)
                for got, ref in ((gq[s, t], rq), (gk[t], rk)):
                    r = O.from_bits16(ref, ofmt).astype(np.float64)
                    e = np.abs(O.from_bits16(got, ofmt).astype(np.float64) - r)
                    rms = np.sqrt(np.mean(r * r))
                    d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
                    big = np.abs(r) >= rms / 8
                    worst = max(worst, int(d[big].max()))
                    if np.any(~big):
                        worst_abs = max(worst_abs, float(e[~big].max() / rms))
                    mism += int(np.count_nonzero(d))
                    total += d.size
    log(f"qwen rows: worst {worst} ulp on elements >= rms/8, {mism}/{total} elements differ, "
        f"worst |error| / rms below rms/8 {worst_abs:.2e}")
    assert worst <= 1 and mism <= 0.02 * total and worst_abs <= (2.0 ** -10 if fmt == abi.F16 else 2.0 ** -7)


def test_qwen_rows_fp32_input_match_per_head_kernel(ctx):
    """fp32 inputs and fp32 rotated queries into a bf16 cache: the row kernel
    against one-token calls of the per-head kernel (the same arithmetic up to
    the order of the per-head sum of squares: within 4 units of fp32 rounding
    of the largest element)."""
    rng = np.random.default_rng(23)
    S, T, start, cap = 1, 20, 1000, 1100
    q = torch.from_numpy(rng.standard_normal((S, T, 32, 128)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((S, T, 4, 128)).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal((S, T, 4, 128)).astype(np.float32)).cuda()
    outs, rows = [], []
    for per_token in (False, True):
        arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, S, cap, abi.BF16)
        arena.set_len(start)
        qo = torch.empty_like(q)
        with rt.Graph(ctx) as g:
            if per_token:
                for t in range(T):
                    rt.rope_kv_batch(g, arena, 0, start + t, q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1],
                                     query_out=qo[:, t:t + 1])
            else:
                rt.rope_kv_batch(g, arena, 0, start, q, k, v, query_out=qo)
            rows.append(arena.gather(g, 0, 0, start, T))
        outs.append(qo)
    assert torch.equal(rows[0][1], rows[1][1])
    d = (outs[0] - outs[1]).abs().max().item()
    assert d <= 4 * 2.0 ** -23 * outs[1].abs().max().item(), d
    kd = (rows[0][0].float() - rows[1][0].float()).abs()
    assert kd.max().item() <= 2.0 ** -7 * rows[1][0].float().abs().max().item()
