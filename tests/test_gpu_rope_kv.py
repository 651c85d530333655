"""GPU parity: consensus math, fused RoPE + KV append, KV indexing.

Granite fp32 RoPE'd keys and queries must be bit-identical to the oracle
(KvCache::append of the rotated key, crates/qx-runtime/src/lib.rs:464-475);
fp16/bf16 caches hold exactly the RNE rounding of those bits.  KV indexing is
checked as a bijection against the reference's position-major index
(pos * KV_HEADS + head) * HEAD_DIM + d (lib.rs:407-415).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0").to(dtype)


def test_device_consensus_math_is_bit_exact(ctx):
    log("consensus conformance")
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        np.array([-87.0, -10.0, -1.0, 0.0, 1.0, 10.0, 88.0, 1e-6, 0.25, 2.0, 1024.0, -100.0, 100.0], np.float32),
        rng.uniform(-87, 88, 20000).astype(np.float32),
        np.exp(rng.uniform(-20, 20, 5000)).astype(np.float32),
    ])
    pos = rng.integers(0, 4097, xs.size).astype(np.uint32)
    pair = rng.integers(0, 32, xs.size).astype(np.uint32)
    pos[:4], pair[:4] = [0, 1, 4095, 4095], [0, 1, 0, 31]
    coords = np.stack([pos, pair], 1).ravel()
    with rt.Graph(ctx) as g:
        e, r, s, c = rt.consensus_conformance(g, dev(xs), dev(coords.view(np.int32), torch.int32))
    e, r, s, c = (t.cpu().numpy().view(np.uint32) for t in (e, r, s, c))
    for i, x in enumerate(xs):
        ref = O.exp_f32(x)
        if ref is not None:
            assert e[i] == O.f32_bits(ref), (x, hex(e[i]))
        ref = O.rsqrt_f32(x)
        if ref is not None:
            assert r[i] == O.f32_bits(ref), (x, hex(r[i]))
        sc = O.granite_rope_sin_cos(int(pos[i]), int(pair[i]))
        assert (s[i], c[i]) == (O.f32_bits(sc[0]), O.f32_bits(sc[1])), (pos[i], pair[i])
    # the reference's golden bits, straight from the device
    assert [hex(v) for v in e[:7]] == [hex(v) for v in [0x00B33687, 0x383E6BCE, 0x3EBC5AB2, 0x3F800000,
                                                        0x402DF854, 0x46AC14EF, 0x7EF882B7]]
    assert (s[2], c[2]) == (0xBF7F7136, 0xBD871E5E)


@pytest.mark.parametrize("kdt", [abi.F32, abi.F16, abi.BF16])
def test_granite_rope_append_matches_oracle_bits(ctx, kdt):
    log("granite rope append", kdt)
    rng = np.random.default_rng(2 + kdt)
    P = 48
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 64, kdt)
    ref = O.KvCache(64, kdt, kdt)
    q = rng.standard_normal((P, 1024)).astype(np.float32)
    k = rng.standard_normal((P, 512)).astype(np.float32)
    v = rng.standard_normal((P, 512)).astype(np.float32)
    qout = torch.empty((P, 1024), device="cuda:0")
    for p in range(P):
        with rt.Graph(ctx) as g:
            rt.rope_kv_batch(g, arena, 0, p, dev(q[p]).reshape(1, 1, 16, 64), dev(k[p]).reshape(1, 1, 8, 64),
                             dev(v[p]).reshape(1, 1, 8, 64), query_out=qout[p].view(1, 1, 16, 64))
        qr, kr = O.apply_granite_rope(q[p], k[p], p)
        ref.append(p, kr, v[p])
        assert np.array_equal(qout[p].cpu().numpy().view(np.uint32), qr.view(np.uint32)), p
    assert arena.len() == P
    with rt.Graph(ctx) as g:
        kk, vv = arena.gather(g, 0, 0, 0, P)
    assert np.array_equal(kk.float().cpu().numpy(), ref.keys())
    assert np.array_equal(vv.float().cpu().numpy(), ref.values())


def test_rope_kv_for_layer_in_place_like_the_reference_call_site(ctx):
    """GpuRuntimeBuffers::encode_attention_layer_with_plan passes `query` as
    both input and query_output (crates/qx-runtime-v2/src/lib.rs:6942-6952);
    the single-token C entry point must rotate in place and append layer 2."""
    log("rope_kv_for_layer in place")
    rng = np.random.default_rng(9)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 3, 1, 32, abi.F32)
    ref = O.KvCache(32)
    for p in range(6):
        q = rng.standard_normal(1024).astype(np.float32)
        k = rng.standard_normal(512).astype(np.float32)
        v = rng.standard_normal(512).astype(np.float32)
        qd, kd, vd = dev(q), dev(k), dev(v)
        with rt.Graph(ctx) as g:
            abi.check(abi.lib().qxh_encode_rope_kv_for_layer(g.handle, arena.handle, qd.data_ptr(), kd.data_ptr(),
                                                             vd.data_ptr(), qd.data_ptr(), 2, p))
        qr, kr = O.apply_granite_rope(q, k, p)
        ref.append(p, kr, v)
        assert np.array_equal(qd.cpu().numpy().view(np.uint32), qr.view(np.uint32)), p
        assert np.array_equal(kd.cpu().numpy(), k)  # the key input is left untouched
    assert arena.len(2, 0) == 6 and arena.len(0, 0) == 0
    with rt.Graph(ctx) as g:
        kk, vv = arena.gather(g, 2, 0, 0, 6)
    assert np.array_equal(kk.cpu().numpy(), ref.keys())
    assert np.array_equal(vv.cpu().numpy(), ref.values())


def test_batched_multi_token_append_and_cursors(ctx):
    log("batched append")
    rng = np.random.default_rng(5)
    S, T, start = 3, 5, 4
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 2, S, 16, abi.F32)
    arena.set_len(start)
    q = rng.standard_normal((S, T, 16, 64)).astype(np.float32)
    k = rng.standard_normal((S, T, 8, 64)).astype(np.float32)
    v = rng.standard_normal((S, T, 8, 64)).astype(np.float32)
    qo = torch.empty((S, T, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.rope_kv_batch(g, arena, 1, start, dev(q), dev(k), dev(v), query_out=qo)
    for s in range(S):
        assert arena.len(1, s) == start + T and arena.len(0, s) == start
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, 1, s, start, T)
        for t in range(T):
            qr, kr = O.apply_granite_rope(q[s, t].ravel(), k[s, t].ravel(), start + t)
            assert np.array_equal(qo[s, t].cpu().numpy().ravel(), qr)
            assert np.array_equal(kk[t].cpu().numpy().ravel(), kr)
            assert np.array_equal(vv[t].cpu().numpy(), v[s, t])


def test_append_rejects_out_of_order_and_overflow(ctx):
    # crates/qx-runtime/src/lib.rs:382-405, :2894-2901
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 2, abi.F32)
    z = torch.zeros((1, 1, 8, 64), device="cuda:0")
    zq = torch.zeros((1, 1, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="does not follow cache length"):
            rt.rope_kv_batch(g, arena, 0, 1, zq, z, z)
        rt.rope_kv_batch(g, arena, 0, 0, zq, z, z)
        rt.rope_kv_batch(g, arena, 0, 1, zq, z, z)
        with pytest.raises(abi.QxhError, match="exceeds context") as ei:
            rt.rope_kv_batch(g, arena, 0, 2, zq, z, z)
        assert ei.value.code == abi.QXH_ERR_KV_POSITION
    assert arena.len() == 2
    arena.rollback(0, 1)
    assert arena.len() == 1
    with pytest.raises(abi.QxhError, match="rollback"):
        arena.rollback(0, 2)
    arena.reset()
    assert arena.len() == 0


def test_head_major_index_is_a_bijection_of_the_reference_index(ctx):
    """Store rows whose values encode their own reference index, then read the
    raw arena: element (layer, seq, head, pos, d) must sit at
    ((((layer*S + seq)*H + head)*cap + pos)*D + d) and hold the value of
    reference index (pos*H + head)*D + d."""
    log("kv index bijection")
    S, L, cap, H, D = 2, 2, 12, 8, 64
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, L, S, cap, abi.F32)
    n = 10
    vals = np.arange(n * H * D, dtype=np.float32).reshape(1, n, H, D)
    with rt.Graph(ctx) as g:
        for layer in range(L):
            for s in range(S):
                off = float((layer * S + s) * 100000)
                kk = dev(vals + off)
                rt.store_kv(g, arena, layer, 0, kk, -kk, first_sequence=s)
    nbytes = L * S * H * cap * D * 4
    koff = arena.layout.keys - arena.arena.data_ptr()
    voff = arena.layout.values - arena.arena.data_ptr()
    kraw = arena.arena[koff:koff + nbytes].view(torch.float32).cpu().numpy().reshape(L, S, H, cap, D)
    vraw = arena.arena[voff:voff + nbytes].view(torch.float32).cpu().numpy().reshape(L, S, H, cap, D)
    pos, head, d = np.meshgrid(np.arange(n), np.arange(H), np.arange(D), indexing="ij")
    ref_index = (pos * H + head) * D + d
    for layer in range(L):
        for s in range(S):
            off = (layer * S + s) * 100000
            got = kraw[layer, s].transpose(1, 0, 2)[:n]  # [pos][head][d]
            assert np.array_equal(got, (ref_index + off).astype(np.float32))
            assert np.array_equal(vraw[layer, s].transpose(1, 0, 2)[:n], -(ref_index + off).astype(np.float32))
    assert arena.layout.head_stride == cap * D and arena.layout.sequence_stride == H * cap * D
    assert arena.layout.layer_stride == S * H * cap * D


def test_gather_rejects_rows_beyond_cursor(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 8, abi.F32)
    arena.set_len(3)
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="outside committed length"):
            arena.gather(g, 0, 0, 2, 2)


@pytest.mark.parametrize("fmt", [abi.F16, abi.BF16])
def test_qwen_norm_rope_append_matches_oracle(ctx, fmt):
    log("qwen norm rope append", fmt)
    rng = np.random.default_rng(7 + fmt)
    dt = torch.float16 if fmt == abi.F16 else torch.bfloat16
    ofmt = O.F16 if fmt == abi.F16 else O.BF16
    cap = 40000
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, cap, fmt)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    worst_ulps = 0
    mismatches = 0
    total = 0
    for pos in [0, 1, 37, 4095, 32767, 39999]:
        arena.set_len(pos, 0)
        qf = rng.standard_normal(4096).astype(np.float32)
        kf = rng.standard_normal(512).astype(np.float32)
        vf = rng.standard_normal(512).astype(np.float32)
        qb, kb, vb = O.to_bits16(qf, ofmt), O.to_bits16(kf, ofmt), O.to_bits16(vf, ofmt)
        qt = torch.from_numpy(qb.view(np.int16).copy()).cuda().view(dt).reshape(1, 1, 32, 128)
        kt = torch.from_numpy(kb.view(np.int16).copy()).cuda().view(dt).reshape(1, 1, 4, 128)
        vt = torch.from_numpy(vb.view(np.int16).copy()).cuda().view(dt).reshape(1, 1, 4, 128)
        qo = torch.empty_like(qt)
        with rt.Graph(ctx) as g:
            rt.rope_kv_batch(g, arena, 0, pos, qt, kt, vt, query_out=qo, query_norm=dev(qn), key_norm=dev(kn))
            kk, vv = arena.gather(g, 0, 0, pos, 1)
        rq, rk = O.qwen_qk_norm_rope(qb, kb, qn, kn, pos, ofmt)
        gq = qo.view(torch.int16).cpu().numpy().ravel().view(np.uint16)
        gk = kk.view(torch.int16).cpu().numpy().ravel().view(np.uint16)
        gv = vv.view(torch.int16).cpu().numpy().ravel().view(np.uint16)
        assert np.array_equal(gv, vb)
        for got, ref in ((gq, rq), (gk, rk)):
            d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
            worst_ulps = max(worst_ulps, int(d.max()))
            mismatches += int(np.count_nonzero(d))
            total += d.size
    log(f"qwen rope: worst {worst_ulps} ulp, {mismatches}/{total} elements differ")
    # the reference uses libm sin/cos and powf; the device uses its own sincos:
    # rounding may flip by one unit in the last place on rare elements
    assert worst_ulps <= 1 and mismatches <= 0.02 * total


def test_qwen_in_place_qk_norm_rope(ctx):
    rng = np.random.default_rng(9)
    qb = O.to_bits16(rng.standard_normal(4096), O.F16)
    kb = O.to_bits16(rng.standard_normal(512), O.F16)
    ones = np.ones(128, np.float32)
    from qx_amd import api
    gq, gk = api.run_qwen_qk_norm_rope(qb, kb, ones, ones, 37)
    rq, rk = O.qwen_qk_norm_rope(qb, kb, ones, ones, 37, O.F16)
    assert np.max(np.abs(gq.astype(np.int32) - rq.astype(np.int32))) <= 1
    assert np.max(np.abs(gk.astype(np.int32) - rk.astype(np.int32))) <= 1


def test_qwen_append_without_query_stores_the_same_rows():
    """A Qwen RoPE append with no query (only the cache rows wanted) stores
    the K/V rows bit for bit as the append with a query does; the query
    heads do nothing when there is no rotated query to write."""
    ctx = rt.Context(0)
    rng = np.random.default_rng(31)
    k = torch.from_numpy(rng.standard_normal((1, 3, 4, 128), dtype=np.float32)).cuda().half()
    v = torch.from_numpy(rng.standard_normal((1, 3, 4, 128), dtype=np.float32)).cuda().half()
    q = torch.from_numpy(rng.standard_normal((1, 3, 32, 128), dtype=np.float32)).cuda().half()
    rows = []
    for query, qout in ((q, torch.empty_like(q)), (None, None)):
        arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, 64, abi.F16)
        with rt.Graph(ctx) as g:
            rt.rope_kv_batch(g, arena, 0, 0, query, k, v, query_out=qout)
            rows.append(arena.gather(g, 0, 0, 0, 3))
    assert torch.equal(rows[0][0], rows[1][0]) and torch.equal(rows[0][1], rows[1][1])
