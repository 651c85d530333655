"""GPU parity for the tiered value cache (QXH_I8_TIERED): recent values in
f16, older values as INT8 blocks of 32 with f16 scales.  The reference only
proposes the format (docs/qx-structural-memory-2026-08-25.md:69-74), so the
check is against the oracle's restatement of this build's definition
(oracle.TieredValueCache, pinned in tests/test_oracle_tiered_v.py):

- cache contents bit for bit: the synthetic fill against its CPU
  restatement (oracle.tiered_fill_values); appends (RoPE append and store-only, every input dtype, appends
  longer than the window) and rollbacks against the tier model;
- attention (decode, batched decode and causal verifier rows) at the fp32 bar
  against the oracle fed the values the cache holds, which are exact in f32;
- the entries that do not serve tiered values refuse them.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_16, TOL_F32, attend64, check_fp32_bar, log, rel_err

pytestmark = pytest.mark.gpu

KVH, D = 8, 64


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def values(arena, layer, seq, length):
    with rt.Graph(arena.ctx) as g:
        kk, vv = arena.gather(g, layer, seq, 0, length)
    return kk, vv.cpu().numpy()


@pytest.mark.parametrize("length", [40, 300])
def test_tiered_fill_matches_its_restatement(ctx, length):
    """The synthetic fill: keys as for any cache, values from the integer
    generator oracle.tiered_fill_values, quantised below length - window."""
    log("tiered fill", length)
    W, S, cap = 64, 2, 512
    plain = rt.KvArena(ctx, abi.SHAPE_GRANITE, 2, S, cap, abi.F32, abi.F16)
    tiered = rt.KvArena(ctx, abi.SHAPE_GRANITE, 2, S, cap, abi.F32, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        plain.fill_normal(g, seed=11, length=length)
        tiered.fill_normal(g, seed=11, length=length)
    for layer in range(2):
        for seq in range(S):
            assert tiered.value_tier(layer, seq) == max(0, length - W)
            k16, _ = values(plain, layer, seq, length)
            kt, vt = values(tiered, layer, seq, length)
            assert torch.equal(k16, kt)
            src = np.stack([O.tiered_fill_values(11, (layer * S + seq) * KVH + h, cap, length)
                            for h in range(KVH)], axis=1)
            model = O.TieredValueCache(W)
            model.append(src.astype(np.float32))
            assert np.array_equal(vt.view(np.uint32), model.rows().view(np.uint32)), (layer, seq)


def test_tiered_appends_and_rollbacks_match_the_model(ctx):
    W, cap = 32, 600
    rng = np.random.default_rng(17)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 2, cap, abi.F32, abi.I8_TIERED, value_window=W)
    models = [O.TieredValueCache(W), O.TieredValueCache(W)]
    dtypes = [torch.float32, torch.float16, torch.bfloat16]
    step = 0
    for op in range(40):
        length = arena.len(0, 0)
        both = arena.len(0, 1) == length and arena.value_tier(0, 0) == arena.value_tier(0, 1)
        if length and rng.random() < 0.3:
            seq = int(rng.integers(0, 2))
            keep = int(rng.integers(0, arena.len(0, seq) + 1))
            arena.rollback(seq, keep)
            models[seq].rollback(keep)
            log(f"op {op}: rollback seq {seq} to {keep}")
        else:
            seqs = [0, 1] if both else [int(np.argmin([arena.len(0, 0), arena.len(0, 1)]))]
            start = arena.len(0, seqs[0])
            t = int(rng.choice([1, 1, 3, 31, 33, 70]))
            if start + t > cap:
                continue
            dt = dtypes[op % 3]
            k = torch.randn((len(seqs), t, KVH, D), device="cuda:0").to(dt)
            v = (torch.randn((len(seqs), t, KVH, D), device="cuda:0") * (0.5 + op)).to(dt)
            with rt.Graph(ctx) as g:
                if op % 2:
                    rt.store_kv(g, arena, 0, start, k, v, first_sequence=seqs[0])
                else:
                    rt.rope_kv_batch(g, arena, 0, start, None, k, v, first_sequence=seqs[0])
            for i, s in enumerate(seqs):
                models[s].append(v[i].float().cpu().numpy())
            log(f"op {op}: append {t} at {start} to {seqs} ({dt})")
        for s in range(2):
            m = models[s]
            assert arena.len(0, s) == m.length and arena.value_tier(0, s) == m.boundary, (op, s)
            if m.length:
                _, vt = values(arena, 0, s, m.length)
                assert np.array_equal(vt.view(np.uint32), m.rows().view(np.uint32)), (op, s)
        step += 1
    assert step > 20
    # set_len moves the cursor and never raises the boundary
    before = [arena.value_tier(0, s) for s in range(2)]
    arena.set_len(3)
    assert [arena.value_tier(0, s) for s in range(2)] == [min(b, 3) for b in before]


def test_tiered_set_len_cannot_raise_past_the_window(ctx):
    """A cursor raise on a tiered cache may only recommit rows that are still
    in the window: after a fill of 4096 rows (window 256) and set_len(100),
    set_len(4096) would claim rows [100, 4096) whose slots hold other rows."""
    W = 256
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 4096, abi.F32, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=7, length=4096)
    assert arena.value_tier() == 4096 - W
    arena.set_len(100)
    assert arena.value_tier() == 100 and arena.len() == 100
    with pytest.raises(abi.QxhError, match="value window") as ei:
        arena.set_len(4096)
    assert ei.value.code == abi.QXH_ERR_KV_POSITION
    assert arena.len() == 100 and arena.value_tier() == 100  # unchanged by the refused call
    arena.set_len(100 + W)  # every row of [100, 356) is still in its slot
    assert arena.len() == 100 + W and arena.value_tier() == 100


@pytest.mark.parametrize("kdt", [abi.F32, abi.F16])
@pytest.mark.parametrize("length", [1, 300, 4096])
def test_tiered_decode_matches_oracle(ctx, kdt, length):
    log("tiered decode", kdt, length)
    rng = np.random.default_rng(length + kdt)
    S, W = 2, 256
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, S, 4096, kdt, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=length + 5, length=length)
    q = dev(rng.standard_normal((S, 16, 64), dtype=np.float32))
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, q, length)
    for s in range(S):
        kk, vf = values(arena, 0, s, length)
        kf = kk.float().cpu().numpy()
        ref_cache = O.KvCache(4096)
        ref_cache.extend(kf, vf)
        qs = q[s].cpu().numpy()
        ref = O.granite_attend(qs.ravel(), ref_cache, length)
        e, _, _ = check_fp32_bar(out[s].cpu().numpy().ravel(), ref, attend64(qs, kf, vf, 0.015625).ravel(), length)
        log(f"  seq {s}: {e:.2e}")


@pytest.mark.parametrize("start,tokens", [(0, 4), (500, 4), (1000, 40)])
def test_tiered_causal_rows_match_oracle(ctx, start, tokens):
    """Verifier rows over a tiered cache whose last rows were appended by the
    RoPE append (and, for 40 rows past a window of 32, partly quantised on
    the way in)."""
    log("tiered causal rows", start, tokens)
    rng = np.random.default_rng(start + tokens)
    W = 32
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 1200, abi.F32, abi.I8_TIERED, value_window=W)
    if start:
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=13, length=start)
    k = dev(rng.standard_normal((1, tokens, KVH, D), dtype=np.float32))
    v = dev(rng.standard_normal((1, tokens, KVH, D), dtype=np.float32))
    with rt.Graph(ctx) as g:
        rt.rope_kv_batch(g, arena, 0, start, None, k, v)
    assert arena.value_tier() == max(0, start + tokens - W)
    kk, vf = values(arena, 0, 0, start + tokens)
    ref = O.KvCache(1200)
    ref.extend(kk.cpu().numpy(), vf)
    q = rng.standard_normal((tokens, 16, 64), dtype=np.float32)
    with rt.Graph(ctx) as g:
        out = rt.prefill_attention(g, arena, 0, start, dev(q))
    r = O.granite_prefill_rows(q.reshape(tokens, -1), ref, start, np.arange(tokens))
    e = rel_err(out.cpu().numpy().reshape(tokens, -1), r)
    log(f"  causal rows max-abs/rms {e:.2e}")
    assert e <= TOL_F32


def test_tiered_graph_replay_after_rollback(ctx):
    """A captured append + decode replayed after rolling back to its start:
    the row that left the window in the first replay has its slot taken by
    the appended row, so later replays must keep its codes (the slot tags)."""
    W, L = 32, 100
    rng = np.random.default_rng(23)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 256, abi.F32, abi.I8_TIERED, value_window=W)
    side = torch.cuda.Stream()
    k = dev(rng.standard_normal((1, 1, KVH, D), dtype=np.float32))
    v = dev(rng.standard_normal((1, 1, KVH, D), dtype=np.float32))
    q = dev(rng.standard_normal((1, 16, 64), dtype=np.float32))
    out = torch.empty_like(q)
    ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, L + 1), 1), dtype=torch.uint8, device="cuda:0")
    model = O.TieredValueCache(W)
    model.append(np.stack([O.tiered_fill_values(3, h, 256, L) for h in range(KVH)], axis=1).astype(np.float32))
    model.append(v[0].cpu().numpy())
    with torch.cuda.stream(side):
        with rt.Graph(ctx, side) as g:
            arena.fill_normal(g, seed=3, length=L)
        side.synchronize()
        g = rt.Graph(ctx, side)
        g.capture_begin()
        rt.rope_kv_batch(g, arena, 0, L, None, k, v)
        rt.attention(g, arena, 0, q, L + 1, out=out, workspace=ws)
        replay = g.capture_end()
        g.discard()
        first = None
        for i in range(3):
            out.zero_()
            side.synchronize()
            replay.launch(side)
            side.synchronize()
            if first is None:
                first = out.clone()
            assert torch.equal(out, first), i
            _, vt = values(arena, 0, 0, L + 1)
            assert arena.value_tier() == model.boundary == L + 1 - W
            assert np.array_equal(vt.view(np.uint32), model.rows().view(np.uint32)), i
            arena.rollback(0, L)
            arena.set_len(L + 1)  # the replay wrote row L again; the boundary stays at L + 1 - W
        del replay
    kk, vf = values(arena, 0, 0, L + 1)
    ref = O.KvCache(256)
    ref.extend(kk.cpu().numpy(), vf)
    assert rel_err(first.cpu().numpy().ravel(), O.granite_attend(q.cpu().numpy().ravel(), ref, L + 1)) <= TOL_F32


@pytest.mark.parametrize("kdt", [abi.BF16, abi.F16, abi.F32])
def test_tiered_qwen_shape(ctx, kdt):
    """Qwen (4 kv heads x 128 dims, G = 8): fill, a RoPE append longer than
    the window, batched decode and causal rows, against the tier model bit
    for bit and float64 attention.  Decode with 16-bit keys runs on the MFMA
    kernel, whose V tile holds the values rounded once to f16: the 16-bit
    bar; fp32 keys and the causal rows (VALU kernel, exact values): the fp32
    bar."""
    log("tiered qwen", kdt)
    W, S, cap, L, T = 64, 2, 1024, 700, 100
    rng = np.random.default_rng(29 + kdt)
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, S, cap, kdt, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=7, length=L)
    models = []
    for seq in range(S):
        m = O.TieredValueCache(W, 4, 128)
        m.append(np.stack([O.tiered_fill_values(7, seq * 4 + h, cap, L, 128) for h in range(4)], axis=1)
                 .astype(np.float32))
        models.append(m)
    k = dev(rng.standard_normal((S, T, 4, 128), dtype=np.float32)).to(rt.torch_dtype(kdt))
    v = dev(rng.standard_normal((S, T, 4, 128), dtype=np.float32)).to(rt.torch_dtype(kdt))
    with rt.Graph(ctx) as g:
        rt.rope_kv_batch(g, arena, 0, L, None, k, v)
    n = L + T
    kf, vf = [], []
    for seq in range(S):
        models[seq].append(v[seq].float().cpu().numpy())
        kk, vt = values(arena, 0, seq, n)
        assert arena.value_tier(0, seq) == models[seq].boundary == n - W
        assert np.array_equal(vt.view(np.uint32), models[seq].rows().view(np.uint32)), seq
        kf.append(kk.float().cpu().numpy())
        vf.append(vt)
    # queries in the key dtype (as the 16-bit decode tests pass them), so both
    # sides see the same q and only the value path differs
    q = torch.from_numpy(rng.standard_normal((S, 32, 128), dtype=np.float32)).to(rt.torch_dtype(kdt)).float().numpy()
    with rt.Graph(ctx) as g:
        out = rt.attention(g, arena, 0, dev(q), n).cpu().numpy()
    tol = TOL_F32 if kdt == abi.F32 else TOL_16
    for seq in range(S):
        e = rel_err(out[seq], attend64(q[seq], kf[seq], vf[seq], 1 / np.sqrt(128)))
        log(f"  decode seq {seq}: {e:.2e}")
        assert e <= tol
    rows = 6
    qr = rng.standard_normal((rows, 32, 128), dtype=np.float32)
    with rt.Graph(ctx) as g:
        pr = rt.prefill_attention(g, arena, 0, n - rows, dev(qr)).cpu().numpy()
    for t in range(rows):
        p = n - rows + t + 1
        assert rel_err(pr[t], attend64(qr[t], kf[0][:p], vf[0][:p], 1 / np.sqrt(128))) <= TOL_F32, t


@pytest.mark.parametrize("shape,kdt,start,T", [(abi.SHAPE_QWEN3, abi.BF16, 1000, 128), (abi.SHAPE_QWEN3, abi.F16, 1000, 128),
                                               (abi.SHAPE_GRANITE, abi.F16, 1000, 128),
                                               (abi.SHAPE_QWEN3, abi.BF16, 4000, 40), (abi.SHAPE_GRANITE, abi.F16, 1000, 40)])
def test_tiered_prefill_on_the_pipelined_kernel(ctx, shape, kdt, start, T):
    """Prompt rows over a tiered cache with 16-bit keys take the pipelined
    MFMA prefill (beyond a few rows; 40 rows at these contexts are past the
    decode-row crossover), its V^T pre-pass building f16 tiles from both
    tiers; the 16-bit bar against float64 attention over the cached values."""
    log("tiered prefill", shape, kdt, start, T)
    hq, hkv, d = (32, 4, 128) if shape == abi.SHAPE_QWEN3 else (16, 8, 64)
    scale = 1 / np.sqrt(128) if shape == abi.SHAPE_QWEN3 else 0.015625
    W, cap = 256, start + T
    rng = np.random.default_rng(41 + shape + kdt)
    dt = rt.torch_dtype(kdt)
    arena = rt.KvArena(ctx, shape, 1, 1, cap, kdt, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=9, length=start)
    k = dev(rng.standard_normal((1, T, hkv, d), dtype=np.float32)).to(dt)
    v = dev(rng.standard_normal((1, T, hkv, d), dtype=np.float32)).to(dt)
    with rt.Graph(ctx) as g:
        rt.store_kv(g, arena, 0, start, k, v)
    assert arena.value_tier() == start + T - W
    q = dev(rng.standard_normal((T, hq, d), dtype=np.float32)).to(dt)
    with rt.Graph(ctx) as g:
        # fp32 output: a 16-bit output alone is ~1e-2 (bf16) of RMS off float64
        out = rt.prefill_attention(g, arena, 0, start, q, out_dtype=torch.float32).cpu().numpy()
    kk, vf = values(arena, 0, 0, start + T)
    kf, qf = kk.float().cpu().numpy(), q.float().cpu().numpy()
    worst = 0.0
    for t in sorted({0, 1, min(63, T - 1), min(64, T - 1), T // 2, T - 1}):
        n = start + t + 1
        worst = max(worst, rel_err(out[t], attend64(qf[t], kf[:n], vf[:n], scale)))
    log(f"  worst row max-abs/rms {worst:.2e}")
    assert worst <= TOL_16


def test_tiered_granite_q4_block(ctx):
    """The Granite attention half with Q4 weights on a tiered cache: the QKV
    kernel leaves the new V row to the tiered append, which demotes the row
    leaving the window.  The cache against the tier model bit for bit (the new
    row bit-equal to the same block's row on an Fp32KFp16V cache), the
    attention at the fp32 bar against the oracle over the cached rows, and
    the o projection + residual of the GPU's attention bit for bit."""
    from tests.test_gpu_q4 import HID, assert_bits, device_layer, q4_weights, workspace_query_and_attention
    rng = np.random.default_rng(47)
    nw, mats = q4_weights(rng)
    layer = device_layer(nw, mats)
    W, cap, p = 64, 512, 300
    tiered = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F32, abi.I8_TIERED, value_window=W)
    plain = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F32, abi.F16)
    with rt.Graph(ctx) as g:
        tiered.fill_normal(g, seed=5, length=p)
        plain.fill_normal(g, seed=5, length=p)
    h = dev(rng.standard_normal(HID, dtype=np.float32))
    outs, wsps = [], []
    for arena in (tiered, plain):
        out = torch.empty(HID, device="cuda:0")
        wsp = torch.zeros(rt.granite_block_workspace_bytes(arena, p + 1), dtype=torch.uint8, device="cuda:0")
        with rt.Graph(ctx) as g:
            rt.granite_attention_block_q4(g, arena, 0, p, layer, h, out, wsp)
        outs.append(out.cpu().numpy())
        wsps.append(wsp)
    assert tiered.len() == p + 1 and tiered.value_tier() == p + 1 - W
    kk, vt = values(tiered, 0, 0, p + 1)
    _, v16 = values(plain, 0, 0, p + 1)
    assert np.array_equal(vt[p].view(np.uint32), v16[p].astype(np.float32).view(np.uint32))
    model = O.TieredValueCache(W)
    model.append(np.stack([O.tiered_fill_values(5, hh, cap, p) for hh in range(KVH)], axis=1).astype(np.float32))
    model.append(vt[p][None])
    assert np.array_equal(vt.view(np.uint32), model.rows().view(np.uint32))
    q_gpu, att_gpu = workspace_query_and_attention(wsps[0])
    ref = O.KvCache(cap)
    ref.extend(kk.cpu().numpy(), vt)
    att_ref = O.granite_attend(q_gpu, ref, p + 1)
    e = rel_err(att_gpu, att_ref)
    log(f"tiered q4 block attention max-abs/rms {e:.2e}")
    assert e <= TOL_F32
    assert_bits(outs[0], O.granite_residual(h.cpu().numpy(), O.q4_mat_vec_simd32(mats[3], att_gpu)),
                "o projection + residual")


def test_tiered_granite_fp32_block(ctx):
    """The fp32-weight Granite attention half on a tiered cache: the new V
    row bit-equal to the same block's row on an Fp32KFp16V cache, the cache
    against the tier model, the attention at the fp32 bar against the oracle
    over the cached rows."""
    from tests.test_gpu_mixed_kv import granite_weights
    rng = np.random.default_rng(53)
    nw, ws = granite_weights(rng)
    layer = rt.GraniteLayer(dev(nw), *[dev(w) for w in ws])
    W, cap, p = 32, 256, 100
    tiered = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F32, abi.I8_TIERED, value_window=W)
    plain = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F32, abi.F16)
    with rt.Graph(ctx) as g:
        tiered.fill_normal(g, seed=6, length=p)
        plain.fill_normal(g, seed=6, length=p)
    h = dev(rng.standard_normal(1024, dtype=np.float32))
    wsps = []
    for arena in (tiered, plain):
        out = torch.empty(1024, device="cuda:0")
        wsp = torch.zeros(rt.granite_block_workspace_bytes(arena, p + 1), dtype=torch.uint8, device="cuda:0")
        with rt.Graph(ctx) as g:
            rt.granite_attention_block(g, arena, 0, p, layer, h, out, wsp)
        wsps.append(wsp)
    assert tiered.value_tier() == p + 1 - W
    kk, vt = values(tiered, 0, 0, p + 1)
    _, v16 = values(plain, 0, 0, p + 1)
    assert np.array_equal(vt[p].view(np.uint32), v16[p].astype(np.float32).view(np.uint32))
    model = O.TieredValueCache(W)
    model.append(np.stack([O.tiered_fill_values(6, hh, cap, p) for hh in range(KVH)], axis=1).astype(np.float32))
    model.append(vt[p][None])
    assert np.array_equal(vt.view(np.uint32), model.rows().view(np.uint32))
    w = wsps[0][:2 * 1024 * 4].view(torch.float32).cpu().numpy()
    ref = O.KvCache(cap)
    ref.extend(kk.cpu().numpy(), vt)
    assert rel_err(w[1024:], O.granite_attend(w[:1024], ref, p + 1)) <= TOL_F32


def test_tiered_qwen_block(ctx):
    """The Qwen attention half (Q4 projections) on a tiered cache with f16
    keys: the value row reaches the cache through the tiered append (the
    window row it leaves quantised), attention on the MFMA tiered decode.
    The cache against the tier model with the new row equal to the block's
    own V stage bit for bit; attention against float64 over the cached rows
    and the o projection of the GPU's attention against the oracle, at the
    16-bit bar."""
    from tests.test_gpu_qwen_block import err16, f16, weights, workspace_stages
    rng = np.random.default_rng(59)
    mats, _, layer = weights(rng)
    W, cap, pos = 64, 512, 300
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, cap, abi.F16, abi.I8_TIERED, value_window=W)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=4, length=pos)
    h = rng.standard_normal(2048).astype(np.float16)
    after = torch.empty(2048, dtype=torch.int16, device="cuda:0")
    moe = torch.empty_like(after)
    wsp = torch.zeros(rt.qwen_block_workspace_bytes(arena, pos + 1), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.qwen_attention_block(g, arena, 0, pos, layer, dev(h.view(np.int16)), after, moe, wsp)
    assert arena.len() == pos + 1 and arena.value_tier() == pos + 1 - W
    _, _, v, qrot, att, proj = workspace_stages(wsp)
    kk, vt = values(arena, 0, 0, pos + 1)
    assert np.array_equal(vt[pos].ravel().view(np.uint32), f16(v).view(np.uint32))
    model = O.TieredValueCache(W, 4, 128)
    model.append(np.stack([O.tiered_fill_values(4, hh, cap, pos, 128) for hh in range(4)], axis=1).astype(np.float32))
    model.append(vt[pos][None])
    assert np.array_equal(vt.view(np.uint32), model.rows().view(np.uint32))
    kf = kk.float().cpu().numpy()
    ref_att = attend64(f16(qrot).reshape(32, 128), kf, vt, 1 / np.sqrt(128)).ravel()
    e_att = err16(f16(att), ref_att)
    log(f"tiered qwen block attention err16 {e_att:.2e}")
    assert e_att <= TOL_16
    ref_proj = O.q4_mat_vec(mats[3], f16(att)).astype(np.float16).astype(np.float32)
    assert err16(f16(proj), ref_proj) <= TOL_16


def test_tiered_decode_step_is_the_two_call_path(ctx):
    """qxh_encode_decode_step_for_layer on a tiered cache: the same bits as
    the RoPE append + attention calls on an identically filled cache."""
    rng = np.random.default_rng(61)
    q, k, v = (dev(rng.standard_normal(s, dtype=np.float32)) for s in ((16, 64), (8, 64), (8, 64)))
    outs = []
    for step in (True, False):
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 256, abi.F32, abi.I8_TIERED, value_window=32)
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=8, length=100)
        qo = torch.empty_like(q)
        ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, 101), 1), dtype=torch.uint8, device="cuda:0")
        with rt.Graph(ctx) as g:
            if step:
                out = rt.decode_step(g, arena, 0, 100, q, k, v, query_out=qo, workspace=ws)
            else:
                rt.rope_kv_batch(g, arena, 0, 100, q[None, None], k[None, None], v[None, None], query_out=qo[None, None])
                out = rt.attention(g, arena, 0, qo[None], 101, workspace=ws)[0]
        assert arena.len() == 101 and arena.value_tier() == 101 - 32
        outs.append(out)
    assert torch.equal(outs[0], outs[1])


def test_tiered_values_are_refused_where_unsupported(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 2, 256, abi.F32, abi.I8_TIERED, value_window=32)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=3, length=100)
    q = torch.zeros((16, 64), device="cuda:0")
    kv = torch.zeros((8, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        # the decode step takes the two-call path on a tiered cache, which
        # needs the rotated query's buffer
        with pytest.raises(abi.QxhError, match="tiered value cache needs query_output"):
            rt.decode_step(g, arena, 0, 100, q, kv, kv)
        with pytest.raises(abi.QxhError, match="tiered"):
            arena.leaf_hashes(g, 0, 0, 4)
    # sequences whose boundaries differ cannot share a launch: sequence 0
    # rolled back to 50 and refilled to 60 keeps boundary 50, sequence 1
    # rolled back from 100 to 60 has boundary min(68, 60)
    arena.rollback(0, 50)
    with rt.Graph(ctx) as g:
        k = torch.zeros((1, 10, KVH, D), device="cuda:0")
        rt.store_kv(g, arena, 0, 50, k, k)
    arena.rollback(1, 60)
    assert arena.len(0, 0) == arena.len(0, 1) == 60
    assert arena.value_tier(0, 0) == 50 and arena.value_tier(0, 1) == 60
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="boundaries differ"):
            rt.attention(g, arena, 0, torch.zeros((2, 16, 64), device="cuda:0"), 60)
        out = rt.attention(g, arena, 0, torch.zeros((1, 16, 64), device="cuda:0"), 60, first_sequence=1)
    assert torch.isfinite(out).all()
