"""GPU parity: the Granite attention block (config 2's per-layer unit) against
the oracle's attention half of GraniteLayerWeights::decode_with_trace
(crates/qx-runtime/src/lib.rs:847-923), and HIP-graph replay consistency."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_F32, log, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def weights(rng):
    nw = (1.0 + 0.05 * rng.standard_normal(1024)).astype(np.float32)
    wq = (0.02 * rng.standard_normal((1024, 1024))).astype(np.float32)
    wk = (0.02 * rng.standard_normal((512, 1024))).astype(np.float32)
    wv = (0.02 * rng.standard_normal((512, 1024))).astype(np.float32)
    wo = (0.02 * rng.standard_normal((1024, 1024))).astype(np.float32)
    return nw, wq, wk, wv, wo


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_block_sequence_matches_oracle(ctx):
    log("granite block 0..23")
    rng = np.random.default_rng(31)
    LAYERS, P = 2, 24
    ws_np = [weights(rng) for _ in range(LAYERS)]
    layers = [rt.GraniteLayer(*[dev(w) for w in ws]) for ws in ws_np]
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, 1, 64, abi.F32)
    refs = [O.KvCache(64) for _ in range(LAYERS)]
    ws = torch.empty(rt.granite_block_workspace_bytes(arena, 64), dtype=torch.uint8, device="cuda:0")
    worst = 0.0
    for p in range(P):
        h = rng.standard_normal(1024, dtype=np.float32)
        cur = dev(h)
        ref = h
        for layer in range(LAYERS):
            nxt = torch.empty(1024, device="cuda:0")
            with rt.Graph(ctx) as g:
                rt.granite_attention_block(g, arena, layer, p, layers[layer], cur, nxt, ws)
            ref = O.granite_attention_block(ref, *ws_np[layer], p, refs[layer])
            e = rel_err(nxt.cpu().numpy(), ref)
            worst = max(worst, e)
            assert e <= TOL_F32, (p, layer, e)
            cur = nxt
    log(f"block worst max-abs/rms {worst:.3e}")
    for layer in range(LAYERS):
        assert arena.len(layer) == P
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, layer, 0, 0, P)
        assert rel_err(kk.cpu().numpy(), refs[layer].keys()) <= TOL_F32
        assert rel_err(vv.cpu().numpy(), refs[layer].values()) <= TOL_F32


def test_block_at_position_4095_with_prefilled_cache(ctx):
    """Config 2's timed unit: a new token at position 4095 over a cache holding
    4095 N(0,1) positions."""
    log("granite block @4095")
    rng = np.random.default_rng(32)
    w_np = weights(rng)
    layer = rt.GraniteLayer(*[dev(w) for w in w_np])
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 4096, abi.F32)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=3, length=4095)
        kk, vv = arena.gather(g, 0, 0, 0, 4095)
    ref = O.KvCache(4096)
    ref.extend(kk.cpu().numpy(), vv.cpu().numpy())
    h = rng.standard_normal(1024, dtype=np.float32)
    out = torch.empty(1024, device="cuda:0")
    ws = torch.empty(rt.granite_block_workspace_bytes(arena, 4096), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.granite_attention_block(g, arena, 0, 4095, layer, dev(h), out, ws)
    r = O.granite_attention_block(h, *w_np, 4095, ref)
    e = rel_err(out.cpu().numpy(), r)
    log(f"block@4095 max-abs/rms {e:.3e}")
    assert e <= TOL_F32


def test_captured_block_replays_match_eager(ctx):
    """HIP-graph replay of 3 layers, replayed 4 times with eager work between
    replays; every replay equals the eager result bit for bit."""
    rng = np.random.default_rng(33)
    LAYERS, POS = 3, 100
    layers = [rt.GraniteLayer(*[dev(w) for w in weights(rng)]) for _ in range(LAYERS)]
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, 1, 128, abi.F32)
    hid = [torch.empty(1024, device="cuda:0") for _ in range(LAYERS + 1)]
    hid[0].copy_(dev(rng.standard_normal(1024, dtype=np.float32)))
    ws = torch.empty(rt.granite_block_workspace_bytes(arena, POS + 1), dtype=torch.uint8, device="cuda:0")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with rt.Graph(ctx, side) as g:
            arena.fill_normal(g, seed=8, length=POS)
            for layer in range(LAYERS):
                rt.granite_attention_block(g, arena, layer, POS, layers[layer], hid[layer], hid[layer + 1], ws)
        eager = hid[-1].clone()
        arena.rollback(0, POS)
        g = rt.Graph(ctx, side)
        g.capture_begin()
        for layer in range(LAYERS):
            rt.granite_attention_block(g, arena, layer, POS, layers[layer], hid[layer], hid[layer + 1], ws)
        replay = g.capture_end()
        g.discard()
        for i in range(4):
            hid[-1].zero_()
            side.synchronize()
            replay.launch(side)
            side.synchronize()
            assert torch.equal(hid[-1], eager), i
            scratch = torch.randn(4096, device="cuda:0")  # unrelated eager work between replays
            _ = (scratch * 2).sum().item()
