"""GPU parity: the Qwen attention half with Q4 projections
(qxh_encode_qwen_attention_block) against the oracle, stage by stage as the
reference's parity tool checks it (tools/qx-qwen-parity/src/main.rs:124-240):
each stage is compared with the oracle fed the GPU's own previous stage, at
the 16-bit tolerance (2e-3 x RMS); the residual add is bit-exact; and the
whole block end to end against the oracle's own composition."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi, api
from qx_amd import runtime as rt
from tests.helpers import TOL_16, log

pytestmark = pytest.mark.gpu

HID = 2048


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_device(m: O.Q4Matrix) -> rt.Q4Matrix:
    return rt.Q4Matrix(dev(m.packed), dev(m.scales.view(np.int16)), m.rows, m.cols)


def f16(t):
    return t.cpu().numpy().view(np.float16).astype(np.float32)


def err16(got, ref):
    """max (|got - ref| - one f16 ulp of ref) / rms(ref), floored at 0: the
    16-bit bar for outputs both sides round to f16.  Two values within the bar
    before rounding can land one f16 ulp apart after it, and on the largest
    elements one ulp alone is ~2.4e-3 x RMS."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.maximum(np.abs(got - ref) - ulp, 0.0))) / max(rms, 1e-30)


def weights(rng):
    mats = [O.q4_quantize((0.02 * rng.standard_normal(s)).astype(np.float32))
            for s in ((4096, HID), (512, HID), (512, HID), (HID, 4096))]
    norms = [(1 + 0.05 * rng.standard_normal(n)).astype(np.float32) for n in (HID, 128, 128, HID)]
    layer = rt.QwenQ4Layer(dev(norms[0]), *[to_device(m) for m in mats[:3]], dev(norms[1]), dev(norms[2]),
                           to_device(mats[3]), dev(norms[3]))
    return mats, norms, layer


def workspace_stages(wsp):
    """The block's workspace starts with f16 query, key, value (before RoPE),
    rotated query, attention [4096] and o projection [2048]."""
    w = wsp[:30720].view(torch.int16)
    cuts = np.cumsum([0, 4096, 512, 512, 4096, 4096, 2048])
    return [w[cuts[i]:cuts[i + 1]] for i in range(6)]


@pytest.mark.parametrize("pos", [0, 37, 3000])
def test_qwen_block_stages(ctx, pos):
    log("qwen block", pos)
    rng = np.random.default_rng(pos + 5)
    mats, norms, layer = weights(rng)
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, 3072, abi.F16)
    if pos:
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=8, length=pos)
    h = rng.standard_normal(HID).astype(np.float16)
    after = torch.empty(HID, dtype=torch.int16, device="cuda:0")
    moe = torch.empty_like(after)
    wsp = torch.zeros(rt.qwen_block_workspace_bytes(arena, pos + 1), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.qwen_attention_block(g, arena, 0, pos, layer, dev(h.view(np.int16)), after, moe, wsp)
        kk, vv = arena.gather(g, 0, 0, 0, pos + 1)
    assert arena.len(0) == pos + 1
    q, k, v, qrot, att, proj = workspace_stages(wsp)
    hf = h.astype(np.float32)
    # 1. norm + Q4 q/k/v (the GPU's lane order against the sequential fold)
    a = O.qwen_rms_norm(hf, norms[0]).astype(np.float16).astype(np.float32)
    for got, m in ((q, mats[0]), (k, mats[1]), (v, mats[2])):
        ref = O.q4_mat_vec(m, a).astype(np.float16).astype(np.float32)
        assert err16(f16(got), ref) <= TOL_16
    # 2. per-head norm + RoPE of the GPU's q/k; the cache holds rotated k and raw v
    qn, kn = O.qwen_qk_norm_rope(q.cpu().numpy().view(np.uint16), k.cpu().numpy().view(np.uint16), norms[1],
                                 norms[2], pos, O.F16)
    assert err16(f16(qrot), qn.view(np.float16).astype(np.float32)) <= TOL_16
    kr = kk[pos].cpu().numpy().ravel()
    assert err16(kr.astype(np.float32), kn.view(np.float16).astype(np.float32)) <= TOL_16
    assert np.array_equal(vv[pos].cpu().numpy().ravel().view(np.uint16), v.cpu().numpy().view(np.uint16))
    # 3. attention of the GPU's rotated q over the cache as stored
    ref_att = O.qwen_gqa_attention(qrot.cpu().numpy().view(np.uint16), kk.cpu().numpy().view(np.uint16),
                                   vv.cpu().numpy().view(np.uint16), O.F16)
    e_att = err16(f16(att), ref_att.view(np.float16).astype(np.float32))
    assert e_att <= TOL_16
    # 4. Q4 o projection of the GPU's attention
    ref_proj = O.q4_mat_vec(mats[3], f16(att)).astype(np.float16).astype(np.float32)
    assert err16(f16(proj), ref_proj) <= TOL_16
    # 5. residual: f16(hidden + projection), bit for bit
    ref_after = (hf + f16(proj)).astype(np.float16)
    assert np.array_equal(after.cpu().numpy().view(np.uint16), ref_after.view(np.uint16))
    # 6. post-attention norm of the GPU's hidden_after
    ref_moe = O.qwen_rms_norm(ref_after.astype(np.float32), norms[3]).astype(np.float16).astype(np.float32)
    assert err16(f16(moe), ref_moe) <= TOL_16
    # end to end against the oracle's own composition
    st = O.qwen_attention_block(h.view(np.uint16), norms[0], *mats[:3], norms[1], norms[2], mats[3], norms[3], pos,
                                kk[:pos].cpu().numpy().view(np.uint16), vv[:pos].cpu().numpy().view(np.uint16))
    e_upd = err16(f16(proj), st["projection"].astype(np.float32))
    e_moe = err16(f16(moe), st["moe_input"].astype(np.float32))
    log(f"  attention {e_att:.2e}  update end-to-end {e_upd:.2e}  moe_input end-to-end {e_moe:.2e}")
    # the update has passed four f16 stages on each side
    assert e_upd <= 2 * TOL_16 and e_moe <= TOL_16
    assert err16(f16(after), st["hidden_after_attention"].astype(np.float32)) <= TOL_16


def bf16_bits_of(x32):
    """float32 -> bfloat16 bits, round to nearest even (no NaNs here)."""
    u = np.asarray(x32, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


# On equal 16-bit caches the block's per-head norm, RoPE and K/V append run
# inside its attention launch.  Position 0 (one row), 31 (the last row of a
# full tile), 32 (the first row of wave 1's tile), 512 (the lone row of the
# last of five 128-position splits), 700 (six splits, the new row in a
# partial last tile) and 32767 (64 splits, the last row of the cache).
@pytest.mark.parametrize("kdt,pos", [(abi.F16, 0), (abi.F16, 31), (abi.BF16, 32), (abi.F16, 512), (abi.F16, 700),
                                     (abi.BF16, 3000), (abi.F16, 32767)])
def test_qwen_block_front_end_inside_the_attention_launch(ctx, kdt, pos):
    """The rotated query matches the standalone front end
    (qxh_run_qwen_qk_norm_rope) bit for bit, and so does the stored key on an
    f16 cache (a bf16 cache rounds the same float once to bf16: within one
    bf16 step of the f16 value); the stored value row is the projection's;
    and the attention equals the plain decode of that rotated query over the
    cache as stored, bit for bit, so the launch used the row it stored."""
    log("qwen block front end in the attention launch", kdt, pos)
    rng = np.random.default_rng(pos + 17 * kdt)
    _, norms, layer = weights(rng)
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, pos + 1, kdt)
    if pos:
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=pos + 1, length=pos)
    h = rng.standard_normal(HID).astype(np.float16)
    after = torch.empty(HID, dtype=torch.int16, device="cuda:0")
    moe = torch.empty_like(after)
    wsp = torch.zeros(rt.qwen_block_workspace_bytes(arena, pos + 1), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.qwen_attention_block(g, arena, 0, pos, layer, dev(h.view(np.int16)), after, moe, wsp)
        kk, vv = arena.gather(g, 0, 0, pos, 1)
    q, k, v, qrot, att, _ = workspace_stages(wsp)
    qo, ko = api.run_qwen_qk_norm_rope(q.cpu().numpy().view(np.uint16), k.cpu().numpy().view(np.uint16), norms[1],
                                       norms[2], pos, O.F16)
    assert np.array_equal(qrot.cpu().numpy().view(np.uint16), qo)
    k_row = kk.contiguous().view(torch.int16).cpu().numpy().ravel().view(np.uint16)
    v_row = vv.contiguous().view(torch.int16).cpu().numpy().ravel().view(np.uint16)
    v16 = v.cpu().numpy().view(np.uint16)
    if kdt == abi.F16:
        assert np.array_equal(k_row, ko)
        assert np.array_equal(v_row, v16)
    else:
        kf = ko.view(np.float16).astype(np.float32)
        kb = (k_row.astype(np.uint32) << 16).view(np.float32)
        assert np.all(np.abs(kb - kf) <= np.abs(kf) * 2.0 ** -8 + 1e-30)
        assert np.array_equal(v_row, bf16_bits_of(v16.view(np.float16).astype(np.float32)))
    qt = qrot.view(torch.float16).reshape(1, 32, 128).contiguous()
    with rt.Graph(ctx) as g:
        plain = rt.attention(g, arena, 0, qt, pos + 1, out_dtype=torch.float16)
    assert torch.equal(plain.reshape(-1).view(torch.int16), att)


def test_qwen_block_graph_replay_is_deterministic(ctx):
    rng = np.random.default_rng(9)
    _, _, layer = weights(rng)
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 2, 1, 256, abi.F16)
    hs = [torch.empty(HID, dtype=torch.int16, device="cuda:0") for _ in range(3)]
    moe = torch.empty(HID, dtype=torch.int16, device="cuda:0")
    hs[0].copy_(dev(rng.standard_normal(HID).astype(np.float16).view(np.int16)))
    wsp = torch.empty(rt.qwen_block_workspace_bytes(arena, 201), dtype=torch.uint8, device="cuda:0")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with rt.Graph(ctx, side) as g:
            arena.fill_normal(g, seed=3, length=200)
            for layer_i in range(2):
                rt.qwen_attention_block(g, arena, layer_i, 200, layer, hs[layer_i], hs[layer_i + 1], moe, wsp)
        eager, eager_moe = hs[2].clone(), moe.clone()
        arena.rollback(0, 200)
        g = rt.Graph(ctx, side)
        g.capture_begin()
        for layer_i in range(2):
            rt.qwen_attention_block(g, arena, layer_i, 200, layer, hs[layer_i], hs[layer_i + 1], moe, wsp)
        replay = g.capture_end()
        g.discard()
        for i in range(3):
            hs[2].zero_()
            moe.zero_()
            side.synchronize()
            replay.launch(side)
            side.synchronize()
            assert torch.equal(hs[2], eager) and torch.equal(moe, eager_moe), i
            _ = (torch.randn(4096, device="cuda:0") * 2).sum().item()
        del replay


def test_qwen_block_rejects_bad_arguments(ctx):
    rng = np.random.default_rng(10)
    mats, norms, layer = weights(rng)
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, 16, abi.F16)
    granite = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 16, abi.F16)
    wsp = torch.empty(rt.qwen_block_workspace_bytes(arena, 16), dtype=torch.uint8, device="cuda:0")
    h = torch.zeros(HID, dtype=torch.int16, device="cuda:0")
    out, moe = torch.empty_like(h), torch.empty_like(h)
    d = [to_device(m) for m in mats]
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="Qwen cache"):
            rt.qwen_attention_block(g, granite, 0, 0, layer, h, out, moe, wsp)
        bad = rt.QwenQ4Layer(dev(norms[0]), d[0], d[0], d[2], dev(norms[1]), dev(norms[2]), d[3], dev(norms[3]))
        with pytest.raises(abi.QxhError, match="k_proj"):
            rt.qwen_attention_block(g, arena, 0, 0, bad, h, out, moe, wsp)
        with pytest.raises(abi.QxhError, match="overlap"):
            rt.qwen_attention_block(g, arena, 0, 0, layer, h, h, moe, wsp)
        with pytest.raises(abi.QxhError, match="does not follow cache length"):
            rt.qwen_attention_block(g, arena, 0, 2, layer, h, out, moe, wsp)
        with pytest.raises(abi.QxhError, match="workspace"):
            rt.qwen_attention_block(g, arena, 0, 0, layer, h, out, moe, wsp[:1024])
    assert arena.len(0) == 0
