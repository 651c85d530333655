"""GPU parity: group-32 Q4 projections (mat_vec_simd32 order,
crates/qx-quant/src/lib.rs:892-938), the 256-thread inverse RMS
(crates/qx-runtime/src/lib.rs:2416-2432) and the Granite attention block with
Q4 projections, against the oracle.  Norm, projections, RoPE, cache rows and
the residual inverse RMS are compared bit for bit; the attention and hence
hidden_out to the fp32 tolerance."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_16, TOL_F32, log, rel_err

pytestmark = pytest.mark.gpu

HID = 1024


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_device(m: O.Q4Matrix) -> rt.Q4Matrix:
    return rt.Q4Matrix(dev(m.packed), dev(m.scales.view(np.int16)), m.rows, m.cols)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bits(got, ref, what):
    g, r = bits(got), bits(ref)
    bad = np.flatnonzero(g != r)
    assert bad.size == 0, f"{what}: {bad.size} words differ, first at {bad[:4]}: {g[bad[:4]]} vs {r[bad[:4]]}"


@pytest.mark.parametrize("rows,cols", [(1, 32), (8, 32), (37, 64), (512, 1024), (1024, 1024), (100, 2048),
                                       (9, 1056), (3, 4096)])
def test_q4_gemv_is_bit_exact(ctx, rows, cols):
    log(f"q4 gemv {rows}x{cols}")
    rng = np.random.default_rng(rows * 7919 + cols)
    m = O.q4_quantize((0.02 * rng.standard_normal((rows, cols))).astype(np.float32))
    # a wide dynamic range makes every reordering of the sums visible
    x = (rng.standard_normal(cols) * np.exp2(rng.integers(-12, 12, cols))).astype(np.float32)
    dm = to_device(m)
    for mult in (1.0, 0.5, 1.7):
        with rt.Graph(ctx) as g:
            out = rt.q4_gemv(g, dm, dev(x), multiplier=mult)
        assert_bits(out.cpu().numpy(), O.q4_mat_vec_simd32(m, x, mult), f"{rows}x{cols} x{mult}")


def test_q4_gemv_tree_and_fold_order(ctx):
    """Inputs where every other summation order gives other float32 bits
    (the oracle pins these sums to 2^24 + 2 and 2^24)."""
    big = np.float32(2.0 ** 24)
    codes = np.full((2, 96), 7, np.uint8)
    codes[0, [0, 8, 24]] = 8    # row 0: lanes 0, 8, 24 in group 0 -> tree order
    codes[1, [0, 32, 64]] = 8   # row 1: lane 0 over groups 0, 1, 2 -> fold order
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    m = O.Q4Matrix(packed, np.full((2, 3), 0x3C00, np.uint16), 2, 96)
    x = np.zeros(96, np.float32)
    x[[0, 8, 24, 32, 64]] = [big, 1, 1, 1, 1]
    with rt.Graph(ctx) as g:
        out = rt.q4_gemv(g, to_device(m), dev(x)).cpu().numpy()
    ref = O.q4_mat_vec_simd32(m, x)
    assert_bits(out, ref, "order")
    assert ref[0] == np.float32(16777218.0) and ref[1] == big


def test_rms_inverse_is_bit_exact(ctx):
    rng = np.random.default_rng(5)
    vecs = [rng.standard_normal(HID).astype(np.float32) * s for s in (1e-3, 1.0, 37.0, 1e3)]
    for small in ([8, 24], [256, 512], [64, 192]):
        x = np.zeros(HID, np.float32)
        x[0] = 4096.0
        x[small] = 1.0
        vecs.append(x)
    vecs.append(np.full(HID, 3.0, np.float32))
    for i, x in enumerate(vecs):
        with rt.Graph(ctx) as g:
            got = rt.rms_inverse(g, dev(x)).cpu().numpy()
        assert_bits(got, [O.granite_rms_norm_simd(x)[2]], f"vector {i}")


def workspace_query_and_attention(wsp):
    """The block keeps the rotated query and the attention output, fp32
    [1024] each, at the start of its workspace."""
    w = wsp[:2 * HID * 4].view(torch.float32).cpu().numpy()
    return w[:HID], w[HID:]


def q4_weights(rng):
    nw = (1.0 + 0.05 * rng.standard_normal(HID)).astype(np.float32)
    mats = [O.q4_quantize((0.02 * rng.standard_normal(shape)).astype(np.float32))
            for shape in ((HID, HID), (512, HID), (512, HID), (HID, HID))]
    return nw, mats


def device_layer(nw, mats):
    return rt.GraniteQ4Layer(dev(nw), *[to_device(m) for m in mats])


@pytest.mark.parametrize("kv_dtype", [abi.F32, abi.F16])
def test_q4_block_sequence(ctx, kv_dtype):
    """2 layers x 24 positions.  Each layer's oracle input is the GPU's own
    hidden_in, so everything before attention must match bit for bit."""
    log(f"q4 block sequence dtype={kv_dtype}")
    rng = np.random.default_rng(41 + kv_dtype)
    LAYERS, P = 2, 24
    ws = [q4_weights(rng) for _ in range(LAYERS)]
    layers = [device_layer(nw, mats) for nw, mats in ws]
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, 1, 64, kv_dtype)
    fmt = O.F32 if kv_dtype == abi.F32 else O.F16
    tol = TOL_F32 if kv_dtype == abi.F32 else TOL_16  # fp16 K/V: P.V runs on fp16 MFMA
    refs = [O.KvCache(64, fmt, fmt) for _ in range(LAYERS)]
    wsp = torch.zeros(rt.granite_block_workspace_bytes(arena, 64), dtype=torch.uint8, device="cuda:0")
    inv = torch.empty(1, device="cuda:0")
    worst = 0.0
    for p in range(P):
        cur = dev(rng.standard_normal(HID, dtype=np.float32))
        for layer in range(LAYERS):
            nxt = torch.empty(HID, device="cuda:0")
            with rt.Graph(ctx) as g:
                rt.granite_attention_block_q4(g, arena, layer, p, layers[layer], cur, nxt, wsp, inv)
            h = cur.cpu().numpy()
            ref, qrot, att_ref, _ = O.granite_q4_attention_block(h, ws[layer][0], *ws[layer][1], p, refs[layer])
            got = nxt.cpu().numpy()
            q_gpu, att_gpu = workspace_query_and_attention(wsp)
            assert_bits(q_gpu, qrot, f"query p={p} l={layer}")
            e_att = rel_err(att_gpu, att_ref)
            assert e_att <= tol, ("attention", p, layer, e_att)
            # o projection + residual of the GPU's own attention: bit for bit
            assert_bits(got, O.granite_residual(h, O.q4_mat_vec_simd32(ws[layer][1][3], att_gpu)),
                        f"o projection + residual p={p} l={layer}")
            assert_bits(inv.cpu().numpy(), [O.granite_rms_norm_simd(got)[2]], f"inverse rms p={p} l={layer}")
            e = rel_err(got, ref)
            worst = max(worst, e_att)
            assert e <= tol, (p, layer, e)
            cur = nxt
    log(f"q4 block worst attention max-abs/rms {worst:.3e}")
    for layer in range(LAYERS):
        assert arena.len(layer) == P
        with rt.Graph(ctx) as g:
            kk, vv = arena.gather(g, layer, 0, 0, P)
        assert_bits(kk.float().cpu().numpy(), refs[layer].keys(), f"keys layer {layer}")
        assert_bits(vv.float().cpu().numpy(), refs[layer].values(), f"values layer {layer}")


def test_q4_block_over_a_long_prefilled_cache(ctx):
    """Position 700 over 700 N(0,1) rows: attention past the 512 positions of
    the reference's hierarchical form (the oracle switches to the sequential
    one there)."""
    log("q4 block @700")
    rng = np.random.default_rng(43)
    nw, mats = q4_weights(rng)
    layer = device_layer(nw, mats)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 1024, abi.F32)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=9, length=700)
        kk, vv = arena.gather(g, 0, 0, 0, 700)
    ref_cache = O.KvCache(1024)
    ref_cache.extend(kk.cpu().numpy(), vv.cpu().numpy())
    h = rng.standard_normal(HID).astype(np.float32)
    out = torch.empty(HID, device="cuda:0")
    wsp = torch.empty(rt.granite_block_workspace_bytes(arena, 701), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        rt.granite_attention_block_q4(g, arena, 0, 700, layer, dev(h), out, wsp)
    ref, _, att_ref, _ = O.granite_q4_attention_block(h, nw, *mats, 700, ref_cache)
    got = out.cpu().numpy()
    _, att_gpu = workspace_query_and_attention(wsp)
    e_att = rel_err(att_gpu, att_ref)
    log(f"q4 block@700 attention max-abs/rms {e_att:.3e}")
    assert e_att <= TOL_F32
    assert_bits(got, O.granite_residual(h, O.q4_mat_vec_simd32(mats[3], att_gpu)), "o projection + residual")
    assert rel_err(got, ref) <= TOL_F32
    with rt.Graph(ctx) as g:
        kk, vv = arena.gather(g, 0, 0, 700, 1)
    assert_bits(kk.cpu().numpy(), ref_cache.keys()[700:], "key row 700")
    assert_bits(vv.cpu().numpy(), ref_cache.values()[700:], "value row 700")


def test_q4_captured_block_replays_match_eager(ctx):
    """HIP-graph replay of 3 Q4 layers, replayed 4 times with eager work
    between replays; every replay equals the eager result bit for bit."""
    rng = np.random.default_rng(44)
    LAYERS, POS = 3, 100
    layers = [device_layer(*q4_weights(rng)) for _ in range(LAYERS)]
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, 1, 128, abi.F32)
    hid = [torch.empty(HID, device="cuda:0") for _ in range(LAYERS + 1)]
    hid[0].copy_(dev(rng.standard_normal(HID, dtype=np.float32)))
    inv = torch.empty(1, device="cuda:0")
    wsp = torch.empty(rt.granite_block_workspace_bytes(arena, POS + 1), dtype=torch.uint8, device="cuda:0")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with rt.Graph(ctx, side) as g:
            arena.fill_normal(g, seed=8, length=POS)
            for layer in range(LAYERS):
                rt.granite_attention_block_q4(g, arena, layer, POS, layers[layer], hid[layer], hid[layer + 1], wsp,
                                              inv)
        eager, eager_inv = hid[-1].clone(), inv.clone()
        arena.rollback(0, POS)
        g = rt.Graph(ctx, side)
        g.capture_begin()
        for layer in range(LAYERS):
            rt.granite_attention_block_q4(g, arena, layer, POS, layers[layer], hid[layer], hid[layer + 1], wsp, inv)
        replay = g.capture_end()
        g.discard()
        for i in range(4):
            hid[-1].zero_()
            inv.zero_()
            side.synchronize()
            replay.launch(side)
            side.synchronize()
            assert torch.equal(hid[-1], eager) and torch.equal(inv, eager_inv), i
            scratch = torch.randn(4096, device="cuda:0")  # unrelated eager work between replays
            _ = (scratch * 2).sum().item()
        del replay


def test_q4_entry_points_reject_bad_arguments(ctx):
    rng = np.random.default_rng(45)
    nw, mats = q4_weights(rng)
    good = [to_device(m) for m in mats]
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 16, abi.F32)
    wsp = torch.empty(rt.granite_block_workspace_bytes(arena, 16), dtype=torch.uint8, device="cuda:0")
    h, out = dev(np.zeros(HID, np.float32)), torch.empty(HID, device="cuda:0")
    with rt.Graph(ctx) as g:
        # k projection with the q shape
        bad = rt.GraniteQ4Layer(dev(nw), good[0], good[0], good[2], good[3])
        with pytest.raises(abi.QxhError, match="k_proj"):
            rt.granite_attention_block_q4(g, arena, 0, 0, bad, h, out, wsp)
        # misaligned codes: an 8-byte offset inside a buffer 16 bytes longer
        # than the matrix, so the view stays in bounds
        p = good[1].tensors[0]
        flat = torch.zeros(p.numel() + 16, dtype=torch.uint8, device="cuda:0")
        shifted = rt.Q4Matrix(flat[8:8 + p.numel()], good[1].tensors[1], 512, HID)
        bad = rt.GraniteQ4Layer(dev(nw), good[0], shifted, good[2], good[3])
        with pytest.raises(abi.QxhError, match="aligned"):
            rt.granite_attention_block_q4(g, arena, 0, 0, bad, h, out, wsp)
        ok = rt.GraniteQ4Layer(dev(nw), *good)
        with pytest.raises(abi.QxhError, match="distinct"):
            rt.granite_attention_block_q4(g, arena, 0, 0, ok, h, h, wsp)
        with pytest.raises(abi.QxhError, match="does not follow cache length"):
            rt.granite_attention_block_q4(g, arena, 0, 3, ok, h, out, wsp)
        # general GEMV: columns not a multiple of 32, empty, overlap
        odd = rt.Q4Matrix(p, good[1].tensors[1], 4, 48)
        with pytest.raises(abi.QxhError, match="multiple of 32"):
            rt.q4_gemv(g, odd, h)
        with pytest.raises(abi.QxhError, match="empty"):
            rt.q4_gemv(g, rt.Q4Matrix(p, good[1].tensors[1], 0, 1024), h, out=out)
        buf = torch.empty(2048, device="cuda:0")
        with pytest.raises(abi.QxhError, match="overlap"):
            rt.q4_gemv(g, good[1], buf[:1024], out=buf[512:1024])
    assert arena.len(0) == 0
