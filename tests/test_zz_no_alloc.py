"""qxh_encode_attention_for_layer_no_alloc against qxh_encode_attention_for_layer.

The no-alloc entry point keeps the split-K partials in the library's per-GPU
device scratch instead of a caller workspace; it runs the same plan and
kernels, so its outputs must equal the workspace entry's bit for bit.  Two
calls in a row, the second with a smaller input, so the second reads a
scratch that still holds the first call's partials; then a request whose
partials exceed the scratch is refused before anything is enqueued.
"""
import pytest
import torch

from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import log

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def run_both(ctx, arena, q, length):
    need = rt.attention_workspace_bytes(arena, q.shape[0], length)
    assert 0 < need <= SCRATCH_BYTES  # the case uses the scratch
    ref = torch.empty_like(q)
    got = torch.full_like(q, float("nan"))
    with rt.Graph(ctx) as g:
        rt.attention(g, arena, 0, q, length, out=ref)
    with rt.Graph(ctx) as g:
        rt.attention_no_alloc(g, arena, 0, q, length, out=got)
    return ref, got, need


def test_no_alloc_matches_workspace_entry_on_two_calls(ctx):
    # call 1: Qwen bf16, one sequence at 32768 positions (64 splits x 4 kv heads)
    log("no-alloc call 1: qwen bf16 1 x 32768")
    big = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, 32768, abi.BF16)
    qb = torch.empty((1, 32, 128), dtype=torch.bfloat16, device="cuda:0")
    with rt.Graph(ctx) as g:
        big.fill_normal(g, seed=31, length=32768)
        rt.fill_normal(g, qb, seed=32)
    ref, got, need1 = run_both(ctx, big, qb, 32768)
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)
    # call 2, smaller: Granite fp32, two sequences at 1000 positions
    log("no-alloc call 2: granite fp32 2 x 1000")
    small = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 2, 1000, abi.F32)
    qs = torch.empty((2, 16, 64), device="cuda:0")
    with rt.Graph(ctx) as g:
        small.fill_normal(g, seed=33, length=1000)
        rt.fill_normal(g, qs, seed=34)
    ref2, got2, need2 = run_both(ctx, small, qs, 1000)
    assert need2 < need1
    assert torch.equal(got2, ref2)
    # and the first shape again, shorter, after the Granite partials
    log("no-alloc call 3: qwen bf16 1 x 5000")
    ref3, got3, _ = run_both(ctx, big, qb, 5000)
    assert torch.equal(got3, ref3)


def test_no_alloc_refuses_partials_beyond_the_scratch(ctx):
    # 511 Qwen sequences at 1024 positions on fp32 caches (the VALU kernel,
    # which splits toward 2048 workgroups): 2044 units x 2 splits (of 512
    # positions) x 8 heads x 130 floats = 17.0 MB of partials, above the
    # 16 MiB scratch
    log("no-alloc: oversize request")
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 511, 1024, abi.F32)
    arena.set_len(1024)
    assert rt.attention_workspace_bytes(arena, 511, 1024) > SCRATCH_BYTES
    q = torch.zeros((511, 32, 128), device="cuda:0")
    out = torch.empty_like(q)
    g = rt.Graph(ctx)
    with pytest.raises(abi.QxhError, match="device scratch") as ei:
        rt.attention_no_alloc(g, arena, 0, q, 1024, out=out)
    assert ei.value.code == abi.QXH_ERR_INVALID_ARGUMENT
    assert g.finish().dispatches == 0  # refused before anything was enqueued
