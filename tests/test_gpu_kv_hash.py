"""GPU parity: KV commitment leaves and per-token verification digests.

The HIP kernels hash token rows straight out of the head-major arena; the
oracle (oracle/qx_oracle_hash.c, pinned by the reference's protocol golden
vectors) hashes the same rows gathered into the reference's position-major
[kv_head][head_dim] bytes.  Digests must be bit-identical.
"""
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


def row_bytes(t):
    return t.contiguous().cpu().view(torch.uint8).numpy().tobytes()


CASES = [
    (abi.SHAPE_GRANITE, abi.F32),   # 2048-byte rows: 8 chunks, one per head
    (abi.SHAPE_GRANITE, abi.F16),   # 1024-byte rows: a chunk spans two heads
    (abi.SHAPE_QWEN3, abi.BF16),    # 1024-byte rows: one head per chunk
    (abi.SHAPE_QWEN3, abi.F32),     # 2048-byte rows: half a head per chunk
]


@pytest.mark.parametrize("shape,dtype", CASES)
def test_kv_leaf_hashes_match_oracle(ctx, shape, dtype):
    log("kv leaf hashes", shape, dtype)
    cap, seqs, layers = 96, 3, 2
    arena = rt.KvArena(ctx, shape, layers, seqs, cap, dtype)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=5 + dtype, length=cap)
    # ragged count (not a multiple of the leaves per wave), nonzero begin, last row
    layer, begin, count = 1, 37, 59
    with rt.Graph(ctx) as g:
        got = arena.leaf_hashes(g, layer, begin, count, first_sequence=1, sequences=2)
        rows = [arena.gather(g, layer, s, begin, count) for s in (1, 2)]
    got = got.cpu().numpy()
    for si, (kk, vv) in enumerate(rows):
        for i in range(count):
            ref = O.kv_leaf_hash_v1(layer, begin + i, row_bytes(kk[i]), row_bytes(vv[i]))
            assert got[si, i].tobytes() == ref, (si, i)


def test_kv_leaf_hashes_of_token_zero_and_the_last_slot(ctx):
    cap = 40
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F16)
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=9, length=cap)
        first = arena.leaf_hashes(g, 0, 0, 1)
        last = arena.leaf_hashes(g, 0, cap - 1, 1)
        k0, v0 = arena.gather(g, 0, 0, 0, 1)
        kl, vl = arena.gather(g, 0, 0, cap - 1, 1)
    assert first.cpu().numpy()[0, 0].tobytes() == O.kv_leaf_hash_v1(0, 0, row_bytes(k0[0]), row_bytes(v0[0]))
    assert last.cpu().numpy()[0, 0].tobytes() == O.kv_leaf_hash_v1(0, cap - 1, row_bytes(kl[0]), row_bytes(vl[0]))


def test_kv_leaf_hash_bounds_are_enforced(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 16, abi.F32)
    arena.set_len(10)
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="committed length"):
            arena.leaf_hashes(g, 0, 5, 6)
        with pytest.raises(abi.QxhError, match="zero rows"):
            arena.leaf_hashes(g, 0, 0, 0)
        short = torch.empty((1, 2, 31), dtype=torch.uint8, device="cuda:0")
        with pytest.raises(abi.QxhError, match="smaller"):
            arena.leaf_hashes(g, 0, 0, 2, out=short)


@pytest.mark.parametrize("shape,dtype,stride", [(abi.SHAPE_GRANITE, abi.F32, 4096), (abi.SHAPE_QWEN3, abi.BF16, 8192)])
def test_verification_hashes_match_oracle(ctx, shape, dtype, stride):
    """encode_verification_hashes (crates/qx-metal/src/lib.rs:9247-9345): genesis,
    checkpoint and plain layers, over the row at `token` of every layer."""
    log("verification hashes", shape, dtype)
    layers, cap, token, interval = 5, 64, 41, 2
    arena = rt.KvArena(ctx, shape, layers, 2, cap, dtype)
    res = torch.randint(0, 256, ((layers + 1) * stride,), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=77, length=cap)
        got = arena.verification_hashes(g, res, stride, token, layers, interval, sequence=1)
        rows = [arena.gather(g, l, 1, token, 1) for l in range(layers)]
    ref = O.verification_hashes(res.cpu().numpy().tobytes(), stride, [row_bytes(k[0]) for k, _ in rows],
                                [row_bytes(v[0]) for _, v in rows], token, layers, interval)
    assert got.cpu().numpy().tobytes() == ref


def test_verification_hash_arguments_are_validated(ctx):
    layers, cap = 3, 16
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, layers, 1, cap, abi.F32)
    arena.set_len(8)
    res = torch.zeros(((layers + 1) * 4096,), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="committed length"):
            arena.verification_hashes(g, res, 4096, 8, layers, 1)
        with pytest.raises(abi.QxhError, match="checkpoint interval"):
            arena.verification_hashes(g, res, 4096, 2, layers, 0)
        with pytest.raises(abi.QxhError, match="layer count"):
            arena.verification_hashes(g, res, 4096, 2, layers + 1, 1)
        with pytest.raises(abi.QxhError, match="power-of-two"):
            arena.verification_hashes(g, res[:(layers + 1) * 768], 768, 2, layers, 1)
        with pytest.raises(abi.QxhError, match="too small"):
            arena.verification_hashes(g, res[:100], 4096, 2, layers, 1)
