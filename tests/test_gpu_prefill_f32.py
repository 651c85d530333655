"""GPU parity: causal prefill on fp32 and mixed K/V caches (Granite shape),
the fp32 matrix-core kernel of prefill_f32.hip.

The reference runs a prompt as repeated decode (crates/qx-runtime/src/lib.rs:
1341-1353), so row t is granite_attention_decode's attention at position
start + t over [0, start + t]; the oracle's granite_prefill_rows restates it.
Its KV plans include fp32 keys with f16 values (KvPrecision::Fp32KFp16V, the
default of new artifacts, crates/qx-format/src/lib.rs:554-558) and the
reverse.  The fp32 bar: within 1e-5 x output RMS of the oracle for rows of
at most 1024 positions, within 5e-6 of float64 attention for every row (the
reference's own sequential folds drift past 1e-5 of exact beyond that
length).  Sampled rows (first, last, seeded random) at full size; the cache
rows are the ones the GPU holds, gathered back.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import attend64, check_fp32_bar, log
from tests.test_gpu_prefill import rows_to_check

pytestmark = pytest.mark.gpu

FMT = {abi.F32: O.F32, abi.F16: O.F16, abi.BF16: O.BF16}
TORCH = {abi.F32: torch.float32, abi.F16: torch.float16, abi.BF16: torch.bfloat16}


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def run_prefill(ctx, kdt, vdt, start, T, seed, qdt=abi.F32, odt=abi.F32):
    rng = np.random.default_rng(seed)
    cap = start + T
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, kdt, vdt)
    q = torch.from_numpy(rng.standard_normal((T, 16, 64), dtype=np.float32)).cuda().to(TORCH[qdt])
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=seed, length=cap)
        out = rt.prefill_attention(g, arena, 0, start, q, out_dtype=TORCH[odt])
        kk, vv = arena.gather(g, 0, 0, 0, cap)
    kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
    ref = O.KvCache(cap, FMT[kdt], FMT[vdt])
    ref.extend(kf, vf)
    return rng, q.float().cpu().numpy(), out.float().cpu().numpy(), ref, kf, vf


def check_rows(q, out, ref, kf, vf, start, rows):
    r = O.granite_prefill_rows(q.reshape(q.shape[0], -1), ref, start, rows)
    worst = (0.0, 0.0)
    for i, t in enumerate(rows):
        L = start + int(t) + 1
        exact = attend64(q[t], kf[:L], vf[:L], 0.015625).ravel()
        e, e64, _ = check_fp32_bar(out[t].ravel(), r[i], exact, L)
        worst = (max(worst[0], e), max(worst[1], e64))
    return worst


# (0, 2048): cfg 3's prompt, two KV chunks merged by the combine kernel;
# (0, 300) and (37, 129): one chunk, ragged last block; (1000, 100): a prompt
# after 1000 cached positions (chunks of the cached range)
@pytest.mark.parametrize("kdt,vdt", [(abi.F32, abi.F16), (abi.F32, abi.F32), (abi.F16, abi.F32),
                                     (abi.F32, abi.BF16), (abi.BF16, abi.F32)])
@pytest.mark.parametrize("start,T", [(0, 2048), (0, 300), (37, 129), (1000, 100)])
def test_f32_prefill_matches_oracle(ctx, kdt, vdt, start, T):
    log("f32 prefill", kdt, vdt, start, T)
    rng, q, out, ref, kf, vf = run_prefill(ctx, kdt, vdt, start, T, seed=T + start + 7 * kdt + vdt)
    rows = rows_to_check(T, rng, first=8, last=8, rand=16)
    e, e64 = check_rows(q, out, ref, kf, vf, start, rows)
    log(f"f32 prefill {kdt}/{vdt} start {start} T {T}: vs oracle {e:.2e}, vs float64 {e64:.2e} ({rows.size} rows)")


def test_f32_prefill_query_and_output_dtypes(ctx):
    """16-bit queries in and 16-bit outputs out: the kernel widens the query
    and rounds each output once (round to nearest even)."""
    rng, q, out, ref, kf, vf = run_prefill(ctx, abi.F32, abi.F16, 0, 200, seed=5, qdt=abi.F16, odt=abi.BF16)
    rows = rows_to_check(200, rng, first=4, last=4, rand=8)
    r = O.granite_prefill_rows(q.reshape(200, -1), ref, 0, rows)
    for i, t in enumerate(rows):
        want = torch.from_numpy(r[i]).to(torch.bfloat16).float().numpy()
        # one bf16 rounding of a result within the fp32 bar of the oracle
        assert np.max(np.abs(out[t].ravel() - want)) <= 2.0 ** -8 * np.max(np.abs(want)) + 1e-6, t


def test_f32_prefill_equals_decode_rows_of_the_same_cache(ctx):
    """Row by row against the causal decode rows this cache took before (a
    call of 8 rows still runs there): the same positions, fp32 both ways."""
    start, T = 500, 72
    rng = np.random.default_rng(11)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, start + T, abi.F32, abi.F16)
    q = torch.from_numpy(rng.standard_normal((T, 16, 64), dtype=np.float32)).cuda()
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=3, length=start + T)
        whole = rt.prefill_attention(g, arena, 0, start, q)
        parts = [rt.prefill_attention(g, arena, 0, start + t0, q[t0:t0 + 8]) for t0 in range(0, T, 8)]
    parts = torch.cat(parts).cpu().numpy()
    whole = whole.cpu().numpy()
    rms = np.sqrt(np.mean(parts.astype(np.float64) ** 2))
    assert np.max(np.abs(whole - parts)) / rms <= 1e-5


@pytest.mark.parametrize("start,T,W", [(0, 300, 64), (500, 100, 256), (37, 129, 32)])
def test_f32_prefill_on_tiered_values(ctx, start, T, W):
    """fp32 keys with tiered values (recent rows f16, older rows block INT8:
    the reference's proposed plan, docs/qx-structural-memory-2026-08-25.md:
    69-74) on the fp32 kernel: each V tile row widened from its tier (INT8
    code x block scale, exact in fp32, or the f16 window slot), against the
    oracle over the values the cache holds (the dequantised gather)."""
    cap = start + T
    rng = np.random.default_rng(cap + W)
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F32, abi.I8_TIERED, value_window=W)
    q = torch.from_numpy(rng.standard_normal((T, 16, 64), dtype=np.float32)).cuda()
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=W, length=cap)
        out = rt.prefill_attention(g, arena, 0, start, q)
        kk, vv = arena.gather(g, 0, 0, 0, cap)
    assert arena.value_tier() == max(0, cap - W)
    kf, vf = kk.float().cpu().numpy(), vv.float().cpu().numpy()
    ref = O.KvCache(cap)
    ref.extend(kf, vf)
    rows = rows_to_check(T, rng, first=8, last=8, rand=16)
    e, e64 = check_rows(q.cpu().numpy(), out.cpu().numpy(), ref, kf, vf, start, rows)
    log(f"f32 prefill tiered W={W} start {start} T {T}: vs oracle {e:.2e}, vs float64 {e64:.2e}")
