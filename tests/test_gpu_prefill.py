"""GPU parity: causal MFMA prefill against the oracle's repeated decode.

The reference runs prompts as repeated decode (crates/qx-runtime/src/lib.rs:1341-1353),
so prompt row t is decode attention at position start + t over [0, start + t].
Granite (config 3): fp16 q/k/v, RoPE'd by the fused kernel; the oracle runs
the fp32 path on the upcast inputs.  Qwen (config 5b): bf16, per-head
RMSNorm + RoPE; the oracle attends with the GPU's own rotated q/k bits so the
attention arithmetic is compared in isolation (the front end is checked in
test_gpu_rope_kv.py).  Tolerance: 2e-3 x the RMS of each output row (a
prompt row is the decode output at its position; the decode tests hold each
output to its own RMS) on fp32 outputs; sampled rows (first, last and seeded
random) at full size: at the configs' prompt lengths the first 64, the last
64 and 128 random rows.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_16, log, rel_err, row_rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def rows_to_check(T, rng, first=32, last=32, rand=32):
    r = set(range(min(first, T))) | set(range(max(0, T - last), T))
    if T > first + last:
        r |= set(int(x) for x in rng.choice(T, size=min(rand, T), replace=False))
    return np.array(sorted(r), np.uint32)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


# (2048, 0): 256 blocks, three KV groups per workgroup; (3000, 500): 376
# blocks, two rounds of workgroups with three KV groups each; (40, 3000):
# the pipelined kernel with the KV range split into 6 chunks; (6, 3000) and
# (20, 3000): causal rows on the MFMA decode kernel, split over the context
@pytest.mark.parametrize("T,start", [(2048, 0), (3000, 500), (100, 0), (77, 30), (1, 5), (33, 0), (200, 900), (40, 3000),
                                     (6, 3000), (20, 3000)])
def test_granite_prefill_fp16(ctx, T, start):
    log("granite prefill", T, start)
    rng = np.random.default_rng(T * 31 + start)
    cap = start + T
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, cap, abi.F16)
    pre_q = rng.standard_normal((start, 16, 64), dtype=np.float32).astype(np.float16)
    pre_k = rng.standard_normal((start, 8, 64), dtype=np.float32).astype(np.float16)
    pre_v = rng.standard_normal((start, 8, 64), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((T, 16, 64), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((T, 8, 64), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((T, 8, 64), dtype=np.float32).astype(np.float16)
    cuda = lambda a: torch.from_numpy(a).cuda()
    with rt.Graph(ctx) as g:
        if start:
            rt.rope_kv_batch(g, arena, 0, 0, cuda(pre_q)[None], cuda(pre_k)[None], cuda(pre_v)[None])
        qo = torch.empty((1, T, 16, 64), dtype=torch.float16, device="cuda:0")
        rt.rope_kv_batch(g, arena, 0, start, cuda(q)[None], cuda(k)[None], cuda(v)[None], query_out=qo)
        out = rt.prefill_attention(g, arena, 0, start, qo[0], out_dtype=torch.float32)
    # oracle: the fp32 path on upcast inputs (apply_granite_rope + KvCache + attend)
    ref = O.KvCache(cap)
    allk = np.concatenate([pre_k, k]).astype(np.float32)
    allv = np.concatenate([pre_v, v]).astype(np.float32)
    allq = np.concatenate([pre_q, q]).astype(np.float32)
    qrot = np.zeros((cap, 1024), np.float32)
    for p in range(cap):
        qr, kr = O.apply_granite_rope(allq[p].ravel(), allk[p].ravel(), p)
        qrot[p] = qr
        ref.append(p, kr, allv[p].ravel())
    rows = rows_to_check(T, rng, 64, 64, 128) if T == 2048 else rows_to_check(T, rng)
    r = O.granite_prefill_rows(qrot[start:], ref, start, rows)
    got = out.cpu().numpy().reshape(T, 1024)[rows]
    e = row_rel_err(got, r)
    log(f"granite prefill T={T} start={start}: max-abs/rms {e:.3e} over {rows.size} rows")
    assert e <= TOL_16


# (40, 8150), (300, 8000) and (512, 2048): the pipelined kernel with each
# block's KV range split into chunks of at least 16 tiles (8, 7 and 2
# chunks); (9, 8150) and (4, 32764): causal rows on the MFMA decode kernel
# (64 splits per row at 32768 positions)
@pytest.mark.parametrize("T,start", [(8192, 0), (300, 0), (129, 64), (40, 8150), (300, 8000), (512, 2048), (9, 8150),
                                     (4, 32764)])
def test_qwen_prefill_bf16(ctx, T, start):
    log("qwen prefill", T, start)
    rng = np.random.default_rng(T + 7 * start)
    cap = start + T
    dt = torch.bfloat16
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, cap, abi.BF16)
    qin = torch.empty((1, cap, 32, 128), dtype=dt, device="cuda:0")
    kin = torch.empty((1, cap, 4, 128), dtype=dt, device="cuda:0")
    vin = torch.empty((1, cap, 4, 128), dtype=dt, device="cuda:0")
    qo = torch.empty_like(qin)
    with rt.Graph(ctx) as g:
        for i, t in enumerate((qin, kin, vin)):
            rt.fill_normal(g, t, seed=100 * T + i)
        if start:
            rt.rope_kv_batch(g, arena, 0, 0, qin[:, :start].contiguous(), kin[:, :start].contiguous(),
                             vin[:, :start].contiguous())
        qtail = qo[:, start:].contiguous()
        rt.rope_kv_batch(g, arena, 0, start, qin[:, start:].contiguous(), kin[:, start:].contiguous(),
                         vin[:, start:].contiguous(), query_out=qtail)
        out = rt.prefill_attention(g, arena, 0, start, qtail[0], out_dtype=torch.float32)
        out16 = rt.prefill_attention(g, arena, 0, start, qtail[0])
        kk, vv = arena.gather(g, 0, 0, 0, cap)
    # cfg 5b's prompt: the first 64, the last 64 and 128 seeded random rows
    # (the oracle's rows on 16 threads); other cases 24 of each
    rows = rows_to_check(T, rng, 64, 64, 128) if T == 8192 else rows_to_check(T, rng, 24, 24, 24)
    rb, rf = O.qwen_prefill_rows(bits(qtail[0]), bits(kk), bits(vv), start, rows, O.BF16, workers=16)
    got = out.cpu().numpy().reshape(T, 4096)[rows]
    e = row_rel_err(got, rf)
    log(f"qwen prefill T={T} start={start}: max-abs/rms {e:.3e} over {rows.size} rows")
    assert e <= TOL_16
    # the bf16 output is the RNE rounding of the fp32 result
    assert np.array_equal(bits(out16).reshape(T, 4096), O.to_bits16(out.cpu().numpy(), O.BF16).reshape(T, 4096))


@pytest.mark.parametrize("shape,dtype", [(abi.SHAPE_GRANITE, abi.F16), (abi.SHAPE_QWEN3, abi.BF16)])
def test_prefill_last_row_equals_decode(ctx, shape, dtype):
    """Size-independent property: prefill row t == decode at length start+t+1."""
    info = rt.shape_info(shape)
    T = 1000
    tdt = rt.torch_dtype(dtype)
    arena = rt.KvArena(ctx, shape, 1, 1, T, dtype)
    q = torch.empty((T, info.q_heads, info.head_dim), dtype=tdt, device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=11, length=T)
        rt.fill_normal(g, q, seed=12)
        pre = rt.prefill_attention(g, arena, 0, 0, q, out_dtype=torch.float32)
        for t in (0, 511, T - 1):
            dec = rt.attention(g, arena, 0, q[t:t + 1].contiguous(), t + 1, out_dtype=torch.float32)
            assert rel_err(pre[t].cpu().numpy(), dec[0].cpu().numpy()) <= TOL_16, t


@pytest.mark.parametrize("shape,T", [(abi.SHAPE_GRANITE, 300), (abi.SHAPE_QWEN3, 300), (abi.SHAPE_QWEN3, 4096),
                                     (abi.SHAPE_QWEN3, 9000)])
def test_bf16_values_outside_f16_range_take_the_exact_pass(ctx, shape, T):
    """bf16 V tiles are multiplied in f16; a value beyond the f16 range must
    route its workgroup to the exact bf16 pass and still match the oracle.
    T = 300 splits each block's KV range into chunks, T = 4096 does not.
    The exact pass after the pipelined kernel runs at most 256 workgroups:
    at Qwen T = 9000 (1,128 blocks, every block of kv heads 0 and 3
    flagged) each walks four or five blocks, reusing its LDS."""
    log("prefill overflow path", shape, T)
    info = rt.shape_info(shape)
    rng = np.random.default_rng(77)
    arena = rt.KvArena(ctx, shape, 1, 1, T, abi.BF16)
    q = torch.empty((T, info.q_heads, info.head_dim), dtype=torch.bfloat16, device="cuda:0")
    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=21, length=T)
        rt.fill_normal(g, q, seed=22)
    # plant a few huge values (finite in bf16, beyond f16) into V rows 5 and 250
    vptr = arena.layout.values
    nbytes = T * info.kv_heads * info.head_dim * 2
    off = vptr - arena.arena.data_ptr()
    vview = arena.arena[off:off + nbytes].view(torch.bfloat16).view(info.kv_heads, T, info.head_dim)
    vview[0, 5, 3] = 3.0e5
    vview[info.kv_heads - 1, 250, 7] = -1.0e9
    torch.cuda.synchronize()
    with rt.Graph(ctx) as g:
        out = rt.prefill_attention(g, arena, 0, 0, q, out_dtype=torch.float32)
        kk, vv = arena.gather(g, 0, 0, 0, T)
    rows = np.array([0, 4, 5, 6, 100, 249, 250, 251, 299] + ([2047, 4095] if T > 300 else []) +
                    ([6000, T - 1] if T > 4096 else []), np.uint32)
    if shape == abi.SHAPE_QWEN3:
        _, ref = O.qwen_prefill_rows(bits(q), bits(kk), bits(vv), 0, rows, O.BF16)
    else:
        c = O.KvCache(T)
        c.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
        ref = O.granite_prefill_rows(q.float().cpu().numpy().reshape(T, -1), c, 0, rows)
    got = out.cpu().numpy().reshape(T, -1)[rows]
    assert np.all(np.isfinite(got))
    e = row_rel_err(got, ref)
    log(f"overflow path max-abs/rms {e:.3e}")
    assert e <= TOL_16


def test_prefill_rejects_rows_beyond_cursor_and_a_query_dtype_the_mfma_path_lacks(ctx):
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, 128, abi.F16)
    arena.set_len(10)
    q = torch.zeros((11, 16, 64), dtype=torch.float16, device="cuda:0")
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError, match="beyond committed length"):
            rt.prefill_attention(g, arena, 0, 0, q)
    # prompts of at least one 64-position tile on 16-bit caches take the MFMA
    # prefill, whose query is the cache dtype (shorter ones run causal rows on
    # the decode kernels, which read any query dtype)
    arena.set_len(64)
    with rt.Graph(ctx) as g:
        with pytest.raises(abi.QxhError) as ei:
            rt.prefill_attention(g, arena, 0, 0, torch.zeros((64, 16, 64), device="cuda:0"))
        assert ei.value.code == abi.QXH_ERR_UNSUPPORTED


@pytest.mark.parametrize("shape,dtype", [(abi.SHAPE_GRANITE, abi.F16), (abi.SHAPE_QWEN3, abi.BF16)])
def test_k_wide_verifier_with_rollback(ctx, shape, dtype):
    """Speculative verification: K = 4 draft tokens are RoPE'd and appended at
    the cursor and attended causally in one call (encode_rope_kv_batch +
    encode_attention_batch_with_plan, crates/qx-metal/src/lib.rs:8105-8267).
    Two drafts are accepted: the cursor rolls back (rollback_kv,
    crates/qx-runtime-v2/src/lib.rs:3271-3285) and four new drafts overwrite
    the rejected slots.  Each verifier row must match the oracle over the cache
    as it stands, the accepted rows must keep their bits, and the overwritten
    slots must hold the new drafts."""
    log("k-wide verifier", shape)
    info = rt.shape_info(shape)
    tdt = rt.torch_dtype(dtype)
    L0, K, accepted = 300, 4, 2
    arena = rt.KvArena(ctx, shape, 1, 1, L0 + 8, dtype)

    def drafts(seed, start):
        q = torch.empty((1, K, info.q_heads, info.head_dim), dtype=tdt, device="cuda:0")
        k = torch.empty((1, K, info.kv_heads, info.head_dim), dtype=tdt, device="cuda:0")
        v = torch.empty_like(k)
        qo = torch.empty_like(q)
        with rt.Graph(ctx) as g:
            for i, t in enumerate((q, k, v)):
                rt.fill_normal(g, t, seed=seed + i)
            rt.rope_kv_batch(g, arena, 0, start, q, k, v, query_out=qo)
            out = rt.prefill_attention(g, arena, 0, start, qo[0], out_dtype=torch.float32)
            kk, vv = arena.gather(g, 0, 0, 0, start + K)
        return qo[0], out, kk, vv

    def check(qo, out, kk, vv, start):
        rows = np.arange(K, dtype=np.uint32)
        if shape == abi.SHAPE_QWEN3:
            _, ref = O.qwen_prefill_rows(bits(qo), bits(kk), bits(vv), start, rows, O.BF16)
        else:
            c = O.KvCache(start + K)
            c.extend(kk.float().cpu().numpy(), vv.float().cpu().numpy())
            ref = O.granite_prefill_rows(qo.float().cpu().numpy().reshape(K, -1), c, start, rows)
        e = row_rel_err(out.cpu().numpy().reshape(K, -1), ref)
        log(f"verifier start={start}: max-abs/rms {e:.3e}")
        assert e <= TOL_16

    with rt.Graph(ctx) as g:
        arena.fill_normal(g, seed=31, length=L0)
    qo1, out1, kk1, vv1 = drafts(40, L0)
    assert arena.len() == L0 + K
    check(qo1, out1, kk1, vv1, L0)

    arena.rollback(0, L0 + accepted)
    assert arena.len() == L0 + accepted
    qo2, out2, kk2, vv2 = drafts(50, L0 + accepted)
    assert arena.len() == L0 + accepted + K
    check(qo2, out2, kk2, vv2, L0 + accepted)
    # accepted rows keep their bits; the rejected slots now hold the new drafts
    n = L0 + accepted
    assert np.array_equal(bits(kk2[:n]), bits(kk1[:n])) and np.array_equal(bits(vv2[:n]), bits(vv1[:n]))
    assert not np.array_equal(bits(kk2[n:n + K - accepted]), bits(kk1[n:]))


TORCH = {abi.F32: torch.float32, abi.F16: torch.float16, abi.BF16: torch.bfloat16}


# Every prefill path, with the prompt ending inside a 64-position tile:
# Granite f16 (V tiles read straight from the cache: workgroups of two KV
# groups (300 rows; 100 rows after 1000, two groups where the grid would have
# split in two), three groups (2000 rows, 256 blocks) and the chunked grid
# with its merge (40 rows after 3000, six chunks)), Granite bf16 and Qwen
# bf16 (V^T pre-pass), Fp32KFp16V (fp32 matrix-core kernel; one chunk, then
# several) and a few rows (causal decode rows).
@pytest.mark.parametrize("shape,kdt,vdt,start,T", [
    (abi.SHAPE_GRANITE, abi.F16, abi.F16, 0, 300), (abi.SHAPE_GRANITE, abi.F16, abi.F16, 1000, 100),
    (abi.SHAPE_GRANITE, abi.F16, abi.F16, 0, 2000), (abi.SHAPE_GRANITE, abi.F16, abi.F16, 3000, 40),
    (abi.SHAPE_GRANITE, abi.BF16, abi.BF16, 0, 300), (abi.SHAPE_QWEN3, abi.BF16, abi.BF16, 0, 300),
    (abi.SHAPE_GRANITE, abi.F32, abi.F16, 0, 300), (abi.SHAPE_GRANITE, abi.F32, abi.F16, 1000, 100),
    (abi.SHAPE_GRANITE, abi.F16, abi.F16, 37, 6)])
def test_prefill_ignores_cache_rows_past_the_prompt(ctx, shape, kdt, vdt, start, T):
    """Rows at and past start + T are outside every prompt row's causal
    range, whatever they hold: with NaN there (appended after the prompt's
    rows, so the cache's length covers them) the output is finite and bit for
    bit the output over finite rows there.  The last tile's tail is neither
    read into a score nor multiplied by a zero probability."""
    kv_len, extra = start + T, 40
    log("prefill with NaN past the prompt", shape, kdt, vdt, start, T)
    heads, kvh, d = (16, 8, 64) if shape == abi.SHAPE_GRANITE else (32, 4, 128)
    rng = np.random.default_rng(kv_len + 7 * kdt)
    q = torch.from_numpy(rng.standard_normal((T, heads, d), dtype=np.float32)).cuda().to(TORCH[kdt])
    outs = []
    for nan_tail in (False, True):
        arena = rt.KvArena(ctx, shape, 1, 1, kv_len + extra, kdt, vdt)
        with rt.Graph(ctx) as g:
            arena.fill_normal(g, seed=9, length=kv_len if nan_tail else kv_len + extra)
            if nan_tail:
                nan = torch.full((1, extra, kvh, d), float("nan"), dtype=TORCH[kdt], device="cuda:0")
                rt.rope_kv_batch(g, arena, 0, kv_len, None, nan, nan)
            outs.append(rt.prefill_attention(g, arena, 0, start, q, out_dtype=torch.float32))
        assert arena.len() == kv_len + extra
    assert torch.isfinite(outs[1]).all()
    assert torch.equal(outs[0], outs[1])
