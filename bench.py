"""Benchmark of the MI355X GQA attention path (one GPU).

Headline workload (config.workload = "cfg4_batched_decode_fp16"): batched
independent-sequence decode attention, 256 sequences x 4096 positions of fp16
KV at Granite shapes (16 q / 8 kv heads, d 64), over 24 layers' worth of
independent caches (51.5 GB resident in HBM).  One step = one query token per
sequence through all 24 layers (24 decode launches, 2.147 GB of KV each).
`value` = microseconds per sequence-token across the 24 layers
(step time / 256).  `roofline` is the decode kernel's achieved HBM GB/s
(algorithmic bytes per launch / average launch time) against 8 TB/s.

The other BASELINE configurations are reported under "detail" with their own
rooflines.  The CPU baseline is the oracle (a restatement of the reference's
single-threaded CPU attention) timed on a bounded sample on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-detail] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def load_traffic(kernel_key):
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get(kernel_key)
    except (OSError, ValueError):
        return None


def roofline_hbm(bytes_per_launch, ms_per_launch, traffic=None):
    gbs = bytes_per_launch / (ms_per_launch * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}


# ---------------------------------------------------------------------------
# Achievable HBM on this box: a plain streaming read of 2 GiB (far beyond the
# 256 MB MALL) by the library's probe kernel, timed like the rest, so the
# decode rooflines can be read against the measured ceiling as well as the
# 8 TB/s specification.
# ---------------------------------------------------------------------------
def bench_hbm_probe(ctx, steps, warmup):
    import torch
    from qx_amd import runtime as rt
    stream = torch.cuda.current_stream()
    nbytes = 2 << 30
    x = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx, stream) as g:
        rt.fill_normal(g, x.view(torch.float32), seed=3)
    best = None
    for blocks in (1024, 2048, 4096):
        sink = torch.empty(blocks, dtype=torch.int32, device="cuda:0")
        g = rt.Graph(ctx, stream)

        def step():
            rt.hbm_read_probe(g, x, sink, blocks)

        ms = timed(step, steps, warmup, stream)
        g.finish()
        gbs = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbs > best[1]:
            best = (blocks, gbs)
    return {"read_gb_per_s": round(best[1], 1), "read_frac_of_peak": round(best[1] / HBM_PEAK_GBS, 4),
            "blocks": best[0],
            "note": "one streaming read of 2 GiB (16-byte nontemporal loads, best of 1024/2048/4096 workgroups; "
                    "qxh_encode_hbm_read_probe): the HBM rate a plain streaming kernel reaches on this box"}


# ---------------------------------------------------------------------------
# cfg4: batched fp16 decode, 256 x 4096, 24 layers of independent caches
# ---------------------------------------------------------------------------
def bench_cfg4(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    S, L, LAYERS = 256, 4096, 24
    stream = torch.cuda.current_stream()
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, S, L, abi.F16)
    q = torch.empty((LAYERS, S, 16, 64), device="cuda:0")
    out = torch.empty_like(q)
    with rt.Graph(ctx, stream) as g:
        arena.fill_normal(g, seed=4, length=L)
        rt.fill_normal(g, q, seed=44)
    ws_bytes = rt.attention_workspace_bytes(arena, S, L)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda:0")

    g = rt.Graph(ctx, stream)

    def step():
        for layer in range(LAYERS):
            rt.attention(g, arena, layer, q[layer], L, out=out[layer], workspace=ws)

    ms = timed(step, steps, warmup, stream)
    g.finish()
    kv_bytes = S * 8 * L * 64 * 2 * 2
    io_bytes = 2 * S * 16 * 64 * 4
    per_launch_ms = ms / LAYERS
    res = {
        "ms_per_step": ms,
        "us_per_sequence_token": ms * 1000.0 / S,
        "us_per_layer_step": per_launch_ms * 1000.0,
        "bytes_per_launch": kv_bytes + io_bytes,
        "roofline": roofline_hbm(kv_bytes + io_bytes, per_launch_ms, load_traffic("cfg4_decode")),
        "launches_per_step": LAYERS,
    }
    del arena
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# Tiered values: Granite batched decode at ctx 4096 on the reference's
# canonical KV plan (fp32 K, f16 V) and on fp32 K with tiered values (f16
# window of 256, INT8 blocks before it), same shape, same kernel family.
# ---------------------------------------------------------------------------
def bench_tiered_v(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    S, L, LAYERS, W = 64, 4096, 8, 256
    stream = torch.cuda.current_stream()
    q = torch.empty((LAYERS, S, 16, 64), device="cuda:0")
    out = torch.empty_like(q)
    with rt.Graph(ctx, stream) as g:
        rt.fill_normal(g, q, seed=45)
    res = {"shape": f"{S} sequences x ctx {L}, Granite, {LAYERS} layers", "window": W}
    k_bytes = S * 8 * L * 64 * 4
    io_bytes = 2 * S * 16 * 64 * 4
    plans = (("fp32k_f16v", abi.F16, 0, S * 8 * L * 64 * 2),
             ("fp32k_tiered", abi.I8_TIERED, W, S * 8 * ((L - W) * (64 + 4) + W * 64 * 2)))
    for name, vdt, window, v_bytes in plans:
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, S, L, abi.F32, vdt, value_window=window)
        with rt.Graph(ctx, stream) as g:
            arena.fill_normal(g, seed=4, length=L)
        ws = torch.empty(max(rt.attention_workspace_bytes(arena, S, L), 1), dtype=torch.uint8, device="cuda:0")
        g = rt.Graph(ctx, stream)

        def step():
            for layer in range(LAYERS):
                rt.attention(g, arena, layer, q[layer], L, out=out[layer], workspace=ws)

        ms = timed(step, steps, warmup, stream)
        g.finish()
        per_launch_ms = ms / LAYERS
        nbytes = k_bytes + v_bytes + io_bytes
        res[name] = {"us_per_layer_step": round(per_launch_ms * 1000.0, 2), "bytes_per_launch": nbytes,
                     "arena_bytes": arena.arena.numel() - 256,
                     "roofline": roofline_hbm(nbytes, per_launch_ms)}
        del arena, ws
        torch.cuda.empty_cache()
    res["speedup"] = round(res["fp32k_f16v"]["us_per_layer_step"] / res["fp32k_tiered"]["us_per_layer_step"], 3)
    # Qwen at cfg 5a's shape (batch 1, ctx 32768, bf16 K, 48 layers replayed)
    # with a window of 1024: the VALU tiered kernel against cfg 5a's MFMA path
    QL, QN, QW = 48, 32768, 1024
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, QL, 1, QN, abi.BF16, abi.I8_TIERED, value_window=QW)
    qq = torch.empty((QL, 1, 32, 128), dtype=torch.bfloat16, device="cuda:0")
    qo = torch.empty_like(qq)
    with rt.Graph(ctx, stream) as g:
        arena.fill_normal(g, seed=5, length=QN)
        rt.fill_normal(g, qq, seed=55)
    ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, QN), 1), dtype=torch.uint8, device="cuda:0")
    g = rt.Graph(ctx, stream)
    g.capture_begin()
    for layer in range(QL):
        rt.attention(g, arena, layer, qq[layer], QN, out=qo[layer], workspace=ws)
    replay = g.capture_end()
    g.discard()
    ms = timed(lambda: replay.launch(stream), steps, warmup, stream)
    per_layer = ms / QL
    nbytes = 4 * (QN * 128 * 2 + (QN - QW) * (128 + 8) + QW * 128 * 2)
    res["qwen_bf16k_tiered_ctx32768"] = {"us_per_layer": round(per_layer * 1000.0, 2), "bytes_per_layer": nbytes,
                                         "roofline": roofline_hbm(nbytes, per_layer)}
    del replay, arena, ws
    torch.cuda.empty_cache()
    # cfg 5b's prompt (Qwen, 8192 tokens, bf16 K) over tiered values: the
    # pipelined prefill with the tiered V^T pre-pass, timed like cfg 5b
    T = 8192
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, 1, 1, T, abi.BF16, abi.I8_TIERED, value_window=QW)
    kv = torch.empty((1, T, 4, 128), dtype=torch.bfloat16, device="cuda:0")
    qp = torch.empty((T, 32, 128), dtype=torch.bfloat16, device="cuda:0")
    with rt.Graph(ctx, stream) as g:
        rt.fill_normal(g, kv, seed=61)
        rt.fill_normal(g, qp, seed=62)
        rt.store_kv(g, arena, 0, 0, kv, kv)
    ws = torch.empty(max(rt.prefill_workspace_bytes(arena, T), 1), dtype=torch.uint8, device="cuda:0")
    po = torch.empty_like(qp)

    g = rt.Graph(ctx, stream)
    ms = timed(lambda: rt.prefill_attention(g, arena, 0, 0, qp, out=po, workspace=ws), steps, warmup, stream)
    g.finish()
    tflops = 4.0 * 128 * 32 * T * (T + 1) / 2 / (ms * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS["bf16"]
    res["qwen_bf16k_tiered_prefill_8192"] = {
        "us_per_prefill": round(ms * 1000.0, 1),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None}}
    del arena, ws
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# cfg1: one Granite layer, positions 0..511 (fp32), captured once, replayed
# ---------------------------------------------------------------------------
def bench_cfg1(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    P = 512
    stream = torch.cuda.current_stream()
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, P, abi.F32)
    q = torch.empty((P, 1, 1, 16, 64), device="cuda:0")
    k = torch.empty((P, 1, 1, 8, 64), device="cuda:0")
    v = torch.empty_like(k)
    qo = torch.empty_like(q)
    out = torch.empty((P, 1, 16, 64), device="cuda:0")
    ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, P), 1), dtype=torch.uint8, device="cuda:0")
    with rt.Graph(ctx, stream) as g:
        for t, s in ((q, 1), (k, 2), (v, 3)):
            rt.fill_normal(g, t, seed=s)
    g = rt.Graph(ctx, stream)
    g.capture_begin()
    for p in range(P):
        # RoPE + append + attention of one token (the reference call site's
        # encode_rope_kv_for_layer + encode_attention pair) in one dispatch
        rt.decode_step(g, arena, 0, p, q[p].view(16, 64), k[p].view(8, 64), v[p].view(8, 64),
                       query_out=qo[p].view(16, 64), out=out[p].view(16, 64), workspace=ws)
    replay = g.capture_end()
    g.discard()
    ms = timed(lambda: replay.launch(stream), steps, warmup, stream)
    total_kv = sum(4096 * (p + 1) for p in range(P))
    return {"us_per_token": ms * 1000.0 / P, "ms_per_512_steps": ms,
            "roofline": roofline_hbm(total_kv / P, ms / P, None),
            "note": "one token = RoPE + append + decode attention in one launch (qxh_encode_decode_step_for_layer), HIP-graph replay"}


# ---------------------------------------------------------------------------
# cfg2: Granite 24-layer attention-only stack at ctx 4096 (fp32 KV); fp32
# dense weights, or (cfg2q4) group-32 Q4 weights
# ---------------------------------------------------------------------------
def bench_cfg2(ctx, steps, warmup, q4=False):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    LAYERS, POS = 24, 4095
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device="cuda:0")
    sets = []
    for s in range(2):  # two independent weight+cache sets so the 256 MB MALL cannot hold a token
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, LAYERS, 1, 4096, abi.F32)
        layers = []
        with rt.Graph(ctx, stream) as g:
            arena.fill_normal(g, seed=10 + s, length=POS)
            for layer in range(LAYERS):
                norm = torch.ones(1024, device="cuda:0")
                if q4:
                    # uniform random codes, scales 0.02 / 7 (f16): the weight values
                    # do not change the work
                    gen.manual_seed(1000 * s + layer)
                    mats = []
                    for rows in (1024, 512, 512, 1024):
                        codes = torch.randint(0, 256, (rows, 512), dtype=torch.uint8, device="cuda:0",
                                              generator=gen)
                        scales = torch.full((rows, 32), 0.02 / 7, dtype=torch.float16,
                                            device="cuda:0").view(torch.int16)
                        mats.append(rt.Q4Matrix(codes, scales, rows, 1024))
                    layers.append(rt.GraniteQ4Layer(norm, *mats))
                    continue
                wq = torch.empty((1024, 1024), device="cuda:0")
                wk = torch.empty((512, 1024), device="cuda:0")
                wv = torch.empty((512, 1024), device="cuda:0")
                wo = torch.empty((1024, 1024), device="cuda:0")
                for i, w in enumerate((wq, wk, wv, wo)):
                    rt.fill_normal(g, w, seed=1000 * s + 10 * layer + i, stddev=0.02)
                layers.append(rt.GraniteLayer(norm, wq, wk, wv, wo))
        hidden = [torch.empty(1024, device="cuda:0") for _ in range(LAYERS + 1)]
        inv = torch.empty(LAYERS, device="cuda:0")
        with rt.Graph(ctx, stream) as g:
            rt.fill_normal(g, hidden[0], seed=77 + s)
        ws = torch.empty(rt.granite_block_workspace_bytes(arena, POS + 1), dtype=torch.uint8, device="cuda:0")
        g = rt.Graph(ctx, stream)
        g.capture_begin()
        for layer in range(LAYERS):
            if q4:
                rt.granite_attention_block_q4(g, arena, layer, POS, layers[layer], hidden[layer], hidden[layer + 1],
                                              ws, inv[layer:layer + 1])
            else:
                rt.granite_attention_block(g, arena, layer, POS, layers[layer], hidden[layer], hidden[layer + 1], ws)
        replay = g.capture_end()
        g.discard()
        sets.append((arena, layers, hidden, ws, replay, inv))
    it = [0]

    def step():
        sets[it[0] & 1][4].launch(stream)
        it[0] += 1

    ms = timed(step, steps, warmup, stream)
    if q4:
        # codes (rows x 512 B) + f16 scales (rows x 64 B) for q, k, v, o
        weights = LAYERS * (1024 + 512 + 512 + 1024) * (512 + 64)
        note = ("24 x (norm+Q4 QKV+RoPE+append, decode attention, Q4 O+residual, residual inverse RMS) per token, "
                "group-32 Q4 weights (random codes), HIP-graph replay, 2 rotated weight/cache sets; roofline is "
                "for the whole token")
    else:
        weights = LAYERS * (1024 * 1024 * 2 + 512 * 1024 * 2) * 4
        note = ("24 x (norm+QKV+RoPE+append, decode attention, O+residual) per token, HIP-graph replay, "
                "2 rotated weight/cache sets; roofline is for the whole token")
    kv = LAYERS * 4096 * 8 * 64 * 4 * 2
    return {"us_per_token": ms * 1000.0, "bytes_per_token": weights + kv,
            "roofline": roofline_hbm(weights + kv, ms, None), "note": note}


# ---------------------------------------------------------------------------
# Qwen attention half (Q4 projections) for 48 layers at ctx 32768, f16 KV
# ---------------------------------------------------------------------------
def bench_qwen_block(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    LAYERS, POS = 48, 32767
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device="cuda:0")
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, LAYERS, 1, POS + 1, abi.F16)
    layers = []
    with rt.Graph(ctx, stream) as g:
        arena.fill_normal(g, seed=21, length=POS)
    for layer in range(LAYERS):
        gen.manual_seed(5000 + layer)
        mats = []
        for rows, cols in ((4096, 2048), (512, 2048), (512, 2048), (2048, 4096)):
            codes = torch.randint(0, 256, (rows, cols // 2), dtype=torch.uint8, device="cuda:0", generator=gen)
            scales = torch.full((rows, cols // 32), 0.02 / 7, dtype=torch.float16, device="cuda:0").view(torch.int16)
            mats.append(rt.Q4Matrix(codes, scales, rows, cols))
        ones = lambda n: torch.ones(n, device="cuda:0")
        layers.append(rt.QwenQ4Layer(ones(2048), mats[0], mats[1], mats[2], ones(128), ones(128), mats[3],
                                     ones(2048)))
    hidden = [torch.empty(2048, dtype=torch.float16, device="cuda:0") for _ in range(LAYERS + 1)]
    moe = torch.empty(2048, dtype=torch.float16, device="cuda:0")
    with rt.Graph(ctx, stream) as g:
        rt.fill_normal(g, hidden[0], seed=78)
    ws = torch.empty(rt.qwen_block_workspace_bytes(arena, POS + 1), dtype=torch.uint8, device="cuda:0")
    g = rt.Graph(ctx, stream)
    g.capture_begin()
    for layer in range(LAYERS):
        rt.qwen_attention_block(g, arena, layer, POS, layers[layer], hidden[layer], hidden[layer + 1], moe, ws)
    replay = g.capture_end()
    g.discard()
    ms = timed(lambda: replay.launch(stream), steps, warmup, stream)
    weights = (4096 + 512 + 512) * (1024 + 128) + 2048 * (2048 + 256)  # Q4 codes + f16 scales
    kv = (POS + 1) * 4 * 128 * 2 * 2
    per_token = LAYERS * (weights + kv)
    return {"us_per_token": ms * 1000.0, "us_per_layer": ms * 1000.0 / LAYERS, "bytes_per_token": per_token,
            "roofline": roofline_hbm(per_token, ms, None),
            "note": "48 x Qwen attention half (norm + Q4 q/k/v, q/k head norm + RoPE + append, split-K attention "
                    "over 32768 f16 positions, Q4 o, residual + post-attention norm) per token, random Q4 codes, "
                    "HIP-graph replay; roofline is for the whole token"}


# ---------------------------------------------------------------------------
# cfg5a: Qwen decode at ctx 32768, bf16 KV, 48 layers' caches rotated
# ---------------------------------------------------------------------------
def bench_cfg5a(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    LAYERS, L = 48, 32768
    stream = torch.cuda.current_stream()
    arena = rt.KvArena(ctx, abi.SHAPE_QWEN3, LAYERS, 1, L, abi.BF16)
    q = torch.empty((LAYERS, 1, 32, 128), dtype=torch.bfloat16, device="cuda:0")
    out = torch.empty_like(q)
    with rt.Graph(ctx, stream) as g:
        arena.fill_normal(g, seed=5, length=L)
        rt.fill_normal(g, q, seed=55)
    ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, L), 1), dtype=torch.uint8, device="cuda:0")
    g = rt.Graph(ctx, stream)
    g.capture_begin()
    for layer in range(LAYERS):
        rt.attention(g, arena, layer, q[layer], L, out=out[layer], workspace=ws)
    replay = g.capture_end()
    g.discard()
    ms = timed(lambda: replay.launch(stream), steps, warmup, stream)
    per_layer = ms / LAYERS
    kv = L * 4 * 128 * 2 * 2
    return {"us_per_layer": per_layer * 1000.0, "bytes_per_layer": kv,
            "roofline": roofline_hbm(kv, per_layer, load_traffic("cfg5a_decode")),
            "note": "48 layers' caches (3.2 GB) replayed per step; per-layer = decode + combine"}


# ---------------------------------------------------------------------------
# KV commitment leaves of every token row of one cfg4-sized layer
# ---------------------------------------------------------------------------
# Algorithmic VALU work of one BLAKE3 compression: 7 rounds x 8 G functions x
# (6 adds + 4 xors + 4 rotates) on 32-bit words.  A leaf of 1024-byte K and V
# rows takes 2 x 4 chunk leaves of 5 blocks, 2 x 3 tree parents and 2 blocks of
# the leaf itself: 48 compressions.
B3_OPS_PER_COMPRESSION = 7 * 8 * 14
VALU_PEAK_TOPS = 256 * 4 * 32 * 2.4e9 / 1e12  # 32-bit lane ops/s: MI355X FP32 vector peak / 2


def bench_kv_hash(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    SEQS, L = 256, 4096
    stream = torch.cuda.current_stream()
    arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, SEQS, L, abi.F16)
    with rt.Graph(ctx, stream) as g:
        arena.fill_normal(g, seed=21, length=L)
    out = torch.empty((SEQS, L, 32), dtype=torch.uint8, device="cuda:0")
    g = rt.Graph(ctx, stream)
    ms = timed(lambda: arena.leaf_hashes(g, 0, 0, L, sequences=SEQS, out=out), steps, warmup, stream)
    g.finish()
    leaves = SEQS * L
    row = 8 * 64 * 2
    ops = leaves * 48 * B3_OPS_PER_COMPRESSION
    tops = ops / (ms * 1e-3) / 1e12
    return {"us_per_layer": ms * 1000.0, "leaves": leaves, "kv_bytes": leaves * 2 * row,
            "gb_per_s": leaves * 2 * row / (ms * 1e-3) / 1e9, "leaves_per_s": leaves / (ms * 1e-3),
            "roofline": {"bound": "valu", "achieved": round(tops, 2), "peak": round(VALU_PEAK_TOPS, 1),
                         "unit": "Top/s", "frac": round(tops / VALU_PEAK_TOPS, 4), "traffic": None},
            "note": "kv_leaf_hash_v1 (BLAKE3) of all 256 x 4096 fp16 token rows of one Granite layer; "
                    "ops = 48 compressions x 784 32-bit ops per leaf"}


# ---------------------------------------------------------------------------
# cfg3 / cfg5b: causal prefill (MFMA)
# ---------------------------------------------------------------------------
def bench_prefill(ctx, steps, warmup, shape_name):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    if shape_name == "cfg3":
        shape, dtype, T = abi.SHAPE_GRANITE, abi.F16, 2048
    else:
        shape, dtype, T = abi.SHAPE_QWEN3, abi.BF16, 8192
    info = rt.shape_info(shape)
    tdt = rt.torch_dtype(dtype)
    stream = torch.cuda.current_stream()
    arena = rt.KvArena(ctx, shape, 1, 1, T, dtype)
    q = torch.empty((1, T, info.q_heads, info.head_dim), dtype=tdt, device="cuda:0")
    k = torch.empty((1, T, info.kv_heads, info.head_dim), dtype=tdt, device="cuda:0")
    v = torch.empty_like(k)
    qo = torch.empty_like(q)
    out = torch.empty((T, info.q_heads, info.head_dim), dtype=tdt, device="cuda:0")
    with rt.Graph(ctx, stream) as g:
        for i, t in enumerate((q, k, v)):
            rt.fill_normal(g, t, seed=200 + i)
        rt.rope_kv_batch(g, arena, 0, 0, q, k, v, query_out=qo)
    ws = torch.empty(max(rt.prefill_workspace_bytes(arena, T), 1), dtype=torch.uint8, device="cuda:0")
    # eager launches on the stream (one prefill call per step): a graph replay
    # adds a fixed launch cost per replay that a single call does not amortise
    g = rt.Graph(ctx, stream)
    ms = timed(lambda: rt.prefill_attention(g, arena, 0, 0, qo[0], out=out, workspace=ws), steps, warmup, stream)
    g.finish()
    flops = 4.0 * info.head_dim * info.q_heads * T * (T + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS["f16" if dtype == abi.F16 else "bf16"]
    return {"us_per_prefill": ms * 1000.0, "tokens": T, "flop": flops,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(tflops / peak, 4), "traffic": None},
            "note": "causal attention only (RoPE/append excluded), eager stream launches; flop = 4*D*Hq*T(T+1)/2"}


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's single-threaded Granite attention on a sample
# ---------------------------------------------------------------------------
def cpu_baseline(seconds=10.0):
    import concurrent.futures as cf

    import numpy as np

    from oracle import oracle as O

    L = 4096
    rng = np.random.default_rng(0)
    keys = rng.standard_normal((L, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    vals = rng.standard_normal((L, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal(1024, dtype=np.float32)

    def make_cache():
        c = O.KvCache(L)
        c.extend(keys, vals)
        return c

    cache = make_cache()
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds or n < 3:
        O.granite_attend(q, cache, L)
        n += 1
    t1 = (time.perf_counter() - t0) / n
    cores = os.cpu_count() or 1
    cores = min(cores, 16)
    caches = [make_cache() for _ in range(cores)]
    per_thread = max(2, n // cores)

    def work(c):
        for _ in range(per_thread):
            O.granite_attend(q, c, L)

    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(cores) as ex:
        list(ex.map(work, caches))
    tall = (time.perf_counter() - t0) / (per_thread * cores)
    # KV commitment leaves of fp16 token rows (1024-byte K and V rows), one thread
    krow = keys[:256].astype(np.float16).tobytes()
    vrow = vals[:256].astype(np.float16).tobytes()
    nh = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 2.0 or nh < 100:
        O.kv_leaf_hash_v1(0, nh, krow[(nh % 256) * 1024:(nh % 256 + 1) * 1024],
                          vrow[(nh % 256) * 1024:(nh % 256 + 1) * 1024])
        nh += 1
    th = (time.perf_counter() - t0) / nh
    return {
        "value": round(t1 * 24 * 1e6, 1), "unit": "us/sequence-token (24 layers)", "cores": 1, "kind": "port",
        "sample": f"{n} single-thread oracle attends of one Granite layer at ctx 4096 (fp16-rounded KV, "
                  f"upcast fp32 math), x24 layers; cfg4 step = 256 sequences",
        "all_core": {"value": round(tall * 24 * 1e6, 1), "cores": cores,
                     "sample": f"{per_thread * cores} attends over {cores} threads (independent sequences)"},
        "kv_hash": {"value": round(1.0 / th, 1), "unit": "leaves/s", "cores": 1, "kind": "port",
                    "sample": f"{nh} oracle kv_leaf_hash_v1 calls on 1024-byte fp16 K and V rows "
                              f"(includes the Python call overhead)"},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (known bytes) to scale rocprofv3 FETCH/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from qx_amd import runtime as rt

    ctx = rt.Context(0)
    side = torch.cuda.Stream()  # default priority; HIP-graph capture needs a non-null stream
    with torch.cuda.stream(side):
        run(ctx, args)


def run(ctx, args):
    import torch

    if args.calibrate_copy:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 1073741824 bytes read + 1073741824 bytes written per dispatch")
        del src, dst

    only = set(filter(None, args.only.split(",")))
    detail = {}
    head = bench_cfg4(ctx, args.steps, args.warmup) if (not only or "cfg4" in only) else None
    if head:
        log("cfg4", json.dumps(head))
    if not args.no_detail:
        for name, fn in (("hbm_probe", bench_hbm_probe), ("cfg1", bench_cfg1), ("cfg2", bench_cfg2),
                         ("cfg2q4", lambda c, k, w: bench_cfg2(c, k, w, q4=True)),
                         ("cfg3", lambda c, k, w: bench_prefill(c, k, w, "cfg3")),
                         ("cfg5a", bench_cfg5a), ("qwenblock", bench_qwen_block), ("cfg5b", lambda c, k, w: bench_prefill(c, k, w, "cfg5b")),
                         ("kvhash", bench_kv_hash), ("tieredv", bench_tiered_v)):
            if only and name not in only:
                continue
            try:
                detail[name] = fn(ctx, max(3, args.steps), args.warmup)
                log(name, json.dumps(detail[name]))
            except Exception as e:  # report, keep the headline
                detail[name] = {"error": str(e)}
                log(name, "error", e)
            torch.cuda.empty_cache()
    if head and isinstance(detail.get("hbm_probe"), dict) and "read_gb_per_s" in detail["hbm_probe"]:
        head["frac_of_hbm_probe"] = round(head["roofline"]["achieved"] / detail["hbm_probe"]["read_gb_per_s"], 4)
    cpu = None if args.no_cpu else cpu_baseline()
    if head is None:
        print(json.dumps({"detail": detail, "cpu_baseline": cpu}))
        return
    line = {
        "metric": "decode attn µs/token & HBM GB/s (% peak); prefill attn TFLOP/s (% MFMA peak)",
        "value": round(head["us_per_sequence_token"], 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: N(0,1) KV and queries generated on device (SplitMix64 + Box-Muller), seeded",
        "config": {"workload": "cfg4_batched_decode_fp16", "sequences": 256, "context": 4096, "layers": 24,
                   "q_heads": 16, "kv_heads": 8, "head_dim": 64, "kv_dtype": "f16",
                   "step": "one query token per sequence through 24 layers of independent caches"},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "detail": {"cfg4": {k: v for k, v in head.items() if k != "roofline"}, **detail},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
