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


_SLEEP_CYCLES_PER_US = None


def gpu_hold(stream, us):
    """Keep the GPU busy for about `us` microseconds (torch's bounded
    cycle-count spin kernel) so that work the host enqueues behind it is
    timed by its events without the host's launch cost in between."""
    import torch
    global _SLEEP_CYCLES_PER_US
    if _SLEEP_CYCLES_PER_US is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record(stream)
        torch.cuda._sleep(2_000_000)
        e1.record(stream)
        e1.synchronize()
        _SLEEP_CYCLES_PER_US = 2_000_000 / max(e0.elapsed_time(e1) * 1000.0, 1.0)
    torch.cuda._sleep(int(us * _SLEEP_CYCLES_PER_US))


def source_digest(paths):
    """sha256 over the named repository files (the sources a kernel is built from)."""
    import hashlib
    h = hashlib.sha256()
    for rel in sorted(paths):
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(rel.encode() + b"\0" + f.read())
    return h.hexdigest()


def load_traffic(kernel_key):
    """HBM bytes per launch of a kernel from profiles/traffic.json (rocprofv3
    FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size).  Reported only
    when the sources the measurement was taken on are the sources of this
    tree, so the figure is evidence for the kernel that ran; else None."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get(kernel_key)
    except (OSError, ValueError):
        return None
    if not isinstance(entry, dict) or "sources" not in entry:
        return None
    try:
        if source_digest(entry["sources"]) != entry["source_sha256"]:
            log(f"traffic {kernel_key}: kernel sources changed since the measurement; not reported")
            return None
    except OSError:
        return None
    return entry["traffic_bytes"]


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
                         "unit": "Top/s", "frac": round(tops / VALU_PEAK_TOPS, 4), "traffic": load_traffic("kvhash")},
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
    flops = 4.0 * info.head_dim * info.q_heads * T * (T + 1) / 2
    tflops = flops / (ms * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS["f16" if dtype == abi.F16 else "bf16"]

    g.finish()

    # the prompt's front end: RoPE of q and k (Qwen: per-head RMSNorm first)
    # and the K/V append of all T rows, one launch per prompt.  Input sets
    # are rotated so they total more than the 256 MB memory-side cache (every
    # call reads its q/k/v from HBM), and all sets' calls are captured in one
    # HIP graph (the cursor rewinds on the host between captured calls), so
    # the replay time is GPU time with no host launch cost per call.
    eb = 2
    fe_in = T * (info.q_heads + 2 * info.kv_heads) * info.head_dim * eb
    fe_bytes = 2 * fe_in
    nsets = max(2, -(-(320 << 20) // fe_in))
    sets = []
    with rt.Graph(ctx, stream) as g:
        for i in range(nsets):
            ts = [torch.empty_like(t) for t in (q, k, v)]
            for j, t in enumerate(ts):
                rt.fill_normal(g, t, seed=400 + 3 * i + j)
            sets.append(ts)
    qos = [torch.empty_like(qo) for _ in range(2)]
    g = rt.Graph(ctx, stream)
    g.capture_begin()
    for i, (qi, ki, vi) in enumerate(sets):
        arena.set_len(0)
        rt.rope_kv_batch(g, arena, 0, 0, qi, ki, vi, query_out=qos[i & 1])
    replay = g.capture_end()
    g.discard()
    ms_fe = timed(lambda: replay.launch(stream), max(3, steps // 2), 2, stream) / nsets
    del replay, sets, qos
    # the floor of a one-shot read + write of the same bytes on this box: the
    # library's copy probe over as many rotated sources, one graph, nontemporal
    # and ordinary stores (the better of the two)
    cp_bytes = -(-fe_in // 4096) * 4096
    srcs = [torch.empty(cp_bytes, dtype=torch.uint8, device="cuda:0") for _ in range(nsets)]
    dsts = [torch.empty(cp_bytes, dtype=torch.uint8, device="cuda:0") for _ in range(2)]
    copy_us = {}
    for nt in (True, False):
        g = rt.Graph(ctx, stream)
        g.capture_begin()
        for i, src in enumerate(srcs):
            rt.hbm_copy_probe(g, src, dsts[i & 1], nt)
        replay = g.capture_end()
        g.discard()
        copy_us[nt] = timed(lambda: replay.launch(stream), max(3, steps // 2), 2, stream) / nsets * 1000.0
        del replay
    del srcs, dsts
    copy_floor = min(copy_us.values())
    return {"us_per_prefill": ms * 1000.0, "tokens": T, "flop": flops,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(tflops / peak, 4), "traffic": None},
            "frontend": {"us": round(ms_fe * 1000.0, 2), "bytes": fe_bytes,
                         "roofline": roofline_hbm(fe_bytes, ms_fe, load_traffic(f"{shape_name}_frontend")),
                         "copy_floor": {"us": round(copy_floor, 2), "bytes": 2 * cp_bytes,
                                        "nontemporal_us": round(copy_us[True], 2), "plain_us": round(copy_us[False], 2),
                                        "frac": round(copy_floor / (ms_fe * 1000.0), 4),
                                        "note": "qxh_encode_hbm_copy_probe: one launch reading and writing the front "
                                                "end's bytes, replayed like it; frac = floor / front end"},
                         "note": "RoPE of q and k" + (" after per-head RMSNorm" if shape != abi.SHAPE_GRANITE else "") +
                                 ", K/V append of every prompt row, one launch (qxh_encode_rope_kv_batch); bytes = "
                                 f"q, k, v read + rotated q, cache K, cache V written; {nsets} input sets rotated "
                                 "(more than the 256 MB memory-side cache), their calls replayed as one HIP graph"},
            "prompt_total_us": round((ms + ms_fe) * 1000.0, 2),
            "note": "us_per_prefill/roofline: causal attention only, eager stream launches; flop = 4*D*Hq*T(T+1)/2; "
                    "prompt_total_us = front end + attention"}


# ---------------------------------------------------------------------------
# Long prompt on the reference's canonical KV plan (Fp32KFp16V: fp32 keys,
# f16 values) and on fp32 K/V: cfg 3's Granite prompt of 2048 tokens, fp32
# queries, causal attention through qxh_encode_prefill_attention.
# ---------------------------------------------------------------------------
def bench_prefill_fp32(ctx, steps, warmup):
    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    T = 2048
    stream = torch.cuda.current_stream()
    res = {}
    for name, kdt, vdt in (("fp32k_f16v", abi.F32, abi.F16), ("fp32", abi.F32, abi.F32),
                           ("fp32k_tiered", abi.F32, abi.I8_TIERED)):
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, T, kdt, vdt, value_window=256 if vdt == abi.I8_TIERED else 0)
        q = torch.empty((1, T, 16, 64), device="cuda:0")
        k = torch.empty((1, T, 8, 64), device="cuda:0")
        v = torch.empty_like(k)
        qo = torch.empty_like(q)
        out = torch.empty((T, 16, 64), device="cuda:0")
        with rt.Graph(ctx, stream) as g:
            for i, t in enumerate((q, k, v)):
                rt.fill_normal(g, t, seed=300 + i)
            rt.rope_kv_batch(g, arena, 0, 0, q, k, v, query_out=qo)
        ws = torch.empty(max(rt.prefill_workspace_bytes(arena, T), 1), dtype=torch.uint8, device="cuda:0")
        g = rt.Graph(ctx, stream)
        ms = timed(lambda: rt.prefill_attention(g, arena, 0, 0, qo[0], out=out, workspace=ws), steps, warmup, stream)
        g.finish()
        flops = 4.0 * 64 * 16 * T * (T + 1) / 2
        tflops = flops / (ms * 1e-3) / 1e12
        res[name] = {"us_per_prefill": round(ms * 1000.0, 1), "tflops": round(tflops, 2),
                     "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 157.3, "unit": "TFLOP/s",
                                  "frac": round(tflops / 157.3, 4), "traffic": None}}
        del arena, ws
        torch.cuda.empty_cache()
    res["note"] = ("Granite causal prefill of 2048 tokens, fp32 queries and outputs; fp32k_tiered: fp32 K with "
                   "tiered values (f16 window of 256 rows, block INT8 below); peak = dense fp32 MFMA "
                   "(157.3 TFLOP/s); flop = 4*D*Hq*T(T+1)/2")
    return res


# ---------------------------------------------------------------------------
# The reference's isolated decode-attention sweep (--v2-attention-sweep:
# Granite, one layer, batch 1, fp32 K/V at ctx 32..512, one attention per
# command buffer, median of the command buffers' GPU times) and its
# K/V-precision table at ctx 512 (fp32 K/V, fp16 K, fp16 V): here each
# attention call is bracketed by HIP events on its stream, all of them queued
# behind a spin kernel so the events time the GPU alone (median of >= 50),
# and separately the host wall time of graph begin -> finish per call.
# ---------------------------------------------------------------------------
def bench_attention_sweep(ctx, steps, warmup):
    import statistics

    import torch
    from qx_amd import abi
    from qx_amd import runtime as rt

    reps = max(50, steps)
    stream = torch.cuda.current_stream()
    cases = [(f"fp32_ctx{L}", L, abi.F32, abi.F32) for L in (32, 64, 128, 256, 512)]
    cases += [("fp16k_ctx512", 512, abi.F16, abi.F32), ("fp16v_ctx512", 512, abi.F32, abi.F16)]
    eb = {abi.F32: 4, abi.F16: 2}
    res = {}
    for name, L, kdt, vdt in cases:
        arena = rt.KvArena(ctx, abi.SHAPE_GRANITE, 1, 1, L, kdt, vdt)
        q = torch.empty((1, 16, 64), device="cuda:0")
        out = torch.empty_like(q)
        with rt.Graph(ctx, stream) as g:
            arena.fill_normal(g, seed=31, length=L)
            rt.fill_normal(g, q, seed=32)
        ws = torch.empty(max(rt.attention_workspace_bytes(arena, 1, L), 1), dtype=torch.uint8, device="cuda:0")
        for _ in range(warmup):
            with rt.Graph(ctx, stream) as g:
                rt.attention(g, arena, 0, q, L, out=out, workspace=ws)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        gpu_hold(stream, 100.0 * reps)
        g = rt.Graph(ctx, stream)
        for e0, e1 in ev:
            e0.record(stream)
            rt.attention(g, arena, 0, q, L, out=out, workspace=ws)
            e1.record(stream)
        g.finish()
        torch.cuda.synchronize()
        gpu = statistics.median(e0.elapsed_time(e1) * 1000.0 for e0, e1 in ev)
        walls = []
        for _ in range(reps):
            t0 = time.perf_counter()
            with rt.Graph(ctx, stream) as g:
                rt.attention(g, arena, 0, q, L, out=out, workspace=ws)
            walls.append((time.perf_counter() - t0) * 1e6)
        # back to back in a decode loop: 32 calls captured in one HIP graph
        g = rt.Graph(ctx, stream)
        g.capture_begin()
        for _ in range(32):
            rt.attention(g, arena, 0, q, L, out=out, workspace=ws)
        replay = g.capture_end()
        g.discard()
        loop_us = timed(lambda: replay.launch(stream), 5, 2, stream) * 1000.0 / 32
        del replay
        nbytes = L * 8 * 64 * (eb[kdt] + eb[vdt]) + 2 * 16 * 64 * 4
        res[name] = {"context": L, "gpu_median_us": round(gpu, 2), "wall_median_us": round(statistics.median(walls), 2),
                     "graph_loop_us": round(loop_us, 2), "bytes": nbytes,
                     "roofline": roofline_hbm(nbytes, gpu / 1000.0, None)}
        del arena, ws
    res["note"] = (f"Granite, 1 layer, batch 1, attention only (qxh_encode_attention_for_layer), {reps} samples "
                   "per case; gpu = HIP events around each launch on its stream, every launch queued behind a "
                   "spin kernel so no host time falls between the events; wall = host time of graph begin -> "
                   "finish (synchronous) per call; graph_loop = per call in a HIP graph of 32 back-to-back calls; "
                   "the reference publishes 54.63-67.75 us GPU medians for the same cases on an Apple M5 Pro")
    return res


# ---------------------------------------------------------------------------
# CPU baselines: the oracle (a contraction-free C restatement of the
# reference's CPU path, built -O2) timed on this host's cores, for every
# configuration.  The reference attention is single-threaded, so each config
# gets a 1-thread figure; the all-core figure runs independent units (whole
# sequences, layers or query rows, each thread with its own cache) on the
# GPU box's CPU share.  Samples are bounded (a few seconds each) and scaled
# to the config's unit as stated in each entry.
# ---------------------------------------------------------------------------
def cpu_threads():
    """Threads for the all-core figures: the CPU share of one GPU on the
    box (16 threads, the OMP_NUM_THREADS the box sets), never more than the
    cores this process may run on."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS") or 16)
    return max(1, min(affinity, share, 16)), affinity, os.cpu_count() or 1


def _timed_loop(fn, seconds, min_iters=1):
    n = 0
    t0 = time.perf_counter()
    while n < min_iters or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def _threaded(fns, reps):
    """Run fns[i]() `reps` times on thread i, all started together (ctypes
    releases the GIL inside the oracle); returns the wall time."""
    import threading
    gate = threading.Barrier(len(fns) + 1)

    def work(fn):
        gate.wait()
        for _ in range(reps):
            fn()

    ts = [threading.Thread(target=work, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    gate.wait()
    t0 = time.perf_counter()
    for t in ts:
        t.join()
    return time.perf_counter() - t0


def _entry(value, unit, sample, all_value, threads, all_sample, **extra):
    e = {"value": round(value, 3), "unit": unit, "cores": 1, "kind": "port", "sample": sample,
         "all_core": {"value": round(all_value, 3), "cores": threads, "sample": all_sample}}
    e.update(extra)
    return e


def cpu_cfg1(O, np, threads, secs):
    """Config 1: granite_attention_decode for positions 0..511 of one layer."""
    P = 512
    g = np.random.default_rng(1)
    q = g.standard_normal((P, 1024), dtype=np.float32)
    k = g.standard_normal((P, 512), dtype=np.float32)
    v = g.standard_normal((P, 512), dtype=np.float32)

    def seq(cache):
        cache.reset()
        for p in range(P):
            O.granite_attention_decode(q[p], k[p], v[p], p, cache)

    c0 = O.KvCache(P)
    t1, n = _timed_loop(lambda: seq(c0), secs)
    caches = [O.KvCache(P) for _ in range(threads)]
    reps = max(1, n // 2)
    wall = _threaded([lambda c=c: seq(c) for c in caches], reps)
    return _entry(t1 * 1e6 / P, "us/token", f"{n} runs of the 512-step sequence (RoPE + append + attention per token)",
                  wall * 1e6 / (P * reps * threads), threads,
                  f"{threads} independent 512-step sequences x {reps} run(s) on {threads} threads; per-token time of "
                  f"the aggregate")


def cpu_cfg2(O, np, threads, secs):
    """Config 2: the attention half of a Granite layer at position 4095 over a
    4095-row fp32 cache; a token is 24 such layers."""
    g = np.random.default_rng(2)
    weights = []
    for _ in range(2):
        weights.append((np.ones(1024, np.float32),
                        (g.standard_normal((1024, 1024), dtype=np.float32) * 0.02),
                        (g.standard_normal((512, 1024), dtype=np.float32) * 0.02),
                        (g.standard_normal((512, 1024), dtype=np.float32) * 0.02),
                        (g.standard_normal((1024, 1024), dtype=np.float32) * 0.02)))
    keys = g.standard_normal((4095, 8, 64), dtype=np.float32)
    vals = g.standard_normal((4095, 8, 64), dtype=np.float32)
    hidden = g.standard_normal(1024, dtype=np.float32)

    def make_cache():
        c = O.KvCache(4096)
        c.extend(keys, vals)
        return c

    it = [0]

    def layer(cache, w):
        O.granite_attention_block(hidden, *w, 4095, cache)
        cache.rollback(4095)

    c0 = make_cache()

    def step():
        layer(c0, weights[it[0] & 1])
        it[0] += 1

    t1, n = _timed_loop(step, secs)
    caches = [make_cache() for _ in range(threads)]
    reps = max(1, n // 2)
    wall = _threaded([lambda c=c, i=i: layer(c, weights[i & 1]) for i, c in enumerate(caches)], reps)
    return _entry(t1 * 24 * 1e6, "us/token (24 layers)",
                  f"{n} single-thread layers (norm + fp32 q/k/v + RoPE + append + attention over 4096 positions + "
                  f"o + residual, two alternating weight sets), x24 layers",
                  wall * 24 * 1e6 / (reps * threads), threads,
                  f"{threads} threads x {reps} layers (own cache each), x24 layers")


def _prefill_scale(rows, T):
    """Work of all T causal rows over the work of the sampled rows (row t
    attends t + 1 positions)."""
    return (T * (T + 1) / 2) / float(sum(int(r) + 1 for r in rows))


def cpu_cfg3(O, np, threads, secs):
    """Config 3: causal prefill of 2048 Granite tokens over fp16-rounded K/V
    (the reference runs a prompt as repeated decode)."""
    T = 2048
    g = np.random.default_rng(3)
    keys = g.standard_normal((T, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    vals = g.standard_normal((T, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = g.standard_normal((T, 1024), dtype=np.float32).astype(np.float16).astype(np.float32)

    def make_cache():
        c = O.KvCache(T)
        c.extend(keys, vals)
        return c

    rows1 = np.linspace(0, T - 1, 64).astype(np.uint32)
    c0 = make_cache()
    t1, n = _timed_loop(lambda: O.granite_prefill_rows(q, c0, 0, rows1), secs)
    rows_all = np.linspace(0, T - 1, 32 * threads).astype(np.uint32)
    caches = [make_cache() for _ in range(threads)]
    wall = _threaded([lambda c=c, i=i: O.granite_prefill_rows(q, c, 0, rows_all[i::threads])
                      for i, c in enumerate(caches)], 1)
    return _entry(t1 * _prefill_scale(rows1, T) * 1e6, "us/prefill",
                  f"64 evenly spaced query rows of 2048 ({n} runs), scaled by the causal work of all rows "
                  f"(x{_prefill_scale(rows1, T):.1f})",
                  wall * _prefill_scale(rows_all, T) * 1e6, threads,
                  f"{rows_all.size} evenly spaced rows over {threads} threads (own cache each), scaled by the causal "
                  f"work of all rows (x{_prefill_scale(rows_all, T):.2f})")


def cpu_cfg4(O, np, threads, secs):
    """Config 4: one sequence-layer of decode at ctx 4096 over fp16-rounded K/V;
    the unit is a sequence-token over 24 layers."""
    L = 4096
    g = np.random.default_rng(0)
    keys = g.standard_normal((L, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    vals = g.standard_normal((L, 8, 64), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = g.standard_normal(1024, dtype=np.float32)

    def make_cache():
        c = O.KvCache(L)
        c.extend(keys, vals)
        return c

    c0 = make_cache()
    t1, n = _timed_loop(lambda: O.granite_attend(q, c0, L), secs)
    caches = [make_cache() for _ in range(threads)]
    reps = max(2, n // 2)
    wall = _threaded([lambda c=c: O.granite_attend(q, c, L) for c in caches], reps)
    return _entry(t1 * 24 * 1e6, "us/sequence-token (24 layers)",
                  f"{n} single-thread attends of one Granite layer at ctx 4096 (fp16-rounded KV, fp32 math), x24 "
                  f"layers; a cfg4 step is 256 sequence-tokens",
                  wall * 24 * 1e6 / (reps * threads), threads,
                  f"{reps * threads} attends over {threads} threads (independent sequences, own cache each), x24")


def cpu_cfg5a(O, np, threads, secs):
    """Config 5a: cpu_gqa_attention of one Qwen token at ctx 32768 (bf16)."""
    N = 32768
    g = np.random.default_rng(5)
    kc = O.to_bits16(g.standard_normal(N * 512, dtype=np.float32), O.BF16)
    vc = O.to_bits16(g.standard_normal(N * 512, dtype=np.float32), O.BF16)
    q = O.to_bits16(g.standard_normal(4096, dtype=np.float32), O.BF16)
    t1, n = _timed_loop(lambda: O.qwen_gqa_attention(q, kc, vc, O.BF16), secs)
    reps = max(1, n // 2)
    wall = _threaded([lambda: O.qwen_gqa_attention(q, kc, vc, O.BF16)] * threads, reps)
    return _entry(t1 * 1e6, "us/layer", f"{n} single-thread Qwen attentions over 32768 bf16 positions",
                  wall * 1e6 / (reps * threads), threads,
                  f"{threads} threads x {reps} attentions (independent layers; the threads share one read-only cache)")


def cpu_cfg5b(O, np, threads, secs):
    """Config 5b: causal prefill of 8192 Qwen tokens (bf16), rows as repeated
    cpu_gqa_attention."""
    T = 8192
    g = np.random.default_rng(6)
    kc = O.to_bits16(g.standard_normal(T * 512, dtype=np.float32), O.BF16)
    vc = O.to_bits16(g.standard_normal(T * 512, dtype=np.float32), O.BF16)
    q = O.to_bits16(g.standard_normal(T * 4096, dtype=np.float32), O.BF16)
    rows1 = np.linspace(0, T - 1, 16).astype(np.uint32)
    t1, n = _timed_loop(lambda: O.qwen_prefill_rows(q, kc, vc, 0, rows1, O.BF16), secs)
    rows_all = np.linspace(0, T - 1, 8 * threads).astype(np.uint32)
    wall = _threaded([lambda i=i: O.qwen_prefill_rows(q, kc, vc, 0, rows_all[i::threads], O.BF16)
                      for i in range(threads)], 1)
    return _entry(t1 * _prefill_scale(rows1, T) * 1e6, "us/prefill",
                  f"16 evenly spaced query rows of 8192 ({n} runs), scaled by the causal work of all rows "
                  f"(x{_prefill_scale(rows1, T):.1f})",
                  wall * _prefill_scale(rows_all, T) * 1e6, threads,
                  f"{rows_all.size} evenly spaced rows over {threads} threads, scaled by the causal work of all rows "
                  f"(x{_prefill_scale(rows_all, T):.2f})")


def cpu_frontends(O, np, threads, secs):
    """The prompt front ends on the CPU: apply_granite_rope of cfg 3's 2048
    tokens and cpu_qk_norm_rope of cfg 5b's 8192 (bf16), as C loops over
    token rows (the K/V append is a row copy, included in neither).  1 thread:
    a run of rows scaled to the prompt; all cores: the prompt's rows split
    over the threads (independent tokens)."""
    g = np.random.default_rng(8)
    q = g.standard_normal((2048, 1024), dtype=np.float32)
    k = g.standard_normal((2048, 512), dtype=np.float32)
    tg, ng = _timed_loop(lambda: O.apply_granite_rope_rows(q[:256], k[:256], 0), secs / 4)
    n = 2048 // threads
    wg = _threaded([lambda i=i: O.apply_granite_rope_rows(q[i * n:(i + 1) * n], k[i * n:(i + 1) * n], i * n)
                    for i in range(threads)], 1)
    qb = O.to_bits16(g.standard_normal((8192, 4096), dtype=np.float32), O.BF16)
    kb = O.to_bits16(g.standard_normal((8192, 512), dtype=np.float32), O.BF16)
    ones = np.ones(128, np.float32)
    tq, nq = _timed_loop(lambda: O.qwen_qk_norm_rope_rows(qb[:256], kb[:256], ones, ones, 0, O.BF16), secs / 4)
    m = 8192 // threads
    wq = _threaded([lambda i=i: O.qwen_qk_norm_rope_rows(qb[i * m:(i + 1) * m], kb[i * m:(i + 1) * m], ones, ones,
                                                         i * m, O.BF16) for i in range(threads)], 1)
    return {"cfg3": _entry(tg * 8 * 1e6, "us/prompt", f"{ng} runs of 256 rows (qxo_apply_granite_rope_rows), x8",
                           wg * 2048 / (n * threads) * 1e6, threads,
                           f"{n * threads} of 2048 rows over {threads} threads, scaled to 2048"),
            "cfg5b": _entry(tq * 32 * 1e6, "us/prompt", f"{nq} runs of 256 bf16 rows (qxo_qwen_qk_norm_rope_rows), "
                            f"x32", wq * 8192 / (m * threads) * 1e6, threads,
                            f"{m * threads} of 8192 rows over {threads} threads, scaled to 8192")}


def cpu_sweep(O, np, threads, secs):
    """granite_attend of one fp32 layer at the sweep's contexts (1 thread)."""
    g = np.random.default_rng(9)
    out = {}
    for L in (32, 64, 128, 256, 512):
        c = O.KvCache(L)
        c.extend(g.standard_normal((L, 8, 64), dtype=np.float32), g.standard_normal((L, 8, 64), dtype=np.float32))
        q = g.standard_normal(1024, dtype=np.float32)
        t, n = _timed_loop(lambda: O.granite_attend(q, c, L), secs / 5, 16)
        out[f"fp32_ctx{L}"] = round(t * 1e6, 2)
    return {"value": out, "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": "single-thread granite_attend (fp32 K/V) per context, repeated for ~0.4 s each"}


def cpu_kv_hash(O, np, threads, secs):
    """kv_leaf_hash_v1 of fp16 Granite token rows (1 KiB K + 1 KiB V), a C loop."""
    R = 2048
    g = np.random.default_rng(7)
    keys = g.integers(0, 256, (R, 1024), dtype=np.uint8)
    vals = g.integers(0, 256, (R, 1024), dtype=np.uint8)
    t1, n = _timed_loop(lambda: O.kv_leaf_hashes(0, 0, keys, vals), secs)
    reps = max(1, n // 2)
    wall = _threaded([lambda: O.kv_leaf_hashes(0, 0, keys, vals)] * threads, reps)
    return _entry(R / t1, "leaves/s", f"{n} C loops over {R} leaves (qxo_kv_leaf_hashes)",
                  R * reps * threads / wall, threads, f"{threads} threads x {reps} loops of {R} leaves")


def cpu_baselines(names=None, secs=2.0):
    import numpy as np

    from oracle import oracle as O

    threads, affinity, nproc = cpu_threads()
    fns = {"cfg1": cpu_cfg1, "cfg2": cpu_cfg2, "cfg3": cpu_cfg3, "cfg4": cpu_cfg4, "cfg5a": cpu_cfg5a,
           "cfg5b": cpu_cfg5b, "kvhash": cpu_kv_hash, "frontend": cpu_frontends, "sweep": cpu_sweep}
    out = {}
    for name, fn in fns.items():
        if names and name not in names:
            continue
        try:
            t0 = time.perf_counter()
            out[name] = fn(O, np, threads, secs)
            out[name]["host"] = {"nproc": nproc, "affinity": affinity}
            log(f"cpu {name}", json.dumps(out[name]), f"({time.perf_counter() - t0:.1f} s)")
        except Exception as e:  # report, keep the rest
            out[name] = {"error": str(e)}
            log(f"cpu {name} error", e)
    return out


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
                         ("kvhash", bench_kv_hash), ("tieredv", bench_tiered_v), ("sweep", bench_attention_sweep),
                         ("prefill_fp32", bench_prefill_fp32)):
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
    wanted = (set(only) | {"cfg4"} | ({"frontend"} if only & {"cfg3", "cfg5b"} else set())) if only else None
    cpu = {} if args.no_cpu else cpu_baselines(wanted)
    for name, entry in cpu.items():
        if name in detail and isinstance(detail[name], dict) and "error" not in detail[name]:
            detail[name]["cpu_baseline"] = entry
    for name, entry in (cpu.get("frontend") or {}).items():
        fe = detail.get(name, {}).get("frontend") if isinstance(detail.get(name), dict) else None
        if isinstance(fe, dict) and isinstance(entry, dict):
            fe["cpu_baseline"] = entry
    headline_cpu = None
    if "cfg4" in cpu:
        headline_cpu = dict(cpu["cfg4"])
        if "kvhash" in cpu:
            headline_cpu["kv_hash"] = cpu["kvhash"]
    if head is None:
        print(json.dumps({"detail": detail, "cpu_baseline": headline_cpu}))
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
        "cpu_baseline": headline_cpu,
        "detail": {"cfg4": {k: v for k, v in head.items() if k != "roofline"}, **detail},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
