"""Host-side mirror of the reference's attention interface over libqx_hip.

The objects follow `qx_metal::platform` (MetalContext, DecodeGraph) and the
V1 runtime (`KvCache`, `granite_attention_decode`,
crates/qx-runtime/src/lib.rs:349-452) with the same argument meaning and
error behaviour: invalid requests raise QxhError carrying the library's
message, the analogue of `Err(String)`.

torch supplies device memory and the stream; every computation runs in the
HIP kernels of libqx_hip.so.
"""
from __future__ import annotations

import ctypes

import torch

from . import abi
from .abi import BF16, F16, F32, SHAPE_GRANITE, SHAPE_QWEN3, check, lib

_TORCH_DTYPE = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}
_QXH_DTYPE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


def qxh_dtype(t: torch.Tensor) -> int:
    try:
        return _QXH_DTYPE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def torch_dtype(code: int):
    return _TORCH_DTYPE[code]


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must live on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def shape_info(shape: int) -> abi.ShapeInfo:
    info = abi.ShapeInfo()
    check(lib().qxh_shape_query(shape, ctypes.byref(info)))
    return info


class Context:
    """platform::MetalContext counterpart: device binding, stream, metrics."""

    def __init__(self, device: int = 0):
        self.device = device
        h = ctypes.c_void_p()
        check(lib().qxh_context_create(device, ctypes.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def metrics(self) -> abi.Metrics:
        m = abi.Metrics()
        check(lib().qxh_context_metrics(self._h, ctypes.byref(m)))
        return m

    def close(self):
        if getattr(self, "_h", None):
            lib().qxh_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Graph:
    """DecodeGraph counterpart: ordered work on one stream (torch's current
    stream by default), finished with GPU time.  Usable as a context manager,
    which finishes (submit + wait) on exit."""

    def __init__(self, ctx: Context, stream=None):
        if stream is None:
            stream = torch.cuda.current_stream(ctx.device)
        self.stream = stream
        h = ctypes.c_void_p()
        check(lib().qxh_graph_begin(ctx.handle, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(h)))
        self._h = h
        self.metrics = None

    @property
    def handle(self):
        if self._h is None:
            raise RuntimeError("graph already finished")
        return self._h

    def finish(self) -> abi.GraphMetrics:
        m = abi.GraphMetrics()
        h, self._h = self._h, None
        check(lib().qxh_graph_finish(h, ctypes.byref(m)))
        self.metrics = m
        return m

    def discard(self):
        if self._h is not None:
            lib().qxh_graph_discard(self._h)
            self._h = None

    def capture_begin(self):
        check(lib().qxh_graph_capture_begin(self.handle))

    def capture_end(self) -> "Replay":
        r = ctypes.c_void_p()
        check(lib().qxh_graph_capture_end(self.handle, ctypes.byref(r)))
        return Replay(r)

    def __enter__(self):
        return self

    def __exit__(self, et, ev, tb):
        if et is None:
            self.finish()
        else:
            self.discard()
        return False


class Replay:
    """An instantiated HIP graph of captured encoders."""

    def __init__(self, h):
        self._h = h

    def launch(self, stream=None):
        stream = stream or torch.cuda.current_stream()
        check(lib().qxh_replay_launch(self._h, ctypes.c_void_p(stream.cuda_stream)))

    def __del__(self):
        # at interpreter shutdown the module globals may already be gone
        if getattr(self, "_h", None) and lib is not None:
            try:
                lib().qxh_replay_destroy(self._h)
            except Exception:
                pass
            self._h = None


class KvArena:
    """Head-major KV arena with per-(layer, sequence) cursors (KvCache and the
    GpuRuntimeBuffers KV views of the reference).  The arena memory is a torch
    uint8 tensor handed to the library, so torch's allocator owns it."""

    def __init__(self, ctx: Context, shape: int, layers: int = 1, sequences: int = 1, capacity: int = 512,
                 key_dtype: int = F32, value_dtype: int | None = None, value_window: int = 0):
        self.ctx = ctx
        self.desc = abi.KvDesc(shape, key_dtype, key_dtype if value_dtype is None else value_dtype, layers,
                               sequences, capacity, value_window)
        nbytes = ctypes.c_uint64()
        check(lib().qxh_kv_cache_bytes(ctypes.byref(self.desc), ctypes.byref(nbytes)))
        self.arena = torch.empty(nbytes.value + 256, dtype=torch.uint8, device=f"cuda:{ctx.device}")
        base = self.arena.data_ptr()
        aligned = (base + 255) & ~255
        h = ctypes.c_void_p()
        check(lib().qxh_kv_cache_create(ctx.handle, ctypes.byref(self.desc), ctypes.c_void_p(aligned),
                                        nbytes.value, ctypes.byref(h)))
        self._h = h
        self.info = shape_info(shape)
        self.layout = abi.KvLayout()
        check(lib().qxh_kv_cache_layout(self._h, ctypes.byref(self.layout)))

    @property
    def handle(self):
        return self._h

    @property
    def key_dtype(self):
        return self.desc.key_dtype

    @property
    def value_dtype(self):
        return self.desc.value_dtype

    def len(self, layer: int = 0, sequence: int = 0) -> int:
        n = ctypes.c_uint32()
        check(lib().qxh_kv_cache_len(self._h, layer, sequence, ctypes.byref(n)))
        return n.value

    def reset(self):
        check(lib().qxh_kv_cache_reset(self._h))

    def rollback(self, sequence: int, length: int):
        check(lib().qxh_kv_cache_rollback(self._h, sequence, length))

    def set_len(self, length: int, sequence: int = 0xFFFFFFFF):
        check(lib().qxh_kv_cache_set_len(self._h, sequence, length))

    def value_tier(self, layer: int = 0, sequence: int = 0) -> int:
        """Tiered values: positions below this boundary are INT8."""
        n = ctypes.c_uint32()
        check(lib().qxh_kv_cache_value_tier(self._h, layer, sequence, ctypes.byref(n)))
        return n.value

    def gather(self, graph: Graph, layer: int, sequence: int, begin: int, count: int):
        """Position-major token rows [count][kv_heads][head_dim] in the cache
        dtypes; tiered values come back as float32."""
        kvh, d = self.info.kv_heads, self.info.head_dim
        dev = f"cuda:{self.ctx.device}"
        k = torch.empty((count, kvh, d), dtype=torch_dtype(self.key_dtype), device=dev)
        vdt = F32 if self.value_dtype == abi.I8_TIERED else self.value_dtype
        v = torch.empty((count, kvh, d), dtype=torch_dtype(vdt), device=dev)
        check(lib().qxh_encode_kv_gather_token_rows(graph.handle, self._h, layer, sequence, begin, count,
                                                    _ptr(k), _ptr(v)))
        return k, v

    def leaf_hashes(self, graph: Graph, layer: int, begin: int, count: int, first_sequence: int = 0,
                    sequences: int = 1, out=None):
        """kv_leaf_hash_v1 digests of token rows [begin, begin + count) of each
        sequence: uint8 [sequences][count][32] on the device."""
        if out is None:
            out = torch.empty((sequences, count, 32), dtype=torch.uint8, device=f"cuda:{self.ctx.device}")
        check(lib().qxh_encode_kv_leaf_hashes(graph.handle, self._h, layer, first_sequence, sequences, begin, count,
                                              _ptr(out), out.numel()))
        return out

    def verification_hashes(self, graph: Graph, residual_snapshots, residual_stride: int, token: int, layers: int,
                            checkpoint_interval: int, sequence: int = 0, out=None):
        """Per-token digests (state root, KV leaf) for p = 0..layers: uint8 [layers + 1][64]."""
        if out is None:
            out = torch.empty((layers + 1, 64), dtype=torch.uint8, device=f"cuda:{self.ctx.device}")
        rb = residual_snapshots.numel() * residual_snapshots.element_size()
        check(lib().qxh_encode_verification_hashes(graph.handle, self._h, sequence, _ptr(residual_snapshots), rb,
                                                   residual_stride, token, layers, checkpoint_interval, _ptr(out),
                                                   out.numel()))
        return out

    def fill_normal(self, graph: Graph, seed: int, length: int):
        check(lib().qxh_encode_kv_fill_normal(graph.handle, self._h, seed, length))

    def close(self):
        if getattr(self, "_h", None):
            lib().qxh_kv_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- encoders -----------------------------------------------------------------

def rope_kv_batch(graph: Graph, cache: KvArena, layer: int, start_position: int, query, key, value,
                  query_out=None, first_sequence: int = 0, query_norm=None, key_norm=None):
    """Fused RoPE (+ Qwen per-head RMSNorm) and KV append.

    key/value: [sequences][tokens][kv_heads][d]; query/query_out:
    [sequences][tokens][q_heads][d] (query_out may be None)."""
    kvh, d = cache.info.kv_heads, cache.info.head_dim
    seqs, tokens = key.shape[0], key.shape[1]
    if key.shape[2:] != (kvh, d) or value.shape != key.shape:
        raise ValueError(f"key/value must be [S][T][{kvh}][{d}], got {tuple(key.shape)} / {tuple(value.shape)}")
    if query is not None and query.shape != (seqs, tokens, cache.info.q_heads, d):
        raise ValueError(f"query must be [S][T][{cache.info.q_heads}][{d}], got {tuple(query.shape)}")
    if query_out is not None and query_out.shape != (seqs, tokens, cache.info.q_heads, d):
        raise ValueError("query_out shape mismatch")
    dt = qxh_dtype(key)
    if value.dtype != key.dtype or (query is not None and query.dtype != key.dtype):
        raise TypeError("query, key and value must share a dtype")
    check(lib().qxh_encode_rope_kv_batch(
        graph.handle, cache.handle, layer, first_sequence, seqs, start_position, tokens, _ptr(query), _ptr(key),
        _ptr(value), dt, _ptr(query_norm), _ptr(key_norm), _ptr(query_out),
        qxh_dtype(query_out) if query_out is not None else dt))


def store_kv(graph: Graph, cache: KvArena, layer: int, start_position: int, key, value, first_sequence: int = 0):
    seqs, tokens = key.shape[0], key.shape[1]
    check(lib().qxh_encode_store_kv(graph.handle, cache.handle, layer, first_sequence, seqs, start_position, tokens,
                                    _ptr(key), _ptr(value), qxh_dtype(key)))


def qwen_qk_norm_rope(graph: Graph, query, key, position: int, query_norm=None, key_norm=None):
    """In-place encode_qwen_qk_norm_rope on q [32*128] and k [4*128]."""
    if query.numel() != 4096 or key.numel() != 512:
        raise ValueError("Qwen q/k buffers are smaller than their fixed shape")
    check(lib().qxh_encode_qwen_qk_norm_rope(graph.handle, _ptr(query), _ptr(key), _ptr(query_norm),
                                             _ptr(key_norm), qxh_dtype(query), position))


def attention_workspace_bytes(cache: KvArena, sequences: int, length: int) -> int:
    n = ctypes.c_uint64()
    check(lib().qxh_attention_workspace_bytes(cache.handle, sequences, length, ctypes.byref(n)))
    return n.value


def decode_step(graph: Graph, cache: KvArena, layer: int, position: int, query, key, value, query_out=None,
                out=None, out_dtype=None, workspace=None):
    """RoPE + append + attention of one Granite token (fp32 q [16][64], k/v [8][64])
    for sequence 0 over positions [0, position]; returns out [16][64]."""
    if out is None:
        out = torch.empty((cache.info.q_heads, cache.info.head_dim), dtype=out_dtype or torch.float32,
                          device=query.device)
    ws_bytes = 0
    if workspace is None and (position + 1 > 1024 or cache.value_dtype == abi.I8_TIERED):  # the two-call path
        need = attention_workspace_bytes(cache, 1, position + 1)
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=query.device) if need else None
    if workspace is not None:
        ws_bytes = workspace.numel() * workspace.element_size()
    check(lib().qxh_encode_decode_step_for_layer(graph.handle, cache.handle, _ptr(query), _ptr(key), _ptr(value),
                                                 _ptr(query_out), layer, position, _ptr(out), qxh_dtype(out),
                                                 _ptr(workspace), ws_bytes))
    return out


def attention(graph: Graph, cache: KvArena, layer: int, query, length: int, out=None, out_dtype=None,
              workspace=None, first_sequence: int = 0):
    """Decode attention of one query token per sequence over positions [0, length).

    query: [sequences][q_heads][d]; returns out of the same shape."""
    seqs = query.shape[0]
    if query.shape[1:] != (cache.info.q_heads, cache.info.head_dim):
        raise ValueError(f"query must be [S][{cache.info.q_heads}][{cache.info.head_dim}]")
    if out is None:
        out = torch.empty(query.shape, dtype=out_dtype or query.dtype, device=query.device)
    need = attention_workspace_bytes(cache, seqs, length)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().qxh_encode_attention_for_layer(graph.handle, cache.handle, layer, first_sequence, seqs, length,
                                               _ptr(query), qxh_dtype(query), _ptr(out), qxh_dtype(out),
                                               _ptr(workspace), ws_bytes))
    return out


def attention_no_alloc(graph: Graph, cache: KvArena, layer: int, query, length: int, out, first_sequence: int = 0):
    """Decode attention through qxh_encode_attention_for_layer_no_alloc: the
    split partials live in the library's per-GPU device scratch, so the call
    allocates nothing (out must be given)."""
    seqs = query.shape[0]
    if query.shape[1:] != (cache.info.q_heads, cache.info.head_dim):
        raise ValueError(f"query must be [S][{cache.info.q_heads}][{cache.info.head_dim}]")
    check(lib().qxh_encode_attention_for_layer_no_alloc(graph.handle, cache.handle, layer, first_sequence, seqs,
                                                        length, _ptr(query), qxh_dtype(query), _ptr(out),
                                                        qxh_dtype(out)))
    return out


def prefill_workspace_bytes(cache: KvArena, tokens: int) -> int:
    n = ctypes.c_uint64()
    check(lib().qxh_prefill_workspace_bytes(cache.handle, tokens, ctypes.byref(n)))
    return n.value


def prefill_attention(graph: Graph, cache: KvArena, layer: int, start_position: int, query, out=None, out_dtype=None,
                      sequence: int = 0, workspace=None):
    """Causal prefill: query [tokens][q_heads][d]; row t attends [0, start+t]."""
    tokens = query.shape[0]
    if out is None:
        out = torch.empty(query.shape, dtype=out_dtype or query.dtype, device=query.device)
    need = prefill_workspace_bytes(cache, tokens)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=query.device)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().qxh_encode_prefill_attention(graph.handle, cache.handle, layer, sequence, start_position, tokens,
                                             _ptr(query), qxh_dtype(query), _ptr(out), qxh_dtype(out),
                                             _ptr(workspace), ws_bytes))
    return out


def fill_normal(graph: Graph, tensor, seed: int, stddev: float = 1.0):
    check(lib().qxh_encode_fill_normal(graph.handle, _ptr(tensor), qxh_dtype(tensor), tensor.numel(), seed, stddev))
    return tensor


def granite_block_workspace_bytes(cache: KvArena, length: int) -> int:
    n = ctypes.c_uint64()
    check(lib().qxh_granite_block_workspace_bytes(cache.handle, length, ctypes.byref(n)))
    return n.value


class GraniteLayer:
    """fp32 weights of one Granite attention block (device tensors)."""

    def __init__(self, input_norm, q_proj, k_proj, v_proj, o_proj):
        self.tensors = (input_norm, q_proj, k_proj, v_proj, o_proj)
        self.struct = abi.GraniteLayerWeights(*[t.data_ptr() for t in self.tensors])


def granite_attention_block(graph: Graph, cache: KvArena, layer: int, position: int, weights: GraniteLayer,
                            hidden_in, hidden_out, workspace):
    check(lib().qxh_encode_granite_attention_block(
        graph.handle, cache.handle, layer, position, ctypes.byref(weights.struct), _ptr(hidden_in),
        _ptr(hidden_out), _ptr(workspace), workspace.numel()))


class Q4Matrix:
    """A group-32 Q4 matrix on the device in qx-quant's RowMajor layout
    (crates/qx-quant/src/lib.rs:313-360): `packed` uint8 [rows, cols/2] and
    `scales` f16 bit patterns [rows, cols/32] (int16 or uint8 tensors)."""

    def __init__(self, packed, scales, rows: int, cols: int):
        self.tensors = (packed, scales)
        self.rows, self.cols = rows, cols
        self.struct = abi.Q4Matrix(packed.data_ptr(), scales.data_ptr(), rows, cols)


def q4_gemv(graph: Graph, matrix: Q4Matrix, vector, out=None, multiplier: float = 1.0):
    """encode_prepared_q4_dense_simd_scaled (crates/qx-metal/src/lib.rs:2655-2736):
    out = (matrix . vector) * multiplier in mat_vec_simd32's order."""
    if out is None:
        out = torch.empty(matrix.rows, dtype=torch.float32, device=vector.device)
    check(lib().qxh_encode_q4_gemv(graph.handle, ctypes.byref(matrix.struct), _ptr(vector), _ptr(out),
                                   float(multiplier)))
    return out


def rms_inverse(graph: Graph, vector, out=None):
    """encode_rmsnorm_scalar (crates/qx-metal/src/lib.rs:7777-7810): the inverse
    RMS of a 1024-wide fp32 vector in rms_norm_simd's order."""
    if out is None:
        out = torch.empty(1, dtype=torch.float32, device=vector.device)
    check(lib().qxh_encode_rms_inverse(graph.handle, _ptr(vector), _ptr(out)))
    return out


class GraniteQ4Layer:
    """Q4 weights of one Granite attention block: fp32 input norm [1024] and
    Q4Matrix q (1024x1024), k, v (512x1024), o (1024x1024)."""

    def __init__(self, input_norm, q_proj: Q4Matrix, k_proj: Q4Matrix, v_proj: Q4Matrix, o_proj: Q4Matrix):
        self.tensors = (input_norm, q_proj, k_proj, v_proj, o_proj)
        self.struct = abi.GraniteQ4LayerWeights(input_norm.data_ptr(), q_proj.struct, k_proj.struct, v_proj.struct,
                                                o_proj.struct)


def granite_attention_block_q4(graph: Graph, cache: KvArena, layer: int, position: int, weights: GraniteQ4Layer,
                               hidden_in, hidden_out, workspace, inverse_rms=None):
    """The Q4 attention half of encode_attention_layer_with_plan
    (crates/qx-runtime-v2/src/lib.rs:6890-6994)."""
    check(lib().qxh_encode_granite_attention_block_q4(
        graph.handle, cache.handle, layer, position, ctypes.byref(weights.struct), _ptr(hidden_in),
        _ptr(hidden_out), None if inverse_rms is None else _ptr(inverse_rms), _ptr(workspace), workspace.numel()))


def hbm_read_probe(graph: Graph, data, sink, blocks: int = 0):
    """One plain streaming read of `data` (the bench's achievable-HBM probe)."""
    check(lib().qxh_encode_hbm_read_probe(graph.handle, _ptr(data), data.numel() * data.element_size(), _ptr(sink),
                                          blocks))


def hbm_copy_probe(graph: Graph, src, dst, nontemporal: bool = True):
    """One plain copy of `src` into `dst` (the bench's one-shot read + write floor)."""
    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() < n:
        raise ValueError("hbm_copy_probe: destination smaller than the source")
    check(lib().qxh_encode_hbm_copy_probe(graph.handle, _ptr(src), _ptr(dst), n, 1 if nontemporal else 0))


class QwenQ4Layer:
    """Q4 weights of one Qwen attention half: fp32 input norm [2048], Q4Matrix
    q (4096x2048), k, v (512x2048), fp32 q/k head norms [128], Q4Matrix o
    (2048x4096), fp32 post-attention norm [2048]."""

    def __init__(self, input_norm, q_proj: Q4Matrix, k_proj: Q4Matrix, v_proj: Q4Matrix, query_norm, key_norm,
                 o_proj: Q4Matrix, post_attention_norm):
        self.tensors = (input_norm, q_proj, k_proj, v_proj, query_norm, key_norm, o_proj, post_attention_norm)
        self.struct = abi.QwenQ4LayerWeights(input_norm.data_ptr(), q_proj.struct, k_proj.struct, v_proj.struct,
                                             query_norm.data_ptr(), key_norm.data_ptr(), o_proj.struct,
                                             post_attention_norm.data_ptr())


def qwen_block_workspace_bytes(cache: KvArena, length: int) -> int:
    n = ctypes.c_uint64()
    check(lib().qxh_qwen_block_workspace_bytes(cache.handle, length, ctypes.byref(n)))
    return n.value


def qwen_attention_block(graph: Graph, cache: KvArena, layer: int, position: int, weights: QwenQ4Layer, hidden,
                         hidden_after, moe_input, workspace):
    """The attention half of PreparedQwenLayer::encode_with_expert_cache
    (crates/qx-runtime-v2/src/lib.rs:904-973); f16 hidden in, f16
    hidden_after_attention and moe_input out."""
    check(lib().qxh_encode_qwen_attention_block(
        graph.handle, cache.handle, layer, position, ctypes.byref(weights.struct), _ptr(hidden), _ptr(hidden_after),
        _ptr(moe_input), _ptr(workspace), workspace.numel()))


def consensus_conformance(graph: Graph, inputs, coords):
    n = inputs.numel()
    outs = [torch.empty(n, dtype=torch.int32, device=inputs.device) for _ in range(4)]
    check(lib().qxh_encode_consensus_conformance(graph.handle, _ptr(inputs), _ptr(coords), n,
                                                 *[_ptr(o) for o in outs]))
    return outs
