"""ctypes bindings of include/qx_hip.h (libqx_hip.so).

Loading fails loudly when the library has not been built: there is no CPU
fallback behind these bindings.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqx_hip.so")

QXH_OK = 0
QXH_ERR_INVALID_ARGUMENT = 1
QXH_ERR_KV_POSITION = 2
QXH_ERR_HIP = 3
QXH_ERR_UNSUPPORTED = 4
QXH_ERR_NO_DEVICE = 5

F32, F16, BF16 = 0, 1, 2
I8_TIERED = 3  # value dtype only: f16 window + INT8 blocks of 32 with f16 scales
SHAPE_GRANITE, SHAPE_QWEN3 = 0, 1

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_uint32 = ctypes.c_uint32
c_uint64 = ctypes.c_uint64
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t
P = ctypes.POINTER


class ShapeInfo(ctypes.Structure):
    _fields_ = [("q_heads", c_uint32), ("kv_heads", c_uint32), ("head_dim", c_uint32), ("hidden", c_uint32),
                ("scale", c_float), ("rope_theta", c_float), ("rms_epsilon", c_float), ("qk_norm", c_uint32)]


class Metrics(ctypes.Structure):
    _fields_ = [("graphs", c_uint64), ("dispatches", c_uint64), ("gpu_ms", ctypes.c_double)]


class GraphMetrics(ctypes.Structure):
    _fields_ = [("dispatches", c_uint32), ("gpu_ms", c_float)]


class BufferView(ctypes.Structure):
    _fields_ = [("buffer", c_void_p), ("offset", c_uint64), ("length", c_uint64)]


class KvDesc(ctypes.Structure):
    _fields_ = [("shape", c_int32), ("key_dtype", c_int32), ("value_dtype", c_int32), ("layers", c_uint32),
                ("sequences", c_uint32), ("capacity", c_uint32), ("value_window", c_uint32)]


class KvLayout(ctypes.Structure):
    _fields_ = [("keys", c_void_p), ("values", c_void_p), ("head_stride", c_uint64), ("sequence_stride", c_uint64),
                ("layer_stride", c_uint64), ("key_elem_bytes", c_uint32), ("value_elem_bytes", c_uint32),
                ("value_scales", c_void_p), ("value_ring", c_void_p), ("value_window", c_uint32)]


class GraniteLayerWeights(ctypes.Structure):
    _fields_ = [("input_norm", c_void_p), ("q_proj", c_void_p), ("k_proj", c_void_p), ("v_proj", c_void_p),
                ("o_proj", c_void_p)]


class Q4Matrix(ctypes.Structure):
    _fields_ = [("packed", c_void_p), ("scales", c_void_p), ("rows", c_uint32), ("cols", c_uint32)]


class GraniteQ4LayerWeights(ctypes.Structure):
    _fields_ = [("input_norm", c_void_p), ("q_proj", Q4Matrix), ("k_proj", Q4Matrix), ("v_proj", Q4Matrix),
                ("o_proj", Q4Matrix)]


class QwenQ4LayerWeights(ctypes.Structure):
    _fields_ = [("input_norm", c_void_p), ("q_proj", Q4Matrix), ("k_proj", Q4Matrix), ("v_proj", Q4Matrix),
                ("query_norm", c_void_p), ("key_norm", c_void_p), ("o_proj", Q4Matrix),
                ("post_attention_norm", c_void_p)]


# name -> (restype, argtypes); must cover every function of include/qx_hip.h
SIGNATURES = {
    "qxh_abi_version": (c_int32, []),
    "qxh_last_error": (c_size_t, [ctypes.c_char_p, c_size_t]),
    "qxh_shape_query": (c_int32, [c_int32, P(ShapeInfo)]),
    "qxh_context_create": (c_int32, [c_int32, P(c_void_p)]),
    "qxh_context_destroy": (c_int32, [c_void_p]),
    "qxh_context_metrics": (c_int32, [c_void_p, P(Metrics)]),
    "qxh_context_stream": (c_int32, [c_void_p, P(c_void_p)]),
    "qxh_graph_begin": (c_int32, [c_void_p, c_void_p, P(c_void_p)]),
    "qxh_graph_submit": (c_int32, [c_void_p]),
    "qxh_graph_wait": (c_int32, [c_void_p, P(GraphMetrics)]),
    "qxh_graph_finish": (c_int32, [c_void_p, P(GraphMetrics)]),
    "qxh_graph_discard": (c_int32, [c_void_p]),
    "qxh_graph_capture_begin": (c_int32, [c_void_p]),
    "qxh_graph_capture_end": (c_int32, [c_void_p, P(c_void_p)]),
    "qxh_replay_launch": (c_int32, [c_void_p, c_void_p]),
    "qxh_replay_destroy": (c_int32, [c_void_p]),
    "qxh_buffer_alloc": (c_int32, [c_void_p, c_uint64, P(BufferView)]),
    "qxh_buffer_free": (c_int32, [c_void_p]),
    "qxh_buffer_subregion": (c_int32, [BufferView, c_uint64, c_uint64, P(BufferView)]),
    "qxh_buffer_device_ptr": (c_int32, [BufferView, P(c_void_p)]),
    "qxh_buffer_write": (c_int32, [BufferView, c_void_p, c_uint64]),
    "qxh_buffer_read": (c_int32, [BufferView, c_void_p, c_uint64]),
    "qxh_kv_cache_bytes": (c_int32, [P(KvDesc), P(c_uint64)]),
    "qxh_kv_cache_create": (c_int32, [c_void_p, P(KvDesc), c_void_p, c_uint64, P(c_void_p)]),
    "qxh_kv_cache_destroy": (c_int32, [c_void_p]),
    "qxh_kv_cache_len": (c_int32, [c_void_p, c_uint32, c_uint32, P(c_uint32)]),
    "qxh_kv_cache_reset": (c_int32, [c_void_p]),
    "qxh_kv_cache_rollback": (c_int32, [c_void_p, c_uint32, c_uint32]),
    "qxh_kv_cache_set_len": (c_int32, [c_void_p, c_uint32, c_uint32]),
    "qxh_kv_cache_layout": (c_int32, [c_void_p, P(KvLayout)]),
    "qxh_kv_cache_desc": (c_int32, [c_void_p, P(KvDesc)]),
    "qxh_kv_cache_value_tier": (c_int32, [c_void_p, c_uint32, c_uint32, P(c_uint32)]),
    "qxh_encode_rope_kv_batch": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                           c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                           c_int32]),
    "qxh_encode_rope_kv_for_layer": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_uint32, c_uint32]),
    "qxh_encode_store_kv": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                      c_void_p, c_void_p, c_int32]),
    "qxh_encode_qwen_qk_norm_rope": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                               c_uint32]),
    "qxh_attention_workspace_bytes": (c_int32, [c_void_p, c_uint32, c_uint32, P(c_uint64)]),
    "qxh_encode_attention_for_layer": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32,
                                                 c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_uint64]),
    "qxh_encode_attention_for_layer_no_alloc": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                                                          c_uint32, c_void_p, c_int32, c_void_p, c_int32]),
    "qxh_prefill_workspace_bytes": (c_int32, [c_void_p, c_uint32, P(c_uint64)]),
    "qxh_encode_prefill_attention": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32,
                                               c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_uint64]),
    "qxh_encode_kv_gather_token_rows": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32,
                                                  c_void_p, c_void_p]),
    "qxh_encode_decode_step_for_layer": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                   c_uint32, c_uint32, c_void_p, c_int32, c_void_p, c_uint64]),
    "qxh_encode_kv_leaf_hashes": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                            c_void_p, c_uint64]),
    "qxh_encode_verification_hashes": (c_int32, [c_void_p, c_void_p, c_uint32, c_void_p, c_uint64, c_uint32,
                                                 c_uint32, c_uint32, c_uint32, c_void_p, c_uint64]),
    "qxh_granite_block_workspace_bytes": (c_int32, [c_void_p, c_uint32, P(c_uint64)]),
    "qxh_encode_granite_attention_block": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32,
                                                     P(GraniteLayerWeights), c_void_p, c_void_p, c_void_p,
                                                     c_uint64]),
    "qxh_encode_q4_gemv": (c_int32, [c_void_p, P(Q4Matrix), c_void_p, c_void_p, c_float]),
    "qxh_encode_rms_inverse": (c_int32, [c_void_p, c_void_p, c_void_p]),
    "qxh_encode_granite_attention_block_q4": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32,
                                                        P(GraniteQ4LayerWeights), c_void_p, c_void_p, c_void_p,
                                                        c_void_p, c_uint64]),
    "qxh_qwen_block_workspace_bytes": (c_int32, [c_void_p, c_uint32, P(c_uint64)]),
    "qxh_encode_qwen_attention_block": (c_int32, [c_void_p, c_void_p, c_uint32, c_uint32, P(QwenQ4LayerWeights),
                                                  c_void_p, c_void_p, c_void_p, c_void_p, c_uint64]),
    "qxh_run_qwen_qk_norm_rope": (c_int32, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t,
                                            c_void_p, c_size_t, c_int32, c_uint32, c_void_p, c_void_p]),
    "qxh_run_qwen_gqa_attention": (c_int32, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t,
                                             c_int32, c_void_p]),
    "qxh_encode_fill_normal": (c_int32, [c_void_p, c_void_p, c_int32, c_uint64, c_uint64, c_float]),
    "qxh_encode_hbm_read_probe": (c_int32, [c_void_p, c_void_p, c_uint64, c_void_p, c_uint32]),
    "qxh_encode_hbm_copy_probe": (c_int32, [c_void_p, c_void_p, c_void_p, c_uint64, c_int32]),
    "qxh_encode_kv_fill_normal": (c_int32, [c_void_p, c_void_p, c_uint64, c_uint32]),
    "qxh_encode_consensus_conformance": (c_int32, [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p,
                                                   c_void_p, c_void_p]),
}

_lib = None


class QxhError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[qxh error {code}] {message}")
        self.code = code


def lib():
    """Load libqx_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                              "or `python qx_amd/build.py` (there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().qxh_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int):
    if status != QXH_OK:
        raise QxhError(status, last_error())
