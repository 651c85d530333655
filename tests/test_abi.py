"""The C-ABI library loads and exports every symbol include/qx_hip.h
declares; host-only entry points behave without a GPU."""
import ctypes
import os
import re

import pytest

from qx_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qx_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*QXH_API\s+(?:int32_t|size_t)\s+(qxh_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    assert len(names) >= 30
    assert "qxh_encode_attention_for_layer" in names and "qxh_encode_rope_kv_for_layer" in names


def test_library_exports_every_declared_symbol():
    lib = abi.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_every_declared_symbol():
    assert sorted(abi.SIGNATURES) == declared_functions()


def test_abi_version_and_shapes():
    lib = abi.lib()
    assert lib.qxh_abi_version() == 2
    info = abi.ShapeInfo()
    assert lib.qxh_shape_query(abi.SHAPE_GRANITE, ctypes.byref(info)) == 0
    assert (info.q_heads, info.kv_heads, info.head_dim, info.hidden) == (16, 8, 64, 1024)
    assert info.scale == 0.015625 and info.qk_norm == 0
    assert lib.qxh_shape_query(abi.SHAPE_QWEN3, ctypes.byref(info)) == 0
    assert (info.q_heads, info.kv_heads, info.head_dim, info.hidden, info.qk_norm) == (32, 4, 128, 2048, 1)
    assert abs(info.scale - 128 ** -0.5) < 1e-7 and info.rope_theta == 1e6
    assert lib.qxh_shape_query(7, ctypes.byref(info)) == abi.QXH_ERR_INVALID_ARGUMENT
    assert "unknown shape" in abi.last_error()


@pytest.mark.parametrize("kd,vd,expected", [
    # crates/qx-runtime-v2/src/lib.rs:7212-7214: 24 layers at ctx 512
    (abi.F32, abi.F32, 50_331_648),
    (abi.F32, abi.F16, 37_748_736),
    (abi.F16, abi.F16, 25_165_824),
])
def test_kv_arena_bytes_match_reference_plan(kd, vd, expected):
    desc = abi.KvDesc(abi.SHAPE_GRANITE, kd, vd, 24, 1, 512)
    n = ctypes.c_uint64()
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    assert n.value == expected


def test_kv_arena_bytes_qwen_and_batched():
    # Qwen: 512 16-bit elements per token per K/V (crates/qx-model/src/lib.rs:365 = 49,152 per token over 48 layers)
    desc = abi.KvDesc(abi.SHAPE_QWEN3, abi.BF16, abi.BF16, 48, 1, 1)
    n = ctypes.c_uint64()
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    assert n.value == 48 * 2 * 512 * 2
    desc = abi.KvDesc(abi.SHAPE_GRANITE, abi.F16, abi.F16, 24, 256, 4096)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    assert n.value == 24 * 256 * 4096 * 8 * 64 * 2 * 2  # 2.147 GB per layer-step x 24


def test_tiered_value_arena_bytes():
    # Granite at ctx 4096 with fp32 K (docs/qx-structural-memory-2026-08-25.md:69-74:
    # "moving old V from FP16 to INT8 can save roughly another 48 MiB before
    # scale metadata"): INT8 codes are 48 MiB below the f16 values, then come
    # one f16 scale per 32 elements and the f16 window
    n = ctypes.c_uint64()
    f16v = abi.KvDesc(abi.SHAPE_GRANITE, abi.F32, abi.F16, 24, 1, 4096)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(f16v), ctypes.byref(n)) == 0
    base = n.value
    tiered = abi.KvDesc(abi.SHAPE_GRANITE, abi.F32, abi.I8_TIERED, 24, 1, 4096, 256)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(tiered), ctypes.byref(n)) == 0
    elems = 24 * 8 * 4096 * 64
    assert base - elems * 4 == 2 * elems and 2 * elems - elems == 48 << 20
    slots = 24 * 8 * 256  # window rows, each with a 4-byte position tag
    assert n.value == elems * 4 + elems + elems // 32 * 2 + slots * 64 * 2 + slots * 4
    assert base - n.value == (48 << 20) - (3 << 20) - (6 << 20) - slots * 4


@pytest.mark.parametrize("window", [48, 16, 0, 1 << 17])  # not a power of two, below 32, none, above 65536
def test_tiered_descriptors_are_validated(window):
    n = ctypes.c_uint64()
    desc = abi.KvDesc(abi.SHAPE_GRANITE, abi.F32, abi.I8_TIERED, 1, 1, 512, window)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == abi.QXH_ERR_INVALID_ARGUMENT
    assert "tiered" in abi.last_error()


def test_tiered_qwen_arena_bytes():
    # Qwen at ctx 32768 with bf16 K: 4 kv heads x 128 dims per position
    n = ctypes.c_uint64()
    desc = abi.KvDesc(abi.SHAPE_QWEN3, abi.BF16, abi.I8_TIERED, 48, 1, 32768, 1024)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    elems = 48 * 4 * 32768 * 128
    slots = 48 * 4 * 1024
    assert n.value == 2 * elems + elems + elems // 16 + slots * 128 * 2 + slots * 4


def test_value_window_needs_tiered_values():
    n = ctypes.c_uint64()
    desc = abi.KvDesc(abi.SHAPE_GRANITE, abi.F32, abi.F16, 1, 1, 512, 64)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == abi.QXH_ERR_INVALID_ARGUMENT
    assert "value_window" in abi.last_error()


def test_capacity_is_bounded():
    # one kv head's rows must fit the kernels' 32-bit buffer ranges: 2^22 positions at most
    n = ctypes.c_uint64()
    desc = abi.KvDesc(abi.SHAPE_QWEN3, abi.F32, abi.F32, 1, 1, 1 << 22)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0
    assert n.value == 2 * 4 * (1 << 22) * 128 * 4
    desc = abi.KvDesc(abi.SHAPE_QWEN3, abi.F32, abi.F32, 1, 1, (1 << 22) + 1)
    assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == abi.QXH_ERR_INVALID_ARGUMENT
    assert "capacity" in abi.last_error()


def test_invalid_descriptors_are_rejected():
    n = ctypes.c_uint64()
    for desc in (abi.KvDesc(abi.SHAPE_GRANITE, 5, 0, 1, 1, 8), abi.KvDesc(abi.SHAPE_GRANITE, 0, 0, 0, 1, 8),
                 abi.KvDesc(9, 0, 0, 1, 1, 8)):
        assert abi.lib().qxh_kv_cache_bytes(ctypes.byref(desc), ctypes.byref(n)) == abi.QXH_ERR_INVALID_ARGUMENT
    assert abi.lib().qxh_kv_cache_bytes(None, ctypes.byref(n)) == abi.QXH_ERR_INVALID_ARGUMENT


def test_null_arguments_return_errors_not_crashes():
    lib = abi.lib()
    assert lib.qxh_graph_submit(None) == abi.QXH_ERR_INVALID_ARGUMENT
    assert lib.qxh_graph_finish(None, None) == abi.QXH_ERR_INVALID_ARGUMENT
    assert lib.qxh_encode_attention_for_layer(None, None, 0, 0, 1, 1, None, 0, None, 0, None, 0) == \
        abi.QXH_ERR_INVALID_ARGUMENT
    assert "null graph" in abi.last_error()
    assert lib.qxh_kv_cache_len(None, 0, 0, None) == abi.QXH_ERR_INVALID_ARGUMENT
    assert lib.qxh_graph_discard(None) == 0 and lib.qxh_kv_cache_destroy(None) == 0


def test_last_error_truncates_and_reports_length():
    lib = abi.lib()
    lib.qxh_shape_query(42, None)
    full = lib.qxh_last_error(None, 0)
    buf = ctypes.create_string_buffer(8)
    assert lib.qxh_last_error(buf, 8) == full and len(buf.value) == 7


def test_context_without_gpu_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    assert abi.lib().qxh_context_create(0, ctypes.byref(h)) == abi.QXH_ERR_NO_DEVICE
    assert not h.value
