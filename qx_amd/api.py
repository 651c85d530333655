"""Reference-shaped entry points running on the HIP path.

These keep the names, argument meaning and error behaviour of the reference
functions they replace, so callers (and parity tests) read like the
reference's own:

  KvCache / granite_attention_decode / apply_granite_rope
      crates/qx-runtime/src/lib.rs:349-452 (V1 runtime API)
  run_qwen_qk_norm_rope / run_qwen_gqa_attention
      crates/qx-metal/src/lib.rs:14373-14599 (synchronous Qwen helpers:
      host 16-bit arrays in, host arrays out, position-major KV rows)

Inputs/outputs are host numpy arrays (or anything numpy accepts); the work is
enqueued on the GPU through libqx_hip and waited on before returning.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import runtime as rt
from .abi import BF16, F16, F32, SHAPE_GRANITE, SHAPE_QWEN3, QxhError, check, lib

_ctx = None


def context() -> rt.Context:
    global _ctx
    if _ctx is None:
        _ctx = rt.Context(0)
    return _ctx


def _dev(a, dtype=torch.float32):
    return torch.as_tensor(np.ascontiguousarray(a)).to(device="cuda:0", dtype=dtype).contiguous()


class KvCache:
    """KvCache (crates/qx-runtime/src/lib.rs:349-431): one Granite layer's
    cache of `max_context` positions, here resident in HBM (head-major)."""

    def __init__(self, max_context: int, key_dtype: int = F32, value_dtype: int | None = None):
        self.arena = rt.KvArena(context(), SHAPE_GRANITE, 1, 1, max_context, key_dtype, value_dtype)
        self.max_context = max_context
        self._ws = None

    def __len__(self):
        return self.arena.len(0, 0)

    def is_empty(self):
        return len(self) == 0

    def reset(self):
        self.arena.reset()

    def token_rows(self, begin: int = 0, count: int | None = None):
        """Position-major K/V rows as float32 numpy ([n][8][64])."""
        n = len(self) - begin if count is None else count
        with rt.Graph(context()) as g:
            k, v = self.arena.gather(g, 0, 0, begin, n)
        return k.float().cpu().numpy(), v.float().cpu().numpy()


def apply_granite_rope(query, key, position: int):
    """apply_granite_rope (lib.rs:434-441) on the GPU; returns rotated copies.
    Runs the fused kernel against a scratch cache and reads K back."""
    cache = KvCache(position + 1)
    cache.arena.set_len(position)
    q = _dev(query).reshape(1, 1, 16, 64)
    k = _dev(key).reshape(1, 1, 8, 64)
    qo = torch.empty_like(q)
    with rt.Graph(context()) as g:
        rt.rope_kv_batch(g, cache.arena, 0, position, q, k, torch.zeros_like(k), query_out=qo)
    krot, _ = cache.token_rows(position, 1)
    return qo.reshape(-1).cpu().numpy(), krot.reshape(-1)


def granite_attention_decode(query, key, value, position: int, cache: KvCache):
    """granite_attention_decode (lib.rs:444-452): RoPE q and k, append the
    rotated key and raw value at `position` (which must equal the cache
    length), attend over the cache.  Returns the [1024] output."""
    q = _dev(query).reshape(16, 64)
    k = _dev(key).reshape(8, 64)
    v = _dev(value).reshape(8, 64)
    qo = torch.empty_like(q)
    with rt.Graph(context()) as g:
        out = rt.decode_step(g, cache.arena, 0, position, q, k, v, query_out=qo)
    return out.reshape(-1).cpu().numpy()


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _np_ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def run_qwen_qk_norm_rope(query_bits, key_bits, query_norm, key_norm, position: int, fmt: int = F16):
    """MetalContext::run_qwen_qk_norm_rope (crates/qx-metal/src/lib.rs:14373-14483),
    through the C ABI's synchronous qxh_run_qwen_qk_norm_rope."""
    q, k, qn, kn = _u16(query_bits), _u16(key_bits), _f32c(query_norm), _f32c(key_norm)
    qo, ko = np.empty_like(q), np.empty_like(k)
    check(lib().qxh_run_qwen_qk_norm_rope(context().handle, _np_ptr(q), q.size, _np_ptr(k), k.size, _np_ptr(qn),
                                          qn.size, _np_ptr(kn), kn.size, fmt, position, _np_ptr(qo), _np_ptr(ko)))
    return qo, ko


def run_qwen_gqa_attention(query_bits, key_cache_bits, value_cache_bits, fmt: int = F16):
    """MetalContext::run_qwen_gqa_attention (crates/qx-metal/src/lib.rs:14488-14599),
    through the C ABI's synchronous qxh_run_qwen_gqa_attention: q [4096],
    position-major caches [ctx][4][128] (16-bit), output [4096]."""
    q, kc, vc = _u16(query_bits), _u16(key_cache_bits), _u16(value_cache_bits)
    out = np.empty(4096, np.uint16)
    check(lib().qxh_run_qwen_gqa_attention(context().handle, _np_ptr(q), q.size, _np_ptr(kc), kc.size, _np_ptr(vc),
                                           vc.size, fmt, _np_ptr(out)))
    return out
