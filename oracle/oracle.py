"""ctypes/numpy front end of the CPU oracle (oracle/qx_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never as a product path.  Every function cites the reference source it
restates; the C file carries the line-by-line citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libqx_oracle.so")

F32, F16, BF16 = 0, 1, 2
GRANITE_Q_HEADS, GRANITE_KV_HEADS, GRANITE_HEAD_DIM, GRANITE_HIDDEN = 16, 8, 64, 1024
QWEN_Q_HEADS, QWEN_KV_HEADS, QWEN_HEAD_DIM = 32, 4, 128

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.qxo_last_error.restype = ctypes.c_char_p
        L.qxo_f32_to_f16.argtypes = [ctypes.c_float]
        L.qxo_f32_to_f16.restype = ctypes.c_uint16
        L.qxo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.qxo_f16_to_f32.restype = ctypes.c_float
        L.qxo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.qxo_f32_to_bf16.restype = ctypes.c_uint16
        L.qxo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.qxo_bf16_to_f32.restype = ctypes.c_float
        L.qxo_granite_inverse_frequency_bits.argtypes = [ctypes.c_uint32]
        L.qxo_granite_inverse_frequency_bits.restype = ctypes.c_uint32
        L.qxo_exp_f32.argtypes = [ctypes.c_float, _f32p]
        L.qxo_rsqrt_f32.argtypes = [ctypes.c_float, _f32p]
        L.qxo_sin_cos_f32.argtypes = [ctypes.c_float, _f32p, _f32p]
        L.qxo_granite_rope_sin_cos.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p]
        L.qxo_granite_rope_pair.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float,
                                            ctypes.c_float, _f32p, _f32p]
        L.qxo_apply_granite_rope.argtypes = [_f32p, _f32p, ctypes.c_uint32]
        L.qxo_kv_cache_new.argtypes = [ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
        L.qxo_kv_cache_new.restype = ctypes.c_void_p
        L.qxo_kv_cache_free.argtypes = [ctypes.c_void_p]
        L.qxo_kv_cache_free.restype = None
        L.qxo_kv_cache_len.argtypes = [ctypes.c_void_p]
        L.qxo_kv_cache_len.restype = ctypes.c_uint32
        L.qxo_kv_cache_reset.argtypes = [ctypes.c_void_p]
        L.qxo_kv_cache_reset.restype = None
        L.qxo_kv_cache_rollback.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.qxo_kv_cache_keys.argtypes = [ctypes.c_void_p]
        L.qxo_kv_cache_keys.restype = _f32p
        L.qxo_kv_cache_values.argtypes = [ctypes.c_void_p]
        L.qxo_kv_cache_values.restype = _f32p
        L.qxo_kv_cache_append.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _f32p, _f32p]
        L.qxo_kv_cache_extend.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _f32p, _f32p]
        L.qxo_granite_attend.argtypes = [_f32p, ctypes.c_void_p, ctypes.c_uint32, _f32p]
        L.qxo_granite_attention_decode.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint32,
                                                   ctypes.c_void_p, _f32p]
        L.qxo_granite_rms_norm.argtypes = [_f32p, _f32p, _f32p]
        L.qxo_dense_apply.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p]
        L.qxo_dense_apply.restype = None
        L.qxo_granite_attention_block.argtypes = [_f32p] * 6 + [ctypes.c_uint32, ctypes.c_void_p, _f32p]
        L.qxo_q4_quantize.argtypes = [_f32p, ctypes.c_uint32, ctypes.c_uint32, _u8p, _u16p]
        L.qxo_q4_dequantize.argtypes = [_u8p, _u16p, ctypes.c_uint32, ctypes.c_uint32, _f32p]
        L.qxo_q4_dequantize.restype = None
        L.qxo_q4_mat_vec_simd32.argtypes = [_u8p, _u16p, ctypes.c_uint32, ctypes.c_uint32, _f32p,
                                            ctypes.c_float, _f32p]
        L.qxo_granite_rms_norm_simd.argtypes = [_f32p] * 5
        L.qxo_q4_mat_vec.argtypes = [_u8p, _u16p, ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p]
        L.qxo_qwen_rms_norm.argtypes = [_f32p, _f32p, ctypes.c_uint32, ctypes.c_float, _f32p]
        L.qxo_qwen_rms_norm.restype = None
        L.qxo_granite_residual.argtypes = [_f32p, _f32p, _f32p]
        L.qxo_granite_residual.restype = None
        L.qxo_granite_attend_simd.argtypes = [_f32p, ctypes.c_void_p, ctypes.c_uint32, _f32p]
        L.qxo_granite_q4_attention_block.argtypes = ([_f32p, _f32p] + [_u8p, _u16p] * 4
                                                     + [ctypes.c_uint32, ctypes.c_void_p] + [_f32p] * 4)
        L.qxo_qwen_qk_norm_rope.argtypes = [_u16p, _u16p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_int,
                                            _u16p, _u16p]
        L.qxo_qwen_qk_norm_rope.restype = None
        L.qxo_qwen_qk_norm_rope_rows.argtypes = [_u16p, _u16p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_uint32,
                                                 ctypes.c_int, _u16p, _u16p]
        L.qxo_qwen_qk_norm_rope_rows.restype = None
        L.qxo_apply_granite_rope_rows.argtypes = [_f32p, _f32p, ctypes.c_uint32, ctypes.c_uint32]
        L.qxo_qwen_inverse_frequency.argtypes = [ctypes.c_uint32]
        L.qxo_qwen_inverse_frequency.restype = ctypes.c_float
        L.qxo_qwen_gqa_attention.argtypes = [_u16p, _u16p, _u16p, ctypes.c_uint32, ctypes.c_int, _u16p, _f32p]
        L.qxo_qwen_prefill_rows.argtypes = [_u16p, _u16p, _u16p, ctypes.c_uint32, _u32p, ctypes.c_uint32,
                                            ctypes.c_int, _u16p, _f32p]
        L.qxo_granite_prefill_rows.argtypes = [_f32p, ctypes.c_void_p, ctypes.c_uint32, _u32p,
                                               ctypes.c_uint32, _f32p]
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _check(status):
    if status != 0:
        raise OracleError(lib().qxo_last_error().decode())


def _p(a, ptype=_f32p):
    return a.ctypes.data_as(ptype)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --- consensus math (crates/qx-consensus-math/src/lib.rs) --------------------

def exp_f32(x: float):
    """exp_f32, lib.rs:69-110.  None where the reference returns None."""
    out = ctypes.c_float()
    return None if lib().qxo_exp_f32(float(x), ctypes.byref(out)) else out.value


def rsqrt_f32(x: float):
    """rsqrt_f32, lib.rs:113-128."""
    out = ctypes.c_float()
    return None if lib().qxo_rsqrt_f32(float(x), ctypes.byref(out)) else out.value


def sin_cos_f32(angle: float):
    """sin_cos_f32, lib.rs:147-189."""
    s, c = ctypes.c_float(), ctypes.c_float()
    return None if lib().qxo_sin_cos_f32(float(angle), ctypes.byref(s), ctypes.byref(c)) else (s.value, c.value)


def granite_rope_sin_cos(position: int, pair: int):
    """granite_rope_sin_cos, lib.rs:191-195."""
    s, c = ctypes.c_float(), ctypes.c_float()
    r = lib().qxo_granite_rope_sin_cos(position, pair, ctypes.byref(s), ctypes.byref(c))
    return None if r else (s.value, c.value)


def granite_rope_pair(position: int, pair: int, left: float, right: float):
    """granite_rope_pair, lib.rs:198-207."""
    f, g = ctypes.c_float(), ctypes.c_float()
    r = lib().qxo_granite_rope_pair(position, pair, float(left), float(right), ctypes.byref(f), ctypes.byref(g))
    return None if r else (f.value, g.value)


def f32_bits(x) -> int:
    return int(np.array(x, dtype=np.float32).view(np.uint32))


def round_to(a, fmt: int):
    """Round fp32 values to the storage format (RNE) and back."""
    a = _f32(a)
    if fmt == F16:
        return a.astype(np.float16).astype(np.float32)
    if fmt == BF16:
        return bf16_bits_to_f32(f32_to_bf16_bits(a))
    return a.copy()


def f32_to_bf16_bits(a):
    """Vectorised RNE fp32 -> bfloat16 bits (same rule as qxo_f32_to_bf16)."""
    x = _f32(a).view(np.uint32).astype(np.uint64)
    nan = (x & 0x7FFFFFFF) > 0x7F800000
    r = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((x[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bits16(a, fmt: int):
    return _f32(a).astype(np.float16).view(np.uint16) if fmt == F16 else f32_to_bf16_bits(a)


def from_bits16(b, fmt: int):
    b = np.asarray(b, dtype=np.uint16)
    return b.view(np.float16).astype(np.float32) if fmt == F16 else bf16_bits_to_f32(b)


# --- Granite (crates/qx-runtime/src/lib.rs) ----------------------------------

def apply_granite_rope(query, key, position: int):
    """apply_granite_rope, lib.rs:434-441.  Returns rotated copies."""
    q, k = _f32(query).copy(), _f32(key).copy()
    _check(lib().qxo_apply_granite_rope(_p(q), _p(k), position))
    return q, k


def apply_granite_rope_rows(query, key, start: int):
    """apply_granite_rope of query [T][1024] and key [T][512] rows at positions
    start + t, in one C loop (the prompt loop's RoPE, lib.rs:1341-1353)."""
    q, k = _f32(query).copy(), _f32(key).copy()
    t = q.shape[0]
    assert q.shape == (t, 1024) and k.shape == (t, 512)
    _check(lib().qxo_apply_granite_rope_rows(_p(q), _p(k), t, start))
    return q, k


class KvCache:
    """KvCache, lib.rs:349-431: position-major fp32 rows with a cursor.

    key_format/value_format round values on append (fp16 Metal stores,
    kernels/v2_decode.metal:445-488); F32 is the reference cache."""

    def __init__(self, capacity: int, key_format: int = F32, value_format: int = F32):
        self.capacity = capacity
        self._h = lib().qxo_kv_cache_new(capacity, key_format, value_format)
        if not self._h:
            raise MemoryError("oracle KvCache allocation failed")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            _lib.qxo_kv_cache_free(h)
            self._h = None

    def __len__(self):
        return lib().qxo_kv_cache_len(self._h)

    def rollback(self, length: int):
        """Cursor-only rewind (rollback_kv, crates/qx-runtime-v2/src/lib.rs:3271-3285)."""
        if lib().qxo_kv_cache_rollback(self._h, length):
            raise OracleError(f"rollback to {length} beyond length {len(self)}")

    def reset(self):
        lib().qxo_kv_cache_reset(self._h)

    def append(self, position: int, key, value):
        k, v = _f32(key), _f32(value)
        _check(lib().qxo_kv_cache_append(self._h, position, _p(k), _p(v)))

    def extend(self, keys, values):
        """Store pre-rotated position-major rows [n][8][64] at the cursor."""
        k, v = _f32(keys), _f32(values)
        n = k.size // (GRANITE_KV_HEADS * GRANITE_HEAD_DIM)
        _check(lib().qxo_kv_cache_extend(self._h, n, _p(k), _p(v)))

    def keys(self):
        n = self.capacity * GRANITE_KV_HEADS * GRANITE_HEAD_DIM
        return np.ctypeslib.as_array(lib().qxo_kv_cache_keys(self._h), shape=(n,)).reshape(
            self.capacity, GRANITE_KV_HEADS, GRANITE_HEAD_DIM)[: len(self)].copy()

    def values(self):
        n = self.capacity * GRANITE_KV_HEADS * GRANITE_HEAD_DIM
        return np.ctypeslib.as_array(lib().qxo_kv_cache_values(self._h), shape=(n,)).reshape(
            self.capacity, GRANITE_KV_HEADS, GRANITE_HEAD_DIM)[: len(self)].copy()


def granite_attention_decode(query, key, value, position: int, cache: KvCache):
    """granite_attention_decode, lib.rs:444-552 (non-hierarchical)."""
    q, k, v = _f32(query), _f32(key), _f32(value)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    _check(lib().qxo_granite_attention_decode(_p(q), _p(k), _p(v), position, cache._h, _p(out)))
    return out


def granite_attend(query_rotated, cache: KvCache, length: int):
    """Attention half of granite_attention_decode (lib.rs:476-549)."""
    q = _f32(query_rotated)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    _check(lib().qxo_granite_attend(_p(q), cache._h, length, _p(out)))
    return out


def granite_prefill_rows(query_rotated, cache: KvCache, start: int, rows):
    """Repeated-decode causal prefill (lib.rs:1341-1353): row t attends [0, start+t]."""
    q = _f32(query_rotated)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    out = np.zeros((rows.size, GRANITE_HIDDEN), np.float32)
    _check(lib().qxo_granite_prefill_rows(_p(q), cache._h, start, _p(rows, _u32p), rows.size, _p(out)))
    return out


def granite_rms_norm(hidden, weight):
    """rms_norm, lib.rs:2406-2414."""
    h, w = _f32(hidden), _f32(weight)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    _check(lib().qxo_granite_rms_norm(_p(h), _p(w), _p(out)))
    return out


def dense_apply(weight, vector):
    """DenseMatrix::apply (non-macOS), lib.rs:625-637."""
    w, x = _f32(weight), _f32(vector)
    rows, cols = w.shape
    out = np.zeros(rows, np.float32)
    lib().qxo_dense_apply(_p(w), rows, cols, _p(x), _p(out))
    return out


def granite_attention_block(hidden, norm_weight, wq, wk, wv, wo, position: int, cache: KvCache):
    """Attention half of GraniteLayerWeights::decode_with_trace, lib.rs:847-929."""
    arrs = [_f32(a) for a in (hidden, norm_weight, wq, wk, wv, wo)]
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    _check(lib().qxo_granite_attention_block(*[_p(a) for a in arrs], position, cache._h, _p(out)))
    return out


# --- group-32 Q4 projections (crates/qx-quant/src/lib.rs) --------------------

class Q4Matrix:
    """A group-32 Q4 matrix in the reference's RowMajor layout: `packed`
    uint8 [rows, cols/2] (value i of a group is nibble i%2, low first, of byte
    i/2) and `scales` f16 bit patterns uint16 [rows, cols/32]."""

    def __init__(self, packed, scales, rows: int, cols: int):
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(rows, cols // 2)
        self.scales = np.ascontiguousarray(scales, dtype=np.uint16).reshape(rows, cols // 32)
        self.rows, self.cols = rows, cols


def q4_quantize(weight) -> Q4Matrix:
    """QuantizedTensor::quantize(Q4, group 32), lib.rs:313-360, 1383-1404."""
    w = _f32(weight)
    rows, cols = w.shape
    packed = np.zeros((rows, cols // 2), np.uint8)
    scales = np.zeros((rows, max(cols // 32, 1)), np.uint16)
    _check(lib().qxo_q4_quantize(_p(w), rows, cols, _p(packed, _u8p), _p(scales, _u16p)))
    return Q4Matrix(packed, scales, rows, cols)


def q4_dequantize(m: Q4Matrix):
    """QuantizedTensor::dequantize, lib.rs:819-846."""
    out = np.zeros((m.rows, m.cols), np.float32)
    lib().qxo_q4_dequantize(_p(m.packed, _u8p), _p(m.scales, _u16p), m.rows, m.cols, _p(out))
    return out


def q4_mat_vec_simd32(m: Q4Matrix, vector, multiplier: float = 1.0):
    """QuantizedTensor::mat_vec_simd32, lib.rs:892-938 (times the Metal
    kernel's multiplier, kernels/q4_dense.metal:151-180)."""
    x = _f32(vector)
    out = np.zeros(m.rows, np.float32)
    _check(lib().qxo_q4_mat_vec_simd32(_p(m.packed, _u8p), _p(m.scales, _u16p), m.rows, m.cols, _p(x),
                                       float(multiplier), _p(out)))
    return out


def q4_mat_vec(m: Q4Matrix, vector):
    """QuantizedTensor::mat_vec (Q4, RowMajor), crates/qx-quant/src/lib.rs:851-891:
    one sequential fma chain per row."""
    x = _f32(vector)
    out = np.zeros(m.rows, np.float32)
    _check(lib().qxo_q4_mat_vec(_p(m.packed, _u8p), _p(m.scales, _u16p), m.rows, m.cols, _p(x), _p(out)))
    return out


def granite_rms_norm_simd(hidden, weight=None):
    """rms_norm_simd, crates/qx-runtime/src/lib.rs:2416-2432.  Returns
    (normalized or None, sum of squares, inverse RMS)."""
    h = _f32(hidden)
    total, inv = ctypes.c_float(), ctypes.c_float()
    out = None
    if weight is not None:
        w = _f32(weight)
        out = np.zeros(GRANITE_HIDDEN, np.float32)
        _check(lib().qxo_granite_rms_norm_simd(_p(h), _p(w), _p(out), ctypes.byref(total), ctypes.byref(inv)))
    else:
        _check(lib().qxo_granite_rms_norm_simd(_p(h), None, None, ctypes.byref(total), ctypes.byref(inv)))
    return out, np.float32(total.value), np.float32(inv.value)


def granite_residual(hidden, projection):
    """fma(0.22, projection, hidden), crates/qx-runtime/src/lib.rs:917-923."""
    h, pr = _f32(hidden), _f32(projection)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    lib().qxo_granite_residual(_p(h), _p(pr), _p(out))
    return out


def granite_attend_simd(query_rotated, cache: "KvCache", length: int):
    """Hierarchical attention half of granite_attention_decode_with_profile,
    crates/qx-runtime/src/lib.rs:476-549 (length <= 512)."""
    q = _f32(query_rotated)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    _check(lib().qxo_granite_attend_simd(_p(q), cache._h, length, _p(out)))
    return out


def granite_q4_attention_block(hidden, norm_weight, wq: Q4Matrix, wk: Q4Matrix, wv: Q4Matrix, wo: Q4Matrix,
                               position: int, cache: "KvCache"):
    """Attention half of the Granite layer with Q4 projections (the V1
    `ordered` profile, crates/qx-runtime/src/lib.rs:847-929).  Returns
    (hidden_out, rotated query, attention, inverse RMS of hidden_out)."""
    h, nw = _f32(hidden), _f32(norm_weight)
    out = np.zeros(GRANITE_HIDDEN, np.float32)
    q = np.zeros(GRANITE_HIDDEN, np.float32)
    att = np.zeros(GRANITE_HIDDEN, np.float32)
    inv = ctypes.c_float()
    mats = []
    for m in (wq, wk, wv, wo):
        mats += [_p(m.packed, _u8p), _p(m.scales, _u16p)]
    _check(lib().qxo_granite_q4_attention_block(_p(h), _p(nw), *mats, position, cache._h, _p(out), _p(q),
                                                _p(att), ctypes.byref(inv)))
    return out, q, att, np.float32(inv.value)


# --- Qwen (tools/qx-qwen-parity/src/main.rs) ---------------------------------

def qwen_qk_norm_rope_rows(query_bits, key_bits, query_norm, key_norm, start: int, fmt: int = F16):
    """cpu_qk_norm_rope of query [T][4096] and key [T][512] 16-bit rows at
    positions start + t, in one C loop."""
    q = np.ascontiguousarray(query_bits, dtype=np.uint16)
    k = np.ascontiguousarray(key_bits, dtype=np.uint16)
    t = q.shape[0]
    assert q.shape == (t, 4096) and k.shape == (t, 512)
    qn, kn = _f32(query_norm), _f32(key_norm)
    qo, ko = np.zeros_like(q), np.zeros_like(k)
    lib().qxo_qwen_qk_norm_rope_rows(_p(q, _u16p), _p(k, _u16p), _p(qn), _p(kn), t, start, fmt, _p(qo, _u16p),
                                     _p(ko, _u16p))
    return qo, ko


def qwen_qk_norm_rope(query_bits, key_bits, query_norm, key_norm, position: int, fmt: int = F16):
    """cpu_qk_norm_rope, main.rs:1170-1210 (16-bit I/O in `fmt`)."""
    q = np.ascontiguousarray(query_bits, dtype=np.uint16)
    k = np.ascontiguousarray(key_bits, dtype=np.uint16)
    qn, kn = _f32(query_norm), _f32(key_norm)
    qo, ko = np.zeros_like(q), np.zeros_like(k)
    lib().qxo_qwen_qk_norm_rope(_p(q, _u16p), _p(k, _u16p), _p(qn), _p(kn), position, fmt,
                                _p(qo, _u16p), _p(ko, _u16p))
    return qo, ko


def qwen_rms_norm(vector, weight, epsilon: float = 1e-6):
    """rms_norm, tools/qx-qwen-parity/src/main.rs:1157-1168."""
    x, w = _f32(vector), _f32(weight)
    out = np.zeros(x.size, np.float32)
    lib().qxo_qwen_rms_norm(_p(x), _p(w), x.size, float(epsilon), _p(out))
    return out


def _f16_round(a):
    return np.asarray(a, np.float32).astype(np.float16)


def qwen_attention_block(hidden_bits, input_norm, wq: "Q4Matrix", wk: "Q4Matrix", wv: "Q4Matrix", query_norm,
                         key_norm, wo: "Q4Matrix", post_attention_norm, position: int, key_cache_bits,
                         value_cache_bits):
    """The attention half of a Qwen layer as the parity tool checks it stage by
    stage (tools/qx-qwen-parity/src/main.rs:124-240; the GPU graph is
    PreparedQwenLayer::encode_with_expert_cache, crates/qx-runtime-v2/src/lib.rs:
    904-973): f16 rms_norm of the f16 hidden state, f16 Q4 q/k/v projections
    (mat_vec), cpu_qk_norm_rope, K/V stored at `position`, cpu_gqa_attention,
    f16 Q4 o projection, hidden_after = f16(hidden + projection) and
    moe_input = f16(rms_norm(hidden_after)).  Caches are position-major f16
    bits [ctx][4][128] holding positions [0, position); the new rows are
    appended in a copy.  Returns a dict of every stage (f16 arrays)."""
    h = np.asarray(hidden_bits, np.uint16).view(np.float16).astype(np.float32)
    a = _f16_round(qwen_rms_norm(h, input_norm))
    q = _f16_round(q4_mat_vec(wq, a.astype(np.float32)))
    k = _f16_round(q4_mat_vec(wk, a.astype(np.float32)))
    v = _f16_round(q4_mat_vec(wv, a.astype(np.float32)))
    qr_bits, kr_bits = qwen_qk_norm_rope(q.view(np.uint16), k.view(np.uint16), query_norm, key_norm, position, F16)
    kc = np.concatenate([np.asarray(key_cache_bits, np.uint16).reshape(-1, 512)[:position],
                         np.asarray(kr_bits, np.uint16).reshape(1, 512)])
    vc = np.concatenate([np.asarray(value_cache_bits, np.uint16).reshape(-1, 512)[:position],
                         v.view(np.uint16).reshape(1, 512)])
    att_bits = qwen_gqa_attention(qr_bits, kc, vc, F16)
    att = np.asarray(att_bits, np.uint16).view(np.float16).astype(np.float32)
    proj = _f16_round(q4_mat_vec(wo, att))
    after = _f16_round(h + proj.astype(np.float32))
    moe = _f16_round(qwen_rms_norm(after.astype(np.float32), post_attention_norm))
    return {"attention_input": a, "query": q, "key": k, "value": v,
            "query_rotated": np.asarray(qr_bits, np.uint16).view(np.float16),
            "key_rotated": np.asarray(kr_bits, np.uint16).view(np.float16),
            "attention": att.astype(np.float16), "projection": proj, "hidden_after_attention": after,
            "moe_input": moe}


def qwen_inverse_frequencies():
    return np.array([lib().qxo_qwen_inverse_frequency(i) for i in range(64)], np.float32)


def qwen_gqa_attention(query_bits, key_cache_bits, value_cache_bits, fmt: int = F16, want_f32=False):
    """cpu_gqa_attention, main.rs:1218-1258 (position-major caches)."""
    q = np.ascontiguousarray(query_bits, dtype=np.uint16)
    kc = np.ascontiguousarray(key_cache_bits, dtype=np.uint16)
    vc = np.ascontiguousarray(value_cache_bits, dtype=np.uint16)
    context = kc.size // (QWEN_KV_HEADS * QWEN_HEAD_DIM)
    out = np.zeros(QWEN_Q_HEADS * QWEN_HEAD_DIM, np.uint16)
    of = np.zeros(QWEN_Q_HEADS * QWEN_HEAD_DIM, np.float32)
    _check(lib().qxo_qwen_gqa_attention(_p(q, _u16p), _p(kc, _u16p), _p(vc, _u16p), context, fmt,
                                        _p(out, _u16p), _p(of)))
    return (out, of) if want_f32 else out


def qwen_prefill_rows(query_bits, key_cache_bits, value_cache_bits, start: int, rows, fmt: int = F16,
                      workers: int = 1):
    """Repeated-decode causal prefill for Qwen; returns (bits, f32) for `rows`.

    workers > 1 splits the rows over that many threads (each row is an
    independent C call that holds no state between calls; ctypes releases
    the GIL while it runs), for samples of long prompts."""
    q = np.ascontiguousarray(query_bits, dtype=np.uint16)
    kc = np.ascontiguousarray(key_cache_bits, dtype=np.uint16)
    vc = np.ascontiguousarray(value_cache_bits, dtype=np.uint16)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    n = QWEN_Q_HEADS * QWEN_HEAD_DIM
    out = np.zeros((rows.size, n), np.uint16)
    of = np.zeros((rows.size, n), np.float32)

    def run(idx):
        r = np.ascontiguousarray(rows[idx])
        o = np.zeros((r.size, n), np.uint16)
        f = np.zeros((r.size, n), np.float32)
        status = lib().qxo_qwen_prefill_rows(_p(q, _u16p), _p(kc, _u16p), _p(vc, _u16p), start, _p(r, _u32p),
                                             r.size, fmt, _p(o, _u16p), _p(f))
        out[idx], of[idx] = o, f
        return status

    w = max(1, min(workers, rows.size))
    if w == 1:
        _check(run(np.arange(rows.size)))
        return out, of
    import concurrent.futures as cf
    # rows dealt round-robin, so long and short rows spread over the threads
    with cf.ThreadPoolExecutor(w) as ex:
        codes = list(ex.map(lambda i: run(np.arange(i, rows.size, w)), range(w)))
    for c in codes:
        _check(c)
    return out, of


# ---------------------------------------------------------------------------
# KV / state commitment hashing (oracle/qx_oracle_hash.c)
# ---------------------------------------------------------------------------
D_KV = b"QX:KV:V1"
D_MERKLE = b"QX:MERKLE:V1"
D_CHECKPOINT = b"QX:CHECKPOINT:V1"
D_STATE, D_STATE_CHUNK = b"QX:STATE:V1", b"QX:STATE:CHUNK:V1"
D_KV_KEY_CHUNK, D_KV_KEY_TREE = b"QX:KV:KEY:CHUNK:V1", b"QX:KV:KEY:TREE:V1"
D_KV_VALUE_CHUNK, D_KV_VALUE_TREE = b"QX:KV:VALUE:CHUNK:V1", b"QX:KV:VALUE:TREE:V1"


def _bytes_arg(b: bytes):
    buf = (ctypes.c_uint8 * max(len(b), 1)).from_buffer_copy(b if b else b"\0")
    return buf


def _digest_call(fn, *args) -> bytes:
    out = (ctypes.c_uint8 * 32)()
    if fn(*args, out) != 0:
        raise RuntimeError("oracle hash: input rejected")
    return bytes(out)


def blake3(data: bytes) -> bytes:
    """BLAKE3 (blake3 crate 1.8.7) of at most one 1024-byte chunk."""
    L = lib()
    return _digest_call(L.qxo_blake3, _bytes_arg(data), ctypes.c_size_t(len(data)))


def hash_domain_b3(domain: bytes, fields) -> bytes:
    """hash_domain(Blake3V1, domain, fields), crates/qx-commit/src/hash.rs:36-65."""
    L = lib()
    bufs = [_bytes_arg(f) for f in fields]
    n = len(fields)
    ptrs = (ctypes.POINTER(ctypes.c_uint8) * max(n, 1))(*[ctypes.cast(b, _u8p) for b in bufs])
    lens = (ctypes.c_size_t * max(n, 1))(*[len(f) for f in fields])
    return _digest_call(L.qxo_hash_domain_b3, _bytes_arg(domain), ctypes.c_size_t(len(domain)), ctypes.c_size_t(n),
                        ptrs, lens)


def chunk_tree_hash(data: bytes, chunk_bytes: int, leaf_domain: bytes, tree_domain: bytes) -> bytes:
    """chunk_tree_hash, crates/qx-commit/src/state.rs:213-250."""
    L = lib()
    return _digest_call(L.qxo_chunk_tree_hash, _bytes_arg(data), ctypes.c_size_t(len(data)),
                        ctypes.c_size_t(chunk_bytes), ctypes.c_char_p(leaf_domain), ctypes.c_char_p(tree_domain))


def state_hash_v1(data: bytes) -> bytes:
    """state_hash_v1, crates/qx-commit/src/state.rs:353-355."""
    return _digest_call(lib().qxo_state_hash_v1, _bytes_arg(data), ctypes.c_size_t(len(data)))


def kv_leaf_hash_v1(layer: int, token: int, key: bytes, value: bytes) -> bytes:
    """kv_leaf_hash_v1, crates/qx-commit/src/state.rs:334-348."""
    return _digest_call(lib().qxo_kv_leaf_hash_v1, ctypes.c_uint16(layer), ctypes.c_uint32(token), _bytes_arg(key),
                        ctypes.c_size_t(len(key)), _bytes_arg(value), ctypes.c_size_t(len(value)))


def kv_leaf_hashes(layer: int, token_begin: int, keys, values):
    """kv_leaf_hash_v1 of every row of position-major keys / values
    ([rows][row bytes] uint8): a C loop, one leaf after another."""
    k = np.ascontiguousarray(keys, dtype=np.uint8)
    v = np.ascontiguousarray(values, dtype=np.uint8)
    rows = k.shape[0]
    out = np.zeros((rows, 32), np.uint8)
    _check(lib().qxo_kv_leaf_hashes(ctypes.c_uint16(layer), ctypes.c_uint32(token_begin), ctypes.c_uint32(rows),
                                    _p(k, _u8p), ctypes.c_size_t(k.shape[1]), _p(v, _u8p),
                                    ctypes.c_size_t(v.shape[1]), _p(out, _u8p)))
    return out


def verification_hashes(residuals: bytes, residual_stride: int, key_rows, value_rows, token: int, layers: int,
                        interval: int) -> bytes:
    """Per-token digests of kernels/verification_hash.metal:349-522: (layers + 1) x 64 bytes."""
    L = lib()
    kb = [_bytes_arg(r) for r in key_rows]
    vb = [_bytes_arg(r) for r in value_rows]
    kp = (ctypes.POINTER(ctypes.c_uint8) * layers)(*[ctypes.cast(b, _u8p) for b in kb])
    vp = (ctypes.POINTER(ctypes.c_uint8) * layers)(*[ctypes.cast(b, _u8p) for b in vb])
    out = (ctypes.c_uint8 * (64 * (layers + 1)))()
    if L.qxo_verification_hashes(_bytes_arg(residuals), ctypes.c_size_t(residual_stride), kp, vp,
                                 ctypes.c_size_t(len(key_rows[0])), ctypes.c_size_t(len(value_rows[0])),
                                 ctypes.c_uint32(token), ctypes.c_uint32(layers),
                                 ctypes.c_uint32(interval), out) != 0:
        raise RuntimeError("oracle verification hashes: input rejected")
    return bytes(out)


# --- tiered value cache ------------------------------------------------------
# The reference proposes a tiered value cache (recent V in fp16, older V in
# block-scaled INT8; docs/qx-structural-memory-2026-08-25.md:69-74) and does
# not implement it, so there is no reference code or golden vector to follow:
# this build defines the format (include/qx_hip.h, QXH_I8_TIERED) and these
# functions restate that definition.  Parity is pinned by mathematics in
# tests/test_oracle_tiered_v.py: exactly representable blocks, brute-force
# nearest codes, the clamp and zero-scale cases, and the invariants of the
# tier boundary under appends and rollbacks.

TIER_BLOCK = 32


def tiered_quantize(values_f16):
    """Rows of binary16 values [..., d] (d a multiple of 32) -> (int8 codes
    [..., d], binary16 scales [..., d / 32]): per block of 32, scale =
    f16(f32(max|v|) / 127), code = clamp(rint(v / scale), -127, 127) in f32
    arithmetic, and code 0 where the scale is 0."""
    v = np.asarray(values_f16, dtype=np.float16).astype(np.float32)
    blocks = v.reshape(v.shape[:-1] + (v.shape[-1] // TIER_BLOCK, TIER_BLOCK))
    amax = np.max(np.abs(blocks), axis=-1)
    scale16 = (amax / np.float32(127.0)).astype(np.float32).astype(np.float16)
    s = scale16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint(blocks / s)
    q = np.where(s > 0, np.clip(q, -127, 127), 0).astype(np.int8)
    return q.reshape(v.shape), scale16


def tiered_dequantize(codes, scales16):
    """code * scale in f32 (exact: 8-bit code times 11-bit significand)."""
    c = np.asarray(codes, dtype=np.int8).astype(np.float32)
    blocks = c.reshape(c.shape[:-1] + (c.shape[-1] // TIER_BLOCK, TIER_BLOCK))
    s = np.asarray(scales16, dtype=np.float16).astype(np.float32)[..., None]
    return (blocks * s).reshape(c.shape)


class TieredValueCache:
    """Value rows of one sequence under the tiered format: position-major
    [n][kv_heads][d] history with the boundary rule of qxh_kv_cache_value_tier.
    `rows()` gives what the cache holds at each committed position as f32:
    binary16 values at and after the boundary, dequantised INT8 before it."""

    def __init__(self, window: int, kv_heads: int = GRANITE_KV_HEADS, head_dim: int = GRANITE_HEAD_DIM):
        self.window, self.kv_heads, self.head_dim = window, kv_heads, head_dim
        self.half = np.zeros((0, kv_heads, head_dim), np.float16)  # binary16 value per position
        self.codes = np.zeros((0, kv_heads, head_dim), np.int8)
        self.scales = np.zeros((0, kv_heads, head_dim // TIER_BLOCK), np.float16)
        self.length = 0
        self.boundary = 0

    def _grow(self, n):
        if n > len(self.half):
            extra = n - len(self.half)
            self.half = np.concatenate([self.half, np.zeros((extra,) + self.half.shape[1:], np.float16)])
            self.codes = np.concatenate([self.codes, np.zeros((extra,) + self.codes.shape[1:], np.int8)])
            self.scales = np.concatenate([self.scales, np.zeros((extra,) + self.scales.shape[1:], np.float16)])

    def append(self, rows):
        """Append value rows [t][kv_heads][d] (any float dtype; rounded to
        binary16) at the cursor."""
        rows = np.asarray(rows, dtype=np.float32).astype(np.float16)
        s, t = self.length, rows.shape[0]
        new_b = max(self.boundary, s + t - self.window)
        self._grow(s + t)
        self.half[s:s + t] = rows
        lo = self.boundary
        if new_b > lo:
            self.codes[lo:new_b], self.scales[lo:new_b] = tiered_quantize(self.half[lo:new_b])
        self.length, self.boundary = s + t, new_b

    def rollback(self, length: int):
        assert length <= self.length
        self.length = length
        self.boundary = min(self.boundary, length)

    def fill(self, rows):
        """A bulk fill of rows [0, n): the boundary settles at max(0, n - window)."""
        self.length, self.boundary = 0, 0
        self.append(rows)

    def rows(self):
        out = self.half[: self.length].astype(np.float32)
        b = self.boundary
        out[:b] = tiered_dequantize(self.codes[:b], self.scales[:b])
        return out


def _splitmix64(x):
    x = (np.asarray(x, dtype=np.uint64) + np.uint64(0x9E3779B97F4A7C15))
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def tiered_fill_values(seed: int, block: int, capacity: int, length: int, head_dim: int = GRANITE_HEAD_DIM):
    """f16 values [length][head_dim] that the library's synthetic fill of a
    tiered value cache (qxh_encode_kv_fill_normal) gives (layer, sequence, kv
    head) block `block` = (layer * sequences + sequence) * kv_heads + head:
    element d of row p is the Irwin-Hall sum of the four 16-bit fields of
    splitmix64(seed ^ 0x5DEECE66DA5A5A5A ^ splitmix64((block * capacity + p)
    * head_dim + d)), centred, times 2^-15 (exact), rounded to f16.  A
    test fixture generator of this library, not a reference function."""
    with np.errstate(over="ignore"):
        ctr = (np.uint64(block) * np.uint64(capacity) + np.arange(length, dtype=np.uint64)[:, None]) * \
            np.uint64(head_dim) + np.arange(head_dim, dtype=np.uint64)[None, :]
        h = _splitmix64(np.uint64(seed ^ 0x5DEECE66DA5A5A5A) ^ _splitmix64(ctr))
    fields = [((h >> np.uint64(16 * i)) & np.uint64(0xFFFF)).astype(np.int64) for i in range(4)]
    total = (fields[0] + fields[1] + fields[2] + fields[3] - 131070).astype(np.float32)
    return (total * np.float32(2.0 ** -15)).astype(np.float16)
