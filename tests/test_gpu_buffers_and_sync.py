"""GPU tests of the C ABI's runtime buffers (RuntimeBuffer and its helpers,
crates/qx-metal/src/lib.rs:1368-1396, :9847-9999) and the synchronous Qwen
helpers (run_qwen_qk_norm_rope / run_qwen_gqa_attention, :14373-14599),
called straight through ctypes as a Rust caller would bind them."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qx_amd import abi
from qx_amd import runtime as rt
from tests.helpers import TOL_16, log, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    return rt.Context(0)


def view():
    return abi.BufferView()


def status(code, match=None):
    if match is not None:
        assert match in abi.last_error(), abi.last_error()
    return code


def test_buffer_alloc_write_subregion_read(ctx):
    L = abi.lib()
    buf = view()
    assert L.qxh_buffer_alloc(ctx.handle, 4096, ctypes.byref(buf)) == 0
    try:
        assert buf.offset == 0 and buf.length == 4096
        data = np.arange(1024, dtype=np.uint32)
        assert L.qxh_buffer_write(buf, data.ctypes.data_as(ctypes.c_void_p), data.nbytes) == 0
        sub = view()
        assert L.qxh_buffer_subregion(buf, 64, 128, ctypes.byref(sub)) == 0
        assert (sub.offset, sub.length) == (64, 128)
        got = np.zeros(32, np.uint32)
        assert L.qxh_buffer_read(sub, got.ctypes.data_as(ctypes.c_void_p), got.nbytes) == 0
        assert np.array_equal(got, data[16:48])
        # a write through a subregion lands at its offset
        ones = np.full(8, 7, np.uint32)
        assert L.qxh_buffer_write(sub, ones.ctypes.data_as(ctypes.c_void_p), ones.nbytes) == 0
        whole = np.zeros(1024, np.uint32)
        assert L.qxh_buffer_read(buf, whole.ctypes.data_as(ctypes.c_void_p), whole.nbytes) == 0
        expect = data.copy()
        expect[16:24] = 7
        assert np.array_equal(whole, expect)
        # the device pointer of a view feeds an encoder: a seeded fill equals torch-tensor fill
        ptr = ctypes.c_void_p()
        assert L.qxh_buffer_device_ptr(sub, ctypes.byref(ptr)) == 0
        t = torch.empty(32, device="cuda:0")
        with rt.Graph(ctx) as g:
            abi.check(L.qxh_encode_fill_normal(g.handle, ptr, abi.F32, 32, 5, ctypes.c_float(1.0)))
            rt.fill_normal(g, t, seed=5)
        back = np.zeros(32, np.float32)
        assert L.qxh_buffer_read(sub, back.ctypes.data_as(ctypes.c_void_p), back.nbytes) == 0
        assert np.array_equal(back, t.cpu().numpy())
        # errors (the reference's Err paths)
        bad = view()
        assert status(L.qxh_buffer_alloc(ctx.handle, 0, ctypes.byref(bad)), "cannot be empty") == 1
        assert status(L.qxh_buffer_subregion(buf, 4000, 100, ctypes.byref(bad)), "exceeds its parent") == 1
        assert status(L.qxh_buffer_subregion(buf, 2**64 - 8, 16, ctypes.byref(bad)), "overflows") == 1
        big = np.zeros(129, np.uint8)
        assert status(L.qxh_buffer_write(sub, big.ctypes.data_as(ctypes.c_void_p), 129), "exceeds runtime buffer") == 1
        assert status(L.qxh_buffer_read(sub, big.ctypes.data_as(ctypes.c_void_p), 129), "exceeds runtime buffer") == 1
    finally:
        assert L.qxh_buffer_free(buf.buffer) == 0


def u16p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("fmt", [abi.F16, abi.BF16])
def test_run_qwen_qk_norm_rope_through_the_c_abi(ctx, fmt):
    rng = np.random.default_rng(41 + fmt)
    q = O.to_bits16(rng.standard_normal(4096), fmt)
    k = O.to_bits16(rng.standard_normal(512), fmt)
    qn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    qo, ko = np.empty_like(q), np.empty_like(k)
    L = abi.lib()
    assert L.qxh_run_qwen_qk_norm_rope(ctx.handle, u16p(q), 4096, u16p(k), 512, u16p(qn), 128, u16p(kn), 128, fmt,
                                       1234, u16p(qo), u16p(ko)) == 0
    rq, rk = O.qwen_qk_norm_rope(q, k, qn, kn, 1234, fmt)
    for got, ref in ((qo, rq), (ko, rk)):
        d = np.abs(got.astype(np.int32) - ref.astype(np.int32))
        assert d.max() <= 1 and np.count_nonzero(d) <= 0.02 * d.size  # libm sin/cos/powf: one ulp at most
    # in place (outputs equal inputs), as the reference rewrites its buffers
    q2, k2 = q.copy(), k.copy()
    assert L.qxh_run_qwen_qk_norm_rope(ctx.handle, u16p(q2), 4096, u16p(k2), 512, u16p(qn), 128, u16p(kn), 128, fmt,
                                       1234, u16p(q2), u16p(k2)) == 0
    assert np.array_equal(q2, qo) and np.array_equal(k2, ko)
    # the reference's shape check
    assert status(L.qxh_run_qwen_qk_norm_rope(ctx.handle, u16p(q), 4095, u16p(k), 512, u16p(qn), 128, u16p(kn), 128,
                                              fmt, 0, u16p(qo), u16p(ko)), "invalid Qwen Q/K shapes") == 1


@pytest.mark.parametrize("fmt,ctxlen", [(abi.F16, 1), (abi.F16, 300), (abi.BF16, 5000)])
def test_run_qwen_gqa_attention_through_the_c_abi(ctx, fmt, ctxlen):
    log("run_qwen_gqa_attention", fmt, ctxlen)
    rng = np.random.default_rng(ctxlen + fmt)
    q = O.to_bits16(rng.standard_normal(4096), fmt)
    kc = O.to_bits16(rng.standard_normal(ctxlen * 512), fmt)
    vc = O.to_bits16(rng.standard_normal(ctxlen * 512), fmt)
    out = np.empty(4096, np.uint16)
    L = abi.lib()
    assert L.qxh_run_qwen_gqa_attention(ctx.handle, u16p(q), 4096, u16p(kc), kc.size, u16p(vc), vc.size, fmt,
                                        u16p(out)) == 0
    _, ref = O.qwen_gqa_attention(q, kc, vc, fmt, want_f32=True)
    got = O.from_bits16(out, fmt).astype(np.float64)
    log(f"  max-abs/rms {rel_err(got, ref):.2e}")
    # the 16-bit bar on a 16-bit output: 2e-3 x RMS plus one unit in the last
    # place of the element (two values within the bar can round one ulp apart)
    mag = np.maximum(np.abs(ref), 1e-30)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - (10 if fmt == abi.F16 else 7))
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert np.all(np.abs(got - ref) <= TOL_16 * rms + ulp)
    if ctxlen == 1:
        assert np.array_equal(out.reshape(32, 128), vc.reshape(4, 128)[np.arange(32) // 8])
    assert status(L.qxh_run_qwen_gqa_attention(ctx.handle, u16p(q), 4096, u16p(kc), kc.size, u16p(vc),
                                               vc.size - 512 if ctxlen > 1 else 0, fmt, u16p(out)),
                  "invalid Qwen GQA shapes") == 1
