"""GPU parity: device quantizer, KV append and the synthetic generator are
bit exact with the oracle (quant.zig:197-288 semantics)."""
import ctypes
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def _tricky_rows(cols: int, bias: int) -> np.ndarray:
    rows = [o.normal(cols, 31, r, 0.5) for r in range(24)]
    zero = np.zeros(cols, np.float32)
    sub = np.zeros(cols, np.float32)
    sub[3] = np.float32(1.5e-7) * bias   # f16 subnormal scale
    sub[70 % cols] = np.float32(-3e-8) * bias
    tie = np.zeros(cols, np.float32)
    tie[0] = np.float32((1.0 + 1.0 / 2048.0) * bias)   # max / bias exactly halfway between f16 values
    tie[1] = np.float32(0.5)
    exact = np.zeros(cols, np.float32)
    exact[0], exact[1] = 7.0, -8.0
    half = (np.arange(cols, dtype=np.float32) - cols / 2) * np.float32(0.5)  # many x.5 quotients
    huge = o.normal(cols, 32, 0, 1.0)
    huge[5] = np.float32(1e7)      # scale overflows f16 to infinity
    return np.stack(rows + [zero, sub, tie, exact, half, huge]).astype(np.float32)


@pytest.mark.parametrize("fmt", [qa.FORMAT_Q4, qa.FORMAT_Q5, qa.FORMAT_Q8])
def test_device_quantizer_is_bit_exact(ctx, fmt):
    bias = {16: 8, 17: 16, 18: 128}[fmt]
    values = _tricky_rows(256, bias)
    rows, cols = values.shape
    s_ref, d_ref = o.quantize_rows(fmt, values)
    vbuf = ctx.to_device(values)
    sbuf = ctx.buffer(s_ref.nbytes)
    dbuf = ctx.buffer(d_ref.nbytes)
    ctx.quantize_rows(fmt, vbuf.ptr, rows, cols, sbuf.ptr, dbuf.ptr)
    s_gpu = sbuf.download(np.uint8)
    d_gpu = dbuf.download(np.uint8)
    assert np.array_equal(s_gpu, s_ref)
    assert np.array_equal(d_gpu, d_ref)
    for b in (vbuf, sbuf, dbuf):
        b.free()


def test_device_quantizer_matches_the_golden_pattern(ctx):
    # selftest.zig:73-126 pattern through the device quantizer: the FNV hash of
    # its q4, q5, q8 planes is the reference's golden quant_hash.
    # The pattern is f32(cos(f32(i) * 0.19)) * 1.75 with the C library's cosf,
    # as the oracle computes it.
    libm = ctypes.CDLL("libm.so.6")
    libm.cosf.restype = ctypes.c_float
    libm.cosf.argtypes = [ctypes.c_float]
    values = np.array([np.float32(libm.cosf(float(np.float32(i) * np.float32(0.19)))) * np.float32(1.75)
                       for i in range(128)], np.float32)
    h = 0xCBF29CE484222325
    h_ref = 0xCBF29CE484222325
    for fmt in (qa.FORMAT_Q4, qa.FORMAT_Q5, qa.FORMAT_Q8):
        s_ref, d_ref = o.quantize_rows(fmt, values)
        vbuf = ctx.to_device(values)
        sbuf = ctx.buffer(s_ref.nbytes)
        dbuf = ctx.buffer(d_ref.nbytes)
        ctx.quantize_rows(fmt, vbuf.ptr, 1, 128, sbuf.ptr, dbuf.ptr)
        h = o.fnv1a64(dbuf.download(np.uint8), o.fnv1a64(sbuf.download(np.uint8), h))
        h_ref = o.fnv1a64(d_ref, o.fnv1a64(s_ref, h_ref))
        for b in (vbuf, sbuf, dbuf):
            b.free()
    assert h_ref == 0xF247917B05691FD1
    assert h == 0xF247917B05691FD1


@pytest.mark.parametrize("seed,stream,count", [(0, 0, 1 << 20), (4, 3, 100003), (0x5EED0001, 17, 4096)])
def test_synthetic_generator_is_bit_exact(ctx, seed, stream, count):
    buf = ctx.buffer(count * 4)
    ctx.synth_normal(seed, stream, count, 1.0, buf.ptr)
    gpu = buf.download(np.float32)
    ref = o.normal(count, seed, stream)
    assert np.array_equal(gpu.view(np.uint32), ref.view(np.uint32))
    buf.free()


def test_synthetic_matrix_matches_oracle_planes(ctx):
    rows, cols, seed, stream = 777, 1024, 1, 8
    handle = ctx.matrix_synthetic(qa.FORMAT_Q4, rows, cols, seed, stream, 0.02)
    s_ref, d_ref = o.quantize_rows(o.Q4, o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols))
    sp, dp = ctx.matrix_planes(handle)
    s_gpu = np.empty(s_ref.size, np.uint8)
    d_gpu = np.empty(d_ref.size, np.uint8)
    ctx._check(ctx.lib.qwh_download(ctx.handle, s_gpu.ctypes.data, sp, s_gpu.nbytes))
    ctx._check(ctx.lib.qwh_download(ctx.handle, d_gpu.ctypes.data, dp, d_gpu.nbytes))
    assert np.array_equal(s_gpu, s_ref) and np.array_equal(d_gpu, d_ref)
    ctx.matrix_release(handle)


def test_kv_append_is_bit_exact(ctx):
    # harness.mjs:285-288: two rows of 128 (kv_width 128), second group of the
    # second row all zeros; then a row appended at position 5 of 8.
    values = o.normal(256, 0x5EED0015)
    values[64 + 64:] = 0.0
    key, value = values[:128].copy(), values[128:].copy()
    kv_width, positions = 128, 8
    gpr = kv_width // 64
    planes = [ctx.buffer(positions * gpr * 2), ctx.buffer(positions * kv_width),
              ctx.buffer(positions * gpr * 2), ctx.buffer(positions * kv_width)]
    for p in planes:
        ctx._check(ctx.lib.qwh_memset(ctx.handle, p.ptr, 0, p.nbytes))
    kbuf, vbuf = ctx.to_device(key), ctx.to_device(value)
    for position in (0, 5):
        ctx.kv_append_q8(kbuf.ptr, vbuf.ptr, kv_width, position, *[p.ptr for p in planes])
    ks_ref, kc_ref = o.quantize_rows(o.Q8, key)
    vs_ref, vc_ref = o.quantize_rows(o.Q8, value)
    ks, kc, vs, vc = [p.download(np.uint8) for p in planes]
    for position in (0, 5):
        assert np.array_equal(ks[position * gpr * 2:(position + 1) * gpr * 2], ks_ref)
        assert np.array_equal(kc[position * kv_width:(position + 1) * kv_width], kc_ref)
        assert np.array_equal(vs[position * gpr * 2:(position + 1) * gpr * 2], vs_ref)
        assert np.array_equal(vc[position * kv_width:(position + 1) * kv_width], vc_ref)
    assert vs_ref.view(np.uint16)[1] == 0  # the zero group stores scale 0
    untouched = [i for i in range(positions) if i not in (0, 5)]
    for i in untouched:
        assert not kc[i * kv_width:(i + 1) * kv_width].any()
    for b in planes + [kbuf, vbuf]:
        b.free()
