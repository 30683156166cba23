"""GPU parity of the q4 / q5 / q8 GEMM with bf16 activations (kernels.zig:118-158 with
tokens = M; the oracle consumes the same bf16 values widened to f32)."""
import os

import numpy as np
import pytest

from oracle import oracle as o
from util import assert_close

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    # half_float.zig:30-39 (round to nearest even; inputs are finite).
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def widen(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def run_gemm(ctx, rows, cols, scales, data, xb16, tokens, fmt=o.Q4):
    handle = ctx.matrix_upload(fmt, rows, cols, scales, data)
    xb = ctx.to_device(xb16)
    ob = ctx.buffer(tokens * rows * 4)
    ctx.linear_bf16(handle, xb.ptr, cols, tokens, ob.ptr)
    out = ob.download(np.float32).reshape(tokens, rows)
    ctx.matrix_release(handle)
    xb.free()
    ob.free()
    return out


@pytest.mark.parametrize("shape", [(6144, 2048), (2048, 6144)])
@pytest.mark.parametrize("m", [128, 512, 1500])
def test_config3_q4_gemm(ctx, shape, m):
    rows, cols = shape
    w = o.normal(rows * cols, 2, 1 if rows == 6144 else 2, 0.02).reshape(rows, cols)
    scales, data = o.quantize_rows(o.Q4, w)
    xb16 = to_bf16_bits(o.normal(m * cols, 2, 10 + m))
    actual = run_gemm(ctx, rows, cols, scales, data, xb16, m)
    # The oracle over a sample of 384 weight rows (every token): the same
    # planes sliced by row.
    gpr = cols // 64
    sample = np.linspace(0, rows - 1, 384).astype(int)
    s_sub = np.concatenate([scales[r * gpr * 2:(r + 1) * gpr * 2] for r in sample])
    d_sub = np.concatenate([data[r * gpr * 32:(r + 1) * gpr * 32] for r in sample])
    expected = o.linear_quantized(o.Q4, s_sub, d_sub, len(sample), cols, widen(xb16), m)
    assert_close(actual[:, sample], expected, what=f"config 3 M {m} {rows}x{cols}")


@pytest.mark.parametrize("rows,cols,m", [(100, 128, 1), (130, 256, 7), (64, 64, 130), (257, 192, 33)])
def test_gemm_edge_shapes(ctx, rows, cols, m):
    w = o.normal(rows * cols, 14, rows, 0.02).reshape(rows, cols)
    scales, data = o.quantize_rows(o.Q4, w)
    xb16 = to_bf16_bits(o.normal(m * cols, 14, 7))
    expected = o.linear_quantized(o.Q4, scales, data, rows, cols, widen(xb16), m)
    actual = run_gemm(ctx, rows, cols, scales, data, xb16, m)
    assert_close(actual, expected, what=f"gemm {m}x{rows}x{cols}")


@pytest.mark.parametrize("rows,cols,m", [(6144, 2048, 390), (6144, 2048, 1500), (2048, 6144, 128), (100, 128, 1),
                                         (130, 256, 7), (257, 192, 33), (64, 64, 130)])
def test_q5_gemm(ctx, rows, cols, m):
    # q5 planes (quant.zig:253-269): 40-byte groups, fifth bits in the last 8.
    # M = 390 is the audio-token count of a 30 s window. M = 1500 at
    # [6144 x 2048] is 576 tiles, more than the two per CU a 256-CU device
    # holds at once: the tiles past the last full wave run as group ranges
    # whose partial tiles a reduce kernel adds (the tail form).
    w = o.normal(rows * cols, 15, rows, 0.02).reshape(rows, cols)
    w[0, :64] = np.float32(-1.0)   # codes at both ends of [-16, 15]
    w[0, 64:128] = np.float32(1.0)
    scales, data = o.quantize_rows(o.Q5, w)
    xb16 = to_bf16_bits(o.normal(m * cols, 15, 9))
    actual = run_gemm(ctx, rows, cols, scales, data, xb16, m, fmt=o.Q5)
    gpr = cols // 64
    sample = np.unique(np.linspace(0, rows - 1, min(rows, 256)).astype(int))
    s_sub = np.concatenate([scales[r * gpr * 2:(r + 1) * gpr * 2] for r in sample])
    d_sub = np.concatenate([data[r * gpr * 40:(r + 1) * gpr * 40] for r in sample])
    expected = o.linear_quantized(o.Q5, s_sub, d_sub, len(sample), cols, widen(xb16), m)
    assert_close(actual[:, sample], expected, what=f"q5 GEMM M {m} {rows}x{cols}")


@pytest.mark.parametrize("rows,cols,m", [(6144, 2048, 1500), (2048, 6144, 512), (6144, 2048, 128), (100, 128, 1),
                                         (130, 256, 7), (257, 192, 33), (64, 64, 130)])
def test_q8_gemm(ctx, rows, cols, m):
    # q8 planes (quant.zig:270-275, 336-340): 64 bytes per group, u - 128.
    # M = 1500 at [6144 x 2048] reaches the tail form on a 256-CU device.
    w = o.normal(rows * cols, 16, rows, 0.02).reshape(rows, cols)
    w[0, :64] = np.float32(-1.0)   # codes at both ends of the q8 range
    w[0, 64:128] = np.float32(1.0)
    scales, data = o.quantize_rows(o.Q8, w)
    xb16 = to_bf16_bits(o.normal(m * cols, 16, 11))
    actual = run_gemm(ctx, rows, cols, scales, data, xb16, m, fmt=o.Q8)
    gpr = cols // 64
    sample = np.unique(np.linspace(0, rows - 1, min(rows, 256)).astype(int))
    s_sub = np.concatenate([scales[r * gpr * 2:(r + 1) * gpr * 2] for r in sample])
    d_sub = np.concatenate([data[r * gpr * 64:(r + 1) * gpr * 64] for r in sample])
    expected = o.linear_quantized(o.Q8, s_sub, d_sub, len(sample), cols, widen(xb16), m)
    assert_close(actual[:, sample], expected, what=f"q8 GEMM M {m} {rows}x{cols}")
