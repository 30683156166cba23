"""GPU parity of the decode GEMV (kernels.zig:118-158 linearQuantized through
Matrix.apply) against the oracle on the same seeded inputs: within 1e-3
relative (f32 accumulate; see util.assert_close for the exact bound)."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def run_linear(ctx, fmt, scales, data, rows, cols, x, tokens):
    handle = ctx.matrix_upload(fmt, rows, cols, scales, data)
    xb = ctx.to_device(np.ascontiguousarray(x, np.float32))
    ob = ctx.buffer(tokens * rows * 4)
    ctx.linear(handle, xb.ptr, cols, tokens, ob.ptr)
    out = ob.download(np.float32).reshape(tokens, rows)
    ctx.matrix_release(handle)
    xb.free()
    ob.free()
    return out


def check(ctx, fmt, w, x, tokens, what):
    rows, cols = w.shape
    scales, data = o.quantize_rows(fmt, w)
    expected = o.linear_quantized(fmt, scales, data, rows, cols, x, tokens)
    actual = run_linear(ctx, fmt, scales, data, rows, cols, x, tokens)
    return assert_close(actual, expected, what=what)


def test_harness_matmul_q4_case(ctx):
    # harness.mjs:189-259: tokens 24, rows 64, cols 256, weights and
    # activations N(0,1) from seeds 0x5eed0002 / 0x5eed0001.
    x = o.normal(24 * 256, 0x5EED0001)
    w = o.normal(64 * 256, 0x5EED0002).reshape(64, 256)
    check(ctx, o.Q4, w, x, 24, "harness matmul_q4")


def test_config1_q8_gemv(ctx):
    # W [1024 x 3072] ~ 0.02 N(0,1) seed 0, x [3072] the next draws.
    draws = o.normal(1024 * 3072 + 3072, 0)
    w = (draws[:1024 * 3072] * np.float32(0.02)).reshape(1024, 3072)
    x = draws[1024 * 3072:]
    check(ctx, o.Q8, w, x, 1, "config 1 q8 [1024x3072]")


SHAPES_06B = {"q": (2048, 1024), "k": (1024, 1024), "v": (1024, 1024), "o": (1024, 2048),
              "gate": (3072, 1024), "up": (3072, 1024), "down": (1024, 3072)}


@pytest.mark.parametrize("name", list(SHAPES_06B))
def test_config2_q4_gemv_shapes(ctx, name):
    rows, cols = SHAPES_06B[name]
    stream = list(SHAPES_06B).index(name) + 1
    w = o.normal(rows * cols, 1, stream, 0.02).reshape(rows, cols)
    x = o.normal(cols, 1, 100 + stream)
    check(ctx, o.Q4, w, x, 1, f"config 2 {name} [{rows}x{cols}]")


def test_config2_lm_head_synthetic_on_device(ctx):
    # lm_head [151936 x 1024]: generated and quantized on the device, checked
    # bit exact against the oracle's planes, then the product.
    rows, cols, seed, stream = 151936, 1024, 1, 8
    handle = ctx.matrix_synthetic(qa.FORMAT_Q4, rows, cols, seed, stream, 0.02)
    s_ref, d_ref = o.quantize_rows(o.Q4, o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols))
    sp, dp = ctx.matrix_planes(handle)
    s_gpu = np.empty(s_ref.size, np.uint8)
    d_gpu = np.empty(d_ref.size, np.uint8)
    ctx._check(ctx.lib.qwh_download(ctx.handle, s_gpu.ctypes.data, sp, s_gpu.nbytes))
    ctx._check(ctx.lib.qwh_download(ctx.handle, d_gpu.ctypes.data, dp, d_gpu.nbytes))
    assert o.fnv1a64(s_gpu) == o.fnv1a64(s_ref) and o.fnv1a64(d_gpu) == o.fnv1a64(d_ref)
    x = o.normal(cols, 1, 108)
    expected = o.linear_quantized(o.Q4, s_ref, d_ref, rows, cols, x, 1)
    xb = ctx.to_device(x)
    ob = ctx.buffer(rows * 4)
    ctx.linear(handle, xb.ptr, cols, 1, ob.ptr)
    actual = ob.download(np.float32).reshape(1, rows)
    assert_close(actual, expected, what="lm_head [151936x1024]")
    ctx.matrix_release(handle)
    xb.free()
    ob.free()


@pytest.mark.parametrize("rows,cols,tokens", [
    (1001, 1024, 1),    # odd rows with two rows per wavefront group
    (33, 64, 1),        # 32 rows per group, partial group
    (70, 128, 2),
    (257, 256, 3),
    (129, 512, 1),
    (64, 1536, 1),      # three slices per lane, four rows per group
    (96, 4096, 1),      # two slices per lane
    (130, 6144, 2),     # three slices per lane, one row per group
    (48, 192, 1),       # generic path (odd slice count)
    (40, 448, 2),       # generic path
    (1, 2048, 5),
])
def test_q4_gemv_edge_shapes(ctx, rows, cols, tokens):
    w = o.normal(rows * cols, 5, rows, 0.02).reshape(rows, cols)
    x = o.normal(tokens * cols, 5, 1000 + cols)
    check(ctx, o.Q4, w, x, tokens, f"q4 {rows}x{cols} tokens {tokens}")


@pytest.mark.parametrize("rows,cols,tokens", [
    (4096, 2048, 16),   # configs[4] q|k|v rows at batch 16
    (2048, 6144, 16),   # configs[4] down projection at batch 16
    (100, 1024, 7),     # partial row tile, partial token tile
    (17, 64, 17),       # one group per row (three idle wavefronts), two token tiles
    (33, 192, 33),      # three groups, three token tiles
    (64, 256, 2),
    (40, 10240, 3),     # K past 8192: activation prep stretch by stretch, two units per wave
    (65600, 256, 2),    # over 4096 row tiles: four tiles per workgroup
    (65600, 128, 3),    # two groups: chunks of 2 groups, two row tiles per wavefront
    (300, 1024, 40),    # K split into 4 slices over three token tiles, partial row block
    (896, 896, 390),    # the 0.6B audio tower's projection: 14 groups in chunks of 2, 25 token tiles
    (3584, 896, 40),    # its ffn_in
    (100, 384, 17),     # six groups in chunks of 2, split into slices
])
def test_q4_batch_gemv(ctx, rows, cols, tokens):
    # Two or more tokens run on the matrix-core kernel.
    w = o.normal(rows * cols, 8, rows, 0.02).reshape(rows, cols)
    x = o.normal(tokens * cols, 8, 2000 + cols)
    check(ctx, o.Q4, w, x, tokens, f"q4 batch {rows}x{cols} tokens {tokens}")


def test_q4_batch_awkward_values(ctx):
    # Per token: an all-zero group, a huge dynamic range inside a group,
    # tiny values; plus an all-zero token and a zero weight row.
    rows, cols, tokens = 48, 512, 5
    w = o.normal(rows * cols, 9, 0, 0.02).reshape(rows, cols)
    w[7] = 0.0
    w[8, :64] = np.float32(-7.5)
    x = o.normal(tokens * cols, 9, 1).reshape(tokens, cols)
    x[0, :64] = 0.0
    x[1, 64] = np.float32(3e4)
    x[1, 65] = np.float32(1e-12)
    x[2, 128:192] = np.float32(1e-30)
    x[3] = 0.0
    x[4, 200] = np.float32(-1e-3)
    scales, data = o.quantize_rows(o.Q4, w)
    expected = o.linear_quantized(o.Q4, scales, data, rows, cols, x.reshape(-1), tokens)
    actual = run_linear(ctx, o.Q4, scales, data, rows, cols, x.reshape(-1), tokens)
    assert np.all(actual[:, 7] == 0.0) and np.all(actual[3] == 0.0)
    assert_close(actual, expected, what="batch awkward values")


@pytest.mark.parametrize("rows,cols,tokens", [(1001, 1024, 1), (33, 64, 2), (130, 6144, 1), (48, 192, 1)])
def test_q8_gemv_edge_shapes(ctx, rows, cols, tokens):
    w = o.normal(rows * cols, 6, rows, 0.02).reshape(rows, cols)
    x = o.normal(tokens * cols, 6, 1000 + cols)
    check(ctx, o.Q8, w, x, tokens, f"q8 {rows}x{cols} tokens {tokens}")


@pytest.mark.parametrize("rows,cols,tokens", [
    # (Planes on 16-byte boundaries up to 32768 rows: the staged form.)
    (1001, 1024, 1),    # one slice per lane, 32 lanes per row (0.6B shapes)
    (130, 2048, 2),     # one slice, 64 lanes per row
    (64, 512, 1),       # 16 lanes per row
    (96, 4096, 1),      # two slices per lane
    (70, 3072, 3),      # three slices, 32 lanes per row
    (33, 6144, 1),      # three slices, 64 lanes per row; the widest encoded row
    (48, 320, 2),       # generic kernel (five groups)
    (17, 896, 1),       # generic kernel (seven slices per lane group)
    (1, 64, 4),
])
def test_q5_gemv_shapes(ctx, rows, cols, tokens):
    # quant.zig:253-269 planes (fifth bits in their own 8 bytes per group).
    w = o.normal(rows * cols, 10, rows, 0.02).reshape(rows, cols)
    x = o.normal(tokens * cols, 10, 1000 + cols)
    check(ctx, o.Q5, w, x, tokens, f"q5 {rows}x{cols} tokens {tokens}")


@pytest.mark.parametrize("rows,cols", [(32770, 1024), (32800, 3072)])
def test_q5_gemv_per_lane_form(ctx, rows, cols):
    # Past 32768 rows a q5 matrix keeps the per-lane loads (the staged whole
    # pieces measured slower on the long lm_head stream): one and three
    # slices per lane, rows past a whole unit.
    w = o.normal(rows * cols, 14, rows, 0.02).reshape(rows, cols)
    x = o.normal(cols, 14, 3000 + cols)
    check(ctx, o.Q5, w, x, 1, f"q5 {rows}x{cols}")


@pytest.mark.parametrize("rows,cols,tokens", [
    (256, 2048, 16),     # one 16-token tile, K split into slices (partial sums + reduce)
    (100, 1024, 17),     # two token tiles, a partial row tile
    (8240, 1024, 3),     # two row tiles per wavefront
    (2048, 6144, 40),    # three token tiles, the widest row
    (896, 896, 390),     # the 0.6B audio tower's 896-wide rows (14 groups: chunks of 2 groups), 30 s of steps
    (3584, 896, 390),    # its ffn_in
    (896, 3584, 390),    # its ffn_out (56 groups: chunks of 4)
])
def test_q5_multi_token_on_matrix_cores(ctx, rows, cols, tokens):
    # Several tokens over q5 codes (K a multiple of 256): u - 16 expanded to
    # signed bytes with the fifth bits, one v_mfma_i32_16x16x64_i8 per
    # activation digit plane, W streamed once per 16 tokens.
    w = o.normal(rows * cols, 13, rows, 0.02).reshape(rows, cols)
    w[rows // 2, :64] = np.float32(-1.0)   # codes at the bottom of the range
    w[rows // 2, 64:128] = np.float32(1.0)
    x = o.normal(tokens * cols, 13, 2000 + cols)
    check(ctx, o.Q5, w, x, tokens, f"q5 {rows}x{cols} tokens {tokens}")


def test_q5_gemv_awkward_values(ctx):
    # Codes at both ends (-16 and 15 in one group), a zero row, a zero group
    # of activations, a huge dynamic range inside one chunk.
    rows, cols, tokens = 40, 1024, 2
    w = o.normal(rows * cols, 11, 0, 0.02).reshape(rows, cols)
    w[3] = 0.0
    w[5, :32] = np.float32(-1.0)
    w[5, 32:64] = np.float32(1.0)
    w[6, ::2] = np.float32(0.5)
    x = o.normal(tokens * cols, 11, 1).reshape(tokens, cols)
    x[0, 64:128] = 0.0
    x[1, 7] = np.float32(2e4)
    x[1, 8] = np.float32(-3e-9)
    scales, data = o.quantize_rows(o.Q5, w)
    expected = o.linear_quantized(o.Q5, scales, data, rows, cols, x.reshape(-1), tokens)
    actual = run_linear(ctx, o.Q5, scales, data, rows, cols, x.reshape(-1), tokens)
    assert np.all(actual[:, 3] == 0.0)
    assert_close(actual, expected, what="q5 awkward values")


def test_q5_lm_head_synthetic_on_device(ctx):
    # The 0.6B lm_head shape in q5, generated and quantized on the device.
    rows, cols, seed, stream = 151936, 1024, 1, 9
    handle = ctx.matrix_synthetic(qa.FORMAT_Q5, rows, cols, seed, stream, 0.02)
    s_ref, d_ref = o.quantize_rows(o.Q5, o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols))
    sp, dp = ctx.matrix_planes(handle)
    d_gpu = np.empty(d_ref.size, np.uint8)
    ctx._check(ctx.lib.qwh_download(ctx.handle, d_gpu.ctypes.data, dp, d_gpu.nbytes))
    assert o.fnv1a64(d_gpu) == o.fnv1a64(d_ref)
    x = o.normal(cols, 1, 109)
    expected = o.linear_quantized(o.Q5, s_ref, d_ref, rows, cols, x, 1)
    xb = ctx.to_device(x)
    ob = ctx.buffer(rows * 4)
    ctx.linear(handle, xb.ptr, cols, 1, ob.ptr)
    actual = ob.download(np.float32).reshape(1, rows)
    assert_close(actual, expected, what="q5 lm_head [151936x1024]")
    ctx.matrix_release(handle)
    xb.free()
    ob.free()


def test_q5_gemv_rejects_unbuilt_width(ctx):
    # Rows wider than the in-LDS activation encoding (6144) are not built.
    rows, cols = 2, 6208
    w = o.normal(rows * cols, 12, 0, 0.02).reshape(rows, cols)
    scales, data = o.quantize_rows(o.Q5, w)
    with pytest.raises(qa.QwhError) as err:
        run_linear(ctx, o.Q5, scales, data, rows, cols, o.normal(cols, 12, 1), 1)
    assert err.value.status == -3


def test_q4_gemv_awkward_values(ctx):
    # Zero rows, a subnormal-scale row, activations with zero chunks and a
    # huge dynamic range inside one chunk.
    rows, cols = 64, 1024
    w = o.normal(rows * cols, 7, 0, 0.02).reshape(rows, cols)
    w[3] = 0.0
    w[4] = 0.0
    w[4, 10] = np.float32(1e-6)
    w[5, :64] = np.float32(7.0)
    x = o.normal(cols, 7, 1)
    x[:32] = 0.0
    x[64] = np.float32(1e3)
    x[65] = np.float32(1e-20)
    x[96:128] = np.float32(1e-30)
    scales, data = o.quantize_rows(o.Q4, w)
    expected = o.linear_quantized(o.Q4, scales, data, rows, cols, x, 1)
    actual = run_linear(ctx, o.Q4, scales, data, rows, cols, x, 1)
    assert actual[0, 3] == 0.0
    assert_close(actual, expected, what="awkward values")


def test_prepared_activations_match_linear(ctx):
    # One prepared activation row feeding q, k and v (decoder.zig:174-176).
    cols = 2048
    x = o.normal(cols, 15, 0)
    xb = ctx.to_device(x)
    prep = ctx.buffer(ctx.activation_bytes(cols, 1))
    ctx.activation_prepare(xb.ptr, cols, 1, prep.ptr)
    for rows, stream in ((2048, 1), (1024, 2), (1024, 3)):
        w = o.normal(rows * cols, 15, stream, 0.02).reshape(rows, cols)
        scales, data = o.quantize_rows(o.Q4, w)
        handle = ctx.matrix_upload(o.Q4, rows, cols, scales, data)
        a = ctx.buffer(rows * 4)
        b = ctx.buffer(rows * 4)
        ctx.linear(handle, xb.ptr, cols, 1, a.ptr)
        ctx.linear_prepared(handle, prep.ptr, 1, b.ptr)
        assert np.array_equal(a.download(np.float32), b.download(np.float32))
        ctx.matrix_release(handle)
        a.free()
        b.free()
    xb.free()
    prep.free()


def test_linear_rejects_shape_mismatch(ctx):
    w = o.normal(64 * 128, 8).reshape(64, 128)
    scales, data = o.quantize_rows(o.Q4, w)
    handle = ctx.matrix_upload(o.Q4, 64, 128, scales, data)
    xb = ctx.buffer(256 * 4)
    ob = ctx.buffer(64 * 4)
    with pytest.raises(qa.QwhError) as err:
        ctx.linear(handle, xb.ptr, 256, 1, ob.ptr)
    assert err.value.status == -7
    with pytest.raises(qa.QwhError) as err:
        ctx.matrix_upload(o.Q4, 64, 128, scales[:-2], data)
    assert err.value.status == -7
    ctx.matrix_release(handle)
    xb.free()
    ob.free()


@pytest.mark.parametrize("rows,cols,tokens", [
    (4096, 2048, 16),     # the 1.7B q|k|v block at batch 16 (split form, 8 slices)
    (12288, 2048, 3),     # gate|up
    (2048, 6144, 33),     # down, three token tiles
    (1001, 1024, 2),      # rows not a multiple of the tile
    (130, 320, 5),        # five groups: the unsplit matrix-core form
    (64, 448, 17),        # seven groups, two token tiles
    (896, 896, 390),      # fourteen groups in chunks of 2
    (300, 384, 5),        # six groups in chunks of 2
])
def test_q8_multi_token_on_matrix_cores(ctx, rows, cols, tokens):
    # kernels.zig:118-158 with tokens > 1 over q8 weights (the audio tower's
    # and the batched decoder's products): one pass over the codes per 16
    # tokens; codes at both ends of the range in the first row.
    w = o.normal(rows * cols, 15, rows, 0.02).reshape(rows, cols)
    w[0, :64] = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    x = o.normal(tokens * cols, 15, 2000 + cols)
    check(ctx, o.Q8, w, x, tokens, f"q8 {rows}x{cols} tokens {tokens}")
