"""GPU parity of f16 / f32 weight matrices (kernels.zig:160-206 Matrix .f16 /
.f32 arms: linearF16 :82-112, linearF32 :54-80) against the oracle on the
same seeded inputs. Below eight tokens, and for f32 weights, both sides
form the same exact f32 products (an f16 weight widens exactly) and only the
summation order differs (the reference's four-lane dotF32 against a
wavefront reduction or MFMA sums). From eight tokens the f16 form multiplies
each activation as two f16 halves carrying it to 2^-22 of its 64-value
step's largest magnitude. The bound is tight either way:
|a - r| <= 1e-4 |r| + 1e-4 rms(r) (util.assert_close)."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from oracle import shard as sh
from util import assert_close

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

TOL = dict(rtol=1e-4, atol_rms=1e-4)


def weights(fmt, rows, cols, seed, stream=0):
    """Seeded weights as the matrix stores them (f16 bits or f32 values)."""
    w = o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols)
    return w.astype(np.float16).view(np.uint16) if fmt == qa.FORMAT_F16 else w


def expected(fmt, w, x, tokens):
    return o.linear_f16(w, x, tokens) if fmt == qa.FORMAT_F16 else o.linear_f32(w, x, tokens)


def run(ctx, handle, x, cols, tokens, rows):
    xb = ctx.to_device(np.ascontiguousarray(x, np.float32))
    ob = ctx.buffer(tokens * rows * 4)
    try:
        ctx.linear(handle, xb.ptr, cols, tokens, ob.ptr)
        return ob.download(np.float32).reshape(tokens, rows)
    finally:
        xb.free()
        ob.free()


FORMATS = [qa.FORMAT_F16, qa.FORMAT_F32]
SHAPES = [  # (rows, cols, tokens): four, two or one token per workgroup
    (1024, 1024, 1),    # decoder k / v (0.6B)
    (3072, 1024, 1),    # gate / up (0.6B)
    (1024, 3072, 5),    # down: a group of four and a group of one
    (1024, 2048, 19),   # four groups of four and a tail of three
    (96, 2048, 3),      # a group of four, one past the last
    (40, 6144, 9),      # rows too wide for four tokens: groups of two
    (64, 12000, 2),     # rows too wide for two: one token per workgroup
    (24, 40956, 2),     # the widest rows (160 KiB of LDS)
    (257, 67, 3),       # rows that are not whole 16-byte slices
    (7, 1, 9),          # one column
    # Eight tokens and more: the matrix cores, 16 x 16 tiles.
    (1000, 1024, 8),    # half a token tile
    (2048, 2048, 16),   # one whole tile of tokens
    (333, 3072, 33),    # rows and tokens past whole tiles
    (64, 128, 40),      # the fewest K-steps the form takes (four per wavefront)
    (96, 6144, 200),    # rows too wide for a token group of four
    # f16 rows of whole 64-value steps, up to 16 tokens: K split over the
    # wavefronts, 1, 2, 3 or 4 row tiles per workgroup by the 16 x 16 tiles
    # per CU (up to 1, 2, 3, more; the counts below are for 256 CUs).
    (520, 4096, 16),    # one row tile, a half tile of rows past the last
    (6000, 512, 16),    # two row tiles, a half tile past the last
    (12008, 256, 9),    # three row tiles, the last workgroup's 8 rows of 48
    (16400, 512, 16),   # four row tiles, one past the last
    (32800, 256, 12),   # four row tiles, two and a half past the last, four tokens short
    # More than 16 tokens: each wavefront on its own rows, T token tiles per
    # workgroup (R row tiles per wavefront, W wavefronts).
    (2000, 1024, 136),  # R 1, T 2, W 4; a half row tile and half a token tile past the last
    (4100, 1024, 40),   # R 1, T 2, W 8; four rows and 24 tokens short of the last workgroup
    (8200, 1024, 130),  # R 2, T 4, W 8; rows and tokens past whole workgroups
    (65600, 256, 20),   # R 1, T 4, W 8: the lm_head form at 17..127 tokens
    (300, 1056, 12),    # f16 rows of 16.5 steps: the f32 matrix-core form
]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols,tokens", SHAPES)
def test_dense_linear(ctx, fmt, rows, cols, tokens):
    w = weights(fmt, rows, cols, 31, rows + cols)
    x = o.normal(tokens * cols, 32, tokens)
    handle = ctx.matrix_upload(fmt, rows, cols, None, w)
    try:
        actual = run(ctx, handle, x, cols, tokens, rows)
    finally:
        ctx.matrix_release(handle)
    assert_close(actual, expected(fmt, w, x, tokens), what=f"format {fmt} {rows}x{cols} tokens {tokens}", **TOL)


@pytest.mark.parametrize("fmt", FORMATS)
def test_dense_activation_range(ctx, fmt):
    # Tokens of very different magnitudes in one batch, past the f16 range
    # and far below it: the matrix-core forms scale each token's activations
    # on their own (the f16 form splits them into two f16 halves per step).
    rows, cols, tokens = 256, 2048, 16
    w = weights(fmt, rows, cols, 41, 7)
    x = o.normal(tokens * cols, 42, tokens).reshape(tokens, cols)
    x[0] *= 6.0e4          # past the f16 range
    x[1] *= 1.0e-30        # far below it
    x[2, ::64] *= 1.0e6    # one large value per step
    x[3, :1000] = 0.0      # steps of zeros
    handle = ctx.matrix_upload(fmt, rows, cols, None, w)
    try:
        actual = run(ctx, handle, x.reshape(-1), cols, tokens, rows)
    finally:
        ctx.matrix_release(handle)
    ref = expected(fmt, w, x.reshape(-1), tokens)
    for t in range(tokens):
        assert_close(actual[t], ref[t], what=f"format {fmt} token {t}", **TOL)


@pytest.mark.parametrize("fmt", FORMATS)
def test_dense_non_finite_activations(ctx, fmt):
    # An inf activation makes its token's sums +-inf (NaN where the weight
    # is 0), a NaN makes them NaN, as f32 products and sums do; the other
    # tokens are untouched.
    rows, cols, tokens = 64, 1024, 16
    w = weights(fmt, rows, cols, 43, 9)
    wf = w.view(np.float16).astype(np.float32) if fmt == qa.FORMAT_F16 else w
    wf[:, 5][:3] = (0.5, -0.25, 0.0)
    w = wf.astype(np.float16).view(np.uint16) if fmt == qa.FORMAT_F16 else wf
    x = o.normal(tokens * cols, 44, tokens).reshape(tokens, cols)
    x[3, 5] = np.inf
    x[7, 100] = np.nan
    handle = ctx.matrix_upload(fmt, rows, cols, None, w)
    try:
        actual = run(ctx, handle, x.reshape(-1), cols, tokens, rows)
    finally:
        ctx.matrix_release(handle)
    col5 = (w.view(np.float16).astype(np.float32) if fmt == qa.FORMAT_F16 else w)[:, 5]
    assert np.all(np.isposinf(actual[3][col5 > 0])) and np.all(np.isneginf(actual[3][col5 < 0]))
    assert np.all(np.isnan(actual[3][col5 == 0])) and (col5 == 0).any()
    assert np.all(np.isnan(actual[7]))
    finite = [t for t in range(tokens) if t not in (3, 7)]
    xf = x.copy()
    xf[3] = 0.0
    xf[7] = 0.0
    ref = expected(fmt, w, xf.reshape(-1), tokens)
    assert_close(actual[finite], ref[finite], what=f"format {fmt} finite tokens", **TOL)


def test_dense_matrix_dispatch_ones(ctx):
    # kernels.zig:932-948: 2 x 64 ones against ones give exactly 64.
    x = np.ones(64, np.float32)
    for fmt, w in ((qa.FORMAT_F32, np.ones((2, 64), np.float32)),
                   (qa.FORMAT_F16, np.full((2, 64), o.to_f16(1.0), np.uint16))):
        handle = ctx.matrix_upload(fmt, 2, 64, None, w)
        try:
            assert run(ctx, handle, x, 64, 1, 2).tolist() == [[64.0, 64.0]]
        finally:
            ctx.matrix_release(handle)


def test_dense_exact_weights_agree(ctx):
    # kernels.zig:863-876: f16 and f32 layers of exactly representable
    # weights give the same outputs; every partial sum is exact in f32, so
    # the device's summation order cannot change a bit.
    x = np.array([0.5, -1.5, 2.0, 1.0, -0.5, 0.25, 1.0, -2.0], np.float32)
    w = np.array([[2.0, 0.5, -1.0, 0.0], [1.0, 1.0, 0.5, -2.0]], np.float32)
    bits = np.array([[o.to_f16(float(v)) for v in row] for row in w], np.uint16)
    for fmt, data in ((qa.FORMAT_F32, w), (qa.FORMAT_F16, bits)):
        handle = ctx.matrix_upload(fmt, 2, 4, None, data)
        try:
            assert run(ctx, handle, x, 4, 2, 2).tolist() == [[-1.75, -2.0], [-1.875, 4.25]], fmt
        finally:
            ctx.matrix_release(handle)


@pytest.mark.parametrize("fmt,rows,cols,tokens", [
    (qa.FORMAT_Q4, 4, 128, 3),      # kernels.zig:878-931's own case
    (qa.FORMAT_Q4, 512, 2048, 1),   # the q4 GEMV
    (qa.FORMAT_Q4, 512, 2048, 5),   # the matrix-core batch GEMV
    (qa.FORMAT_Q5, 300, 1024, 1),   # the byte-plane GEMV
    (qa.FORMAT_Q5, 256, 2048, 4),
    (qa.FORMAT_Q8, 300, 1024, 1),
    (qa.FORMAT_Q8, 256, 2048, 3),
])
def test_quantized_matches_dequantized_dense(ctx, fmt, rows, cols, tokens):
    # kernels.zig:878-931 on the device: a quantized matrix and the f32
    # matrix of its dequantized values (exact: an integer code times an f16
    # scale) give the same products, through two independent kernels.
    if (rows, cols) == (4, 128):
        idx = np.arange(rows * cols, dtype=np.float32)
        values = (np.cos(idx * np.float32(0.07)) * np.float32(1.25)).reshape(rows, cols).astype(np.float32)
        xi = np.arange(tokens * cols, dtype=np.float32)
        x = (np.sin(xi * np.float32(0.11)) * np.float32(0.75)).astype(np.float32)
    else:
        values = o.normal(rows * cols, 38, fmt, 0.05).reshape(rows, cols)
        x = o.normal(tokens * cols, 39, fmt)
    scales, data = o.quantize_rows(fmt, values)
    dense = o.dequantize_rows(fmt, scales, data, rows, cols).astype(np.float32)
    hq = ctx.matrix_upload(fmt, rows, cols, scales, data)
    hd = ctx.matrix_upload(qa.FORMAT_F32, rows, cols, None, dense)
    try:
        got_q = run(ctx, hq, x, cols, tokens, rows)
        got_d = run(ctx, hd, x, cols, tokens, rows)
    finally:
        ctx.matrix_release(hq)
        ctx.matrix_release(hd)
    assert_close(got_q, got_d, what=f"format {fmt} against its dequantized f32 matrix", **TOL)
    assert_close(got_d, o.linear_f32(dense, x, tokens), what="dense against the oracle", **TOL)


@pytest.mark.parametrize("fmt,offset", [(qa.FORMAT_F16, 2), (qa.FORMAT_F16, 6), (qa.FORMAT_F32, 4)])
def test_dense_wrap_unaligned_rows(ctx, fmt, offset):
    # Elements aligned to their size but not to 16 bytes take the
    # element-wise form.
    rows, cols, tokens = 96, 512, 3
    w = weights(fmt, rows, cols, 33)
    x = o.normal(tokens * cols, 34)
    buf = ctx.buffer(w.nbytes + 16)
    buf.upload(w, offset)
    handle = ctx.matrix_wrap(fmt, rows, cols, 0, buf.ptr + offset)
    try:
        actual = run(ctx, handle, x, cols, tokens, rows)
    finally:
        ctx.matrix_release(handle)
        buf.free()
    assert_close(actual, expected(fmt, w, x, tokens), what=f"wrapped format {fmt} at +{offset}", **TOL)


@pytest.mark.parametrize("fmt", FORMATS)
def test_dense_synthetic(ctx, fmt):
    # f32(N(0,1)) * scale from the synthetic generator, rounded to f16 (RNE,
    # half_float.zig:12-16) for f16 matrices: bit exact against the oracle's
    # generator and numpy's f16 rounding.
    rows, cols, seed, stream, scale = 300, 1000, 9, 4, 0.05
    handle = ctx.matrix_synthetic(fmt, rows, cols, seed, stream, scale)
    try:
        scales_dev, data_dev = ctx.matrix_planes(handle)
        assert scales_dev is None
        values = o.normal(rows * cols, seed, stream, scale).reshape(rows, cols)
        if fmt == qa.FORMAT_F16:
            want = values.astype(np.float16).view(np.uint16)
            sample = np.array([o.to_f16(float(v)) for v in values.flat[:512]], np.uint16)
            assert np.array_equal(sample, want.flat[:512])
        else:
            want = values
        got = np.empty_like(want)
        ctx._check(ctx.lib.qwh_download(ctx.handle, got.ctypes.data, data_dev, got.nbytes))
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
        x = o.normal(2 * cols, 35)
        actual = run(ctx, handle, x, cols, 2, rows)
    finally:
        ctx.matrix_release(handle)
    assert_close(actual, expected(fmt, want, x, 2), what=f"synthetic format {fmt}", **TOL)


def test_dense_shard_matrices(ctx):
    # model.zig:92-96 Binding.matrix: f32 / f16 tensors of rank 2 are
    # matrices over their elements in place; vectors are not matrices.
    specs = [(sh.KIND_DECODER_Q, 1, qa.FORMAT_F16, 200, 1024), (sh.KIND_DECODER_FFN_DOWN, 1, qa.FORMAT_F32, 130, 520)]
    tensors, mats = [], {}
    for i, (kind, layer, fmt, rows, cols) in enumerate(specs):
        w = weights(fmt, rows, cols, 36, i)
        mats[(kind, layer)] = (fmt, rows, cols, w)
        tensors.append(dict(kind=kind, layer=layer, format=fmt, dims=(rows, cols), payload=w.tobytes()))
    tensors.append(dict(kind=sh.KIND_DECODER_FINAL_NORM, layer=0, format=sh.F16, dims=(1024,),
                        payload=np.ones(1024, np.float16).tobytes()))
    shard = ctx.shard_load(sh.build(tensors))
    handles = []
    try:
        for (kind, layer), (fmt, rows, cols, w) in mats.items():
            m = ctx.shard_matrix(shard, kind, layer)
            handles.append(m)
            x = o.normal(3 * cols, 37, kind)
            assert_close(run(ctx, m, x, cols, 3, rows), expected(fmt, w, x, 3), what=f"shard kind {kind}", **TOL)
        with pytest.raises(qa.QwhError) as err:
            ctx.shard_matrix(shard, sh.KIND_DECODER_FINAL_NORM, 0)
        assert err.value.status == sh.NOT_FOUND
    finally:
        for m in handles:
            ctx.matrix_release(m)
        ctx.shard_release(shard)


def test_dense_errors(ctx):
    f16 = np.zeros((4, 64), np.uint16)
    # A scale plane for an element format.
    with pytest.raises(qa.QwhError) as err:
        ctx.matrix_upload(qa.FORMAT_F16, 4, 64, np.zeros(2, np.uint8), f16)
    assert err.value.status == -7
    # Elements not aligned to their size.
    buf = ctx.buffer(1024)
    try:
        with pytest.raises(qa.QwhError) as err:
            ctx.matrix_wrap(qa.FORMAT_F16, 4, 64, 0, buf.ptr + 1)
        assert err.value.status == -1
        with pytest.raises(qa.QwhError) as err:
            ctx.matrix_wrap(qa.FORMAT_F32, 4, 64, 0, buf.ptr + 2)
        assert err.value.status == -1
        # No columns.
        with pytest.raises(qa.QwhError) as err:
            ctx.matrix_wrap(qa.FORMAT_F32, 4, 0, 0, buf.ptr)
        assert err.value.status == -7
        # Device quantization only writes quantized planes.
        with pytest.raises(qa.QwhError) as err:
            ctx.quantize_rows(qa.FORMAT_F16, buf.ptr, 1, 64, buf.ptr, buf.ptr)
        assert err.value.status == -3
    finally:
        buf.free()
    # Rows wider than one token's activations in LDS.
    wide = 40957
    handle = ctx.matrix_upload(qa.FORMAT_F32, 1, wide, None, np.zeros(wide, np.float32))
    xb = ctx.buffer(wide * 4)
    ob = ctx.buffer(64)
    try:
        with pytest.raises(qa.QwhError) as err:
            ctx.linear(handle, xb.ptr, wide, 1, ob.ptr)
        assert err.value.status == -3
        with pytest.raises(qa.QwhError) as err:
            ctx.linear_bf16(handle, xb.ptr, wide, 1, ob.ptr)
        assert err.value.status == -3
    finally:
        ctx.matrix_release(handle)
        xb.free()
        ob.free()
