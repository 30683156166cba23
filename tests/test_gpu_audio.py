"""GPU parity of the audio tower path (model.zig:646-735): LayerNorm, bias /
GELU epilogues, windowed encoder attention (kernels.zig:429-484), one whole
audio layer and the projector, each through the C ABI against the oracle.

Tolerances: the reference harness's (harness.mjs:83-86: gelu 1e-5, layernorm
1e-4) for the elementwise parts; attention 1e-4 relative; whole layers and the
projector 1e-3 relative (the north-star bound for quantized linears, f32
accumulate) with the output's rms as the floor near zero."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, normal, quantized_matrix

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def test_layer_norm_harness_case(ctx):
    # harness.mjs:129-131 / :344-349: 32 rows x 256, eps 1e-5.
    rows, cols, eps = 32, 256, 1e-5
    x = normal(rows * cols, 0x5EED0009) * np.float32(2.0) + np.float32(0.5)
    w = normal(cols, 0x5EED000A)
    b = normal(cols, 0x5EED000B)
    expected = o.layer_norm(x, w, b, cols, eps)
    xb, wb, bb = ctx.to_device(x), ctx.to_device(w), ctx.to_device(b)
    ob = ctx.buffer(x.nbytes)
    ctx.layer_norm(ob.ptr, xb.ptr, wb.ptr, bb.ptr, cols, rows, eps)
    assert_close(ob.download(np.float32), expected, rtol=1e-4, atol_rms=1e-4, what="layer norm")
    # In place (kernels.zig:242-255 layerNorm), width past one workgroup's stride.
    cols = 3584
    x = normal(7 * cols, 12)
    w, b = normal(cols, 13), normal(cols, 14)
    xb, wb, bb = ctx.to_device(x), ctx.to_device(w), ctx.to_device(b)
    ctx.layer_norm(xb.ptr, xb.ptr, wb.ptr, bb.ptr, cols, 7, eps)
    assert_close(xb.download(np.float32), o.layer_norm(x, w, b, cols, eps), rtol=1e-4, atol_rms=1e-4,
                 what="layer norm in place")


def test_add_bias_and_gelu(ctx):
    # kernels.zig:1162-1171 known answer.
    xb = ctx.to_device(np.array([1, 2, 3, 4], np.float32))
    bb = ctx.to_device(np.array([10, 20], np.float32))
    ctx.add_bias(xb.ptr, bb.ptr, 2, 2)
    assert xb.download(np.float32).tolist() == [11.0, 22.0, 13.0, 24.0]
    # harness.mjs:128, :343: 1024 values, seed 0x5eed0008, 1e-5.
    g = normal(1024, 0x5EED0008) * np.float32(3.0)
    gb = ctx.to_device(g)
    ctx.gelu(gb.ptr, g.size)
    assert_close(gb.download(np.float32), o.gelu_array(g), rtol=1e-5, atol_rms=1e-5, what="gelu")


def pad_head(rows, head_dim):
    out = np.zeros((len(rows), head_dim), np.float32)
    for i, r in enumerate(rows):
        out[i, :len(r)] = r
    return out.reshape(-1)


def test_audio_attention_known_answers(ctx):
    # kernels.zig:1043-1078 with each head row padded by zeros to head_dim 32
    # (the dot products and value rows are unchanged by the padding).
    hd = 32
    q = pad_head([[1, 0], [0, 1]], hd)
    v = pad_head([[5, 6], [7, 8]], hd)
    qb, vb = ctx.to_device(q), ctx.to_device(v)
    ob = ctx.to_device(np.zeros(2 * hd, np.float32))
    ctx.audio_attention_window(ob.ptr, hd, qb.ptr, hd, qb.ptr, hd, vb.ptr, hd, 0, 1, 1, hd)
    out = ob.download(np.float32).reshape(2, hd)
    assert np.allclose(out[0, :2], [5, 6], atol=1e-6) and np.all(out[1] == 0)
    ob = ctx.to_device(np.zeros(2 * hd, np.float32))
    ctx.audio_attention_window(ob.ptr, hd, qb.ptr, hd, qb.ptr, hd, vb.ptr, hd, 1, 1, 1, hd)
    out = ob.download(np.float32).reshape(2, hd)
    assert np.all(out[0] == 0) and np.allclose(out[1, :2], [7, 8], atol=1e-6)
    q = pad_head([[1, 0], [1, 0]], hd)
    v = pad_head([[2, 0], [4, 0]], hd)
    qb, vb = ctx.to_device(q), ctx.to_device(v)
    ob = ctx.to_device(np.zeros(2 * hd, np.float32))
    ctx.audio_attention_window(ob.ptr, hd, qb.ptr, hd, qb.ptr, hd, vb.ptr, hd, 0, 2, 1, hd)
    out = ob.download(np.float32).reshape(2, hd)
    assert abs(out[0, 0] - 3.0) <= 1e-5 and abs(out[1, 0] - 3.0) <= 1e-5
    with pytest.raises(qa.QwhError):
        ctx.audio_attention_window(ob.ptr, 2, qb.ptr, 2, qb.ptr, 2, vb.ptr, 2, 0, 1, 1, 2)


@pytest.mark.parametrize("steps,window,heads,head_dim", [
    (390, 104, 14, 64),   # Qwen3-ASR-0.6B audio tower at 30 s (tensor_names.zig:416-419)
    (37, 13, 3, 128),
    (70, 70, 2, 32),
    (200, 64, 4, 64),     # windows of exactly one key chunk
    (300, 150, 2, 128),   # three key chunks per window at the widest head
    (5, 1, 2, 64),        # windows of one step: each output is its own value row
])
def test_audio_attention_windows(ctx, steps, window, heads, head_dim):
    width = heads * head_dim
    # model.zig:792-822: q | k | v packed in one buffer with row stride 3 * width.
    qkv = normal(steps * 3 * width, 31, steps)
    expected = np.zeros(steps * width, np.float32)
    start = 0
    while start < steps:
        length = min(window, steps - start)
        o.audio_attention_window(expected, qkv, qkv[width:], qkv[2 * width:], (width, 3 * width, 3 * width, 3 * width),
                                 start, length, heads, head_dim)
        start += length
    qb = ctx.to_device(qkv)
    ob = ctx.buffer(steps * width * 4)
    ctx.audio_attention(ob.ptr, width, qb.ptr, qb.ptr + 4 * width, qb.ptr + 8 * width, 3 * width, steps, window,
                        heads, head_dim)
    assert_close(ob.download(np.float32), expected, rtol=1e-4, atol_rms=1e-4, what="audio attention")


def test_audio_attention_window_inside_a_larger_buffer(ctx):
    # One window [50, 110) of a 160-step buffer with distinct row strides:
    # rows outside the window keep their contents.
    steps, heads, hd = 160, 3, 64
    width = heads * hd
    q = normal(steps * (width + 64), 61)
    k = normal(steps * (width + 128), 62)
    v = normal(steps * width, 63)
    out0 = normal(steps * (width + 32), 64)
    strides = (width + 32, width + 64, width + 128, width)
    expected = out0.copy()
    o.audio_attention_window(expected, q, k, v, strides, 50, 60, heads, hd)
    qb, kb, vb, ob = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), ctx.to_device(out0)
    ctx.audio_attention_window(ob.ptr, strides[0], qb.ptr, strides[1], kb.ptr, strides[2], vb.ptr, strides[3], 50, 60,
                               heads, hd)
    got = ob.download(np.float32)
    rows = got.reshape(steps, -1)
    assert np.array_equal(rows[:50], out0.reshape(steps, -1)[:50])
    assert np.array_equal(rows[110:], out0.reshape(steps, -1)[110:])
    assert_close(got, expected, rtol=1e-4, atol_rms=1e-4, what="audio attention window")


def layer_matrix(fmt, rows, cols, seed, stream):
    """(fmt, scales, data) of seeded 0.05 N(0,1) weights: quantized planes, or
    f16 bits (scales None) for the converter's unquantized form."""
    if fmt == qa.FORMAT_F16:
        return fmt, None, normal(rows * cols, seed, stream, 0.05).astype(np.float16).view(np.uint16)
    _, scales, data = quantized_matrix(fmt, rows, cols, seed, stream, 0.05)
    return fmt, scales, data


def make_layer(ctx, fmt, d_model, ffn_dim, seed):
    host, dev, keep = {}, {}, []
    for i, (name, rows, cols) in enumerate((("q", d_model, d_model), ("k", d_model, d_model), ("v", d_model, d_model),
                                             ("o", d_model, d_model), ("ffn_in", ffn_dim, d_model),
                                             ("ffn_out", d_model, ffn_dim))):
        host[name] = layer_matrix(fmt, rows, cols, seed, i)
        dev[name] = ctx.matrix_upload(fmt, rows, cols, host[name][1], host[name][2])
        host[name + "_bias"] = normal(rows, seed, 10 + i, 0.1)
    for j, name in enumerate(("attention_norm", "final_norm")):
        host[name + "_weight"] = np.float32(1.0) + normal(d_model, seed, 20 + j, 0.1)
        host[name + "_bias"] = normal(d_model, seed, 30 + j, 0.1)
    weights = qa.AudioLayerWeights()
    for name in qa.AudioLayerWeights.MATRICES:
        setattr(weights, name, dev[name])
    for name in qa.AudioLayerWeights.VECTORS:
        buf = ctx.to_device(host[name])
        keep.append(buf)
        setattr(weights, name, buf.ptr)
    return host, weights, keep


@pytest.mark.parametrize("fmt,d_model,heads,ffn_dim,steps,window", [
    (qa.FORMAT_Q4, 256, 4, 512, 50, 13),
    (qa.FORMAT_Q8, 256, 4, 512, 50, 13),
    (qa.FORMAT_Q5, 256, 4, 512, 21, 8),
    (qa.FORMAT_Q4, 256, 4, 512, 1, 8),  # one step: the per-linear path, separate bias and norm kernels
    (qa.FORMAT_Q4, 896, 14, 3584, 390, 104),  # Qwen3-ASR-0.6B audio layer, 30 s
    (qa.FORMAT_Q5, 896, 14, 3584, 390, 104),  # the same in q5 (896-wide rows: 14 groups)
    (qa.FORMAT_F16, 256, 4, 512, 50, 13),     # f16 weights: the dense GEMV per linear
    (qa.FORMAT_F16, 896, 14, 3584, 390, 104),
])
def test_audio_layer(ctx, fmt, d_model, heads, ffn_dim, steps, window):
    eps = 1e-5
    host, weights, keep = make_layer(ctx, fmt, d_model, ffn_dim, 40 + fmt)
    enc = normal(steps * d_model, 41, fmt)
    expected = o.audio_layer(enc, host, steps, d_model, heads, ffn_dim, window, eps)
    eb = ctx.to_device(enc)
    ctx.audio_layer(weights, eb.ptr, steps, d_model, heads, ffn_dim, window, eps)
    assert_close(eb.download(np.float32), expected, rtol=1e-3, atol_rms=1e-3, what=f"audio layer fmt {fmt}")
    # Two layers in a row on the same context scratch: the second reads the first's output.
    expected2 = o.audio_layer(expected, host, steps, d_model, heads, ffn_dim, window, eps)
    ctx.audio_layer(weights, eb.ptr, steps, d_model, heads, ffn_dim, window, eps)
    assert_close(eb.download(np.float32), expected2, rtol=1e-3, atol_rms=1e-3, what="second audio layer")


def test_audio_layer_rejects_mismatched_matrices(ctx):
    host, weights, keep = make_layer(ctx, qa.FORMAT_Q4, 256, 512, 3)
    eb = ctx.to_device(np.zeros(4 * 256, np.float32))
    with pytest.raises(qa.QwhError, match="shape_mismatch"):
        ctx.audio_layer(weights, eb.ptr, 4, 256, 4, 1024, 4, 1e-5)


@pytest.mark.parametrize("fmt", [qa.FORMAT_Q4, qa.FORMAT_F16])
def test_audio_projector(ctx, fmt):
    # model.zig:707-735 at the 0.6B shapes: d_model 896 -> text hidden 1024, 390 steps.
    steps, d_model, hidden = 390, 896, 1024
    _, s_in, d_in = layer_matrix(fmt, d_model, d_model, 50, 0)
    _, s_out, d_out = layer_matrix(fmt, hidden, d_model, 50, 1)
    b_in, b_out = normal(d_model, 50, 2, 0.1), normal(hidden, 50, 3, 0.1)
    enc = normal(steps * d_model, 51)
    expected = o.audio_projector(enc, (fmt, s_in, d_in), b_in, (fmt, s_out, d_out), b_out, steps, d_model, hidden)
    m_in = ctx.matrix_upload(fmt, d_model, d_model, s_in, d_in)
    m_out = ctx.matrix_upload(fmt, hidden, d_model, s_out, d_out)
    bi, bo, eb = ctx.to_device(b_in), ctx.to_device(b_out), ctx.to_device(enc)
    ob = ctx.buffer(steps * hidden * 4)
    ctx.audio_projector(m_in, bi.ptr, m_out, bo.ptr, eb.ptr, steps, ob.ptr)
    assert_close(ob.download(np.float32), expected, rtol=1e-3, atol_rms=1e-3, what="audio projector")


def test_audio_attention_rejects_too_many_windows(ctx):
    # 70000 windows of one step exceed the launch's 65535 window rows: refused
    # before any device work. The buffer covers every row the call names, so
    # a regression of the guard fails the assertion instead of reading past
    # the allocation.
    buf = ctx.buffer(70000 * 32 * 4)
    with pytest.raises(qa.QwhError, match="limit_exceeded"):
        ctx.audio_attention(buf.ptr, 32, buf.ptr, buf.ptr, buf.ptr, 32, 70000, 1, 1, 32)
    buf.free()
