"""CPU checks that pin the oracle's audio tower restatements (oracle/qwref.c
audio glue, oracle/oracle.py audio_layer / audio_projector).

Pins, in order: the reference's own known answers (math.zig:134-171 erf and
gelu, kernels.zig:1043-1078 windowed attention, kernels.zig:1162-1171
addBias), then float64 brute force written independently in numpy / scipy
(layer norm, windowed softmax attention, a whole layer over dequantized
weights), chosen so that a dropped bias, a wrong residual, a transposed
projection or a window that leaks fails.
"""
import math

import numpy as np
import pytest
from scipy.special import erf as erf64

from oracle import oracle as o
from util import normal


@pytest.mark.parametrize("x,expected", [
    (0.0, 0.0), (0.1, 0.1124629160182849), (0.5, 0.5204998778130465), (1.0, 0.8427007929497149),
    (1.5, 0.9661051464753107), (2.0, 0.9953222650189527), (3.0, 0.9999779095030014),
    (4.0, 0.9999999845827421), (-0.75, -0.7111556336535151), (-2.5, -0.999593047982555),
])
def test_erf_known_answers(x, expected):
    # math.zig:134-152, same tolerance.
    assert abs(o.erf(x) - expected) <= 2e-7


def test_erf_odd_and_saturates():
    # math.zig:154-162.
    assert o.erf(0.0) == 0.0
    assert abs(o.erf(-40.0) + 1.0) <= 1e-6 and abs(o.erf(40.0) - 1.0) <= 1e-6
    for x in np.arange(-6.0, 6.0001, 0.25):
        assert abs(-o.erf(-x) - o.erf(x)) <= 1e-7


def test_gelu_known_answers_and_definition():
    # math.zig:164-171.
    assert abs(o.gelu(0.0)) <= 1e-7
    assert abs(o.gelu(1.0) - 0.84134475) <= 1e-6
    assert abs(o.gelu(-1.0) + 0.15865525) <= 1e-6
    assert abs(o.gelu(-10.0)) <= 1e-6
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    exact = 0.5 * x.astype(np.float64) * (1.0 + erf64(x.astype(np.float64) / math.sqrt(2.0)))
    got = o.gelu_array(x).astype(np.float64)
    # The fit's erf error is below 1.2e-7; what is left is f32 rounding of x.
    assert np.max(np.abs(got - exact) / (1.0 + np.abs(x))) < 2e-7


def test_add_bias_known_answer():
    # kernels.zig:1162-1171.
    out = o.add_bias(np.array([1, 2, 3, 4], np.float32), np.array([10, 20], np.float32), 2, 2)
    assert out.tolist() == [11.0, 22.0, 13.0, 24.0]
    with pytest.raises(ValueError):
        o.add_bias(np.zeros(5, np.float32), np.zeros(2, np.float32), 2, 2)


def test_layer_norm_against_float64():
    rng = np.random.default_rng(11)
    rows, cols, eps = 32, 256, 1e-5  # harness.mjs:129-131 layernorm shape
    x = (rng.standard_normal((rows, cols)) * 3 + 0.7).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    got = o.layer_norm(x, w, b, cols, eps).reshape(rows, cols)
    xd = x.astype(np.float64)
    mean = xd.mean(axis=1, keepdims=True)
    var = ((xd - mean) ** 2).mean(axis=1, keepdims=True)
    want = (xd - mean) / np.sqrt(var + eps) * w + b
    assert np.max(np.abs(got - want)) <= 1e-4 + 1e-4 * np.max(np.abs(want))
    # A constant row has zero variance: the output is the bias exactly.
    const = o.layer_norm(np.full(cols, 2.5, np.float32), w, b, cols, eps)
    assert np.array_equal(const, b)


def test_windowed_attention_known_answers():
    # kernels.zig:1043-1066: two windows of length one, each output its own value.
    q = np.array([1, 0, 0, 1], np.float32)
    k = q.copy()
    v = np.array([5, 6, 7, 8], np.float32)
    out = np.zeros(4, np.float32)
    o.audio_attention_window(out, q, k, v, (2, 2, 2, 2), 0, 1, 1, 2)
    assert np.allclose(out, [5, 6, 0, 0], atol=1e-6)
    out[:] = 0
    o.audio_attention_window(out, q, k, v, (2, 2, 2, 2), 1, 1, 1, 2)
    assert np.allclose(out, [0, 0, 7, 8], atol=1e-6)
    # kernels.zig:1068-1078: identical keys average the values.
    q = np.array([1, 0, 1, 0], np.float32)
    v = np.array([2, 0, 4, 0], np.float32)
    out = np.zeros(4, np.float32)
    o.audio_attention_window(out, q, q, v, (2, 2, 2, 2), 0, 2, 1, 2)
    assert abs(out[0] - 3.0) <= 1e-5 and abs(out[2] - 3.0) <= 1e-5


def windowed_attention_f64(q, k, v, steps, window, heads, head_dim):
    q, k, v = (a.reshape(steps, heads, head_dim).astype(np.float64) for a in (q, k, v))
    out = np.zeros((steps, heads, head_dim))
    for start in range(0, steps, window):
        end = min(start + window, steps)
        for h in range(heads):
            s = q[start:end, h] @ k[start:end, h].T / math.sqrt(head_dim)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[start:end, h] = p @ v[start:end, h]
    return out.reshape(-1)


@pytest.mark.parametrize("steps,window,heads,head_dim", [(37, 13, 3, 64), (50, 50, 2, 32), (9, 4, 1, 128)])
def test_windowed_attention_against_float64(steps, window, heads, head_dim):
    rng = np.random.default_rng(steps)
    q, k, v = (rng.standard_normal(steps * heads * head_dim).astype(np.float32) for _ in range(3))
    got = o.audio_attention(q, k, v, steps, window, heads, head_dim)
    want = windowed_attention_f64(q, k, v, steps, window, heads, head_dim)
    assert np.max(np.abs(got - want)) <= 1e-5 * (1 + np.max(np.abs(want)))


def make_audio_layer(seed, d_model, ffn_dim, fmt=o.Q4):
    rng = np.random.default_rng(seed)
    layer = {}
    for name, rows, cols in (("q", d_model, d_model), ("k", d_model, d_model), ("v", d_model, d_model),
                             ("o", d_model, d_model), ("ffn_in", ffn_dim, d_model), ("ffn_out", d_model, ffn_dim)):
        w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        scales, data = o.quantize_rows(fmt, w)
        layer[name] = (fmt, scales, data)
        layer[name + "_bias"] = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    for name in ("attention_norm", "final_norm"):
        layer[name + "_weight"] = (1 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
        layer[name + "_bias"] = (0.1 * rng.standard_normal(d_model)).astype(np.float32)
    return layer


def test_audio_layer_against_float64():
    d_model, heads, ffn_dim, steps, window, eps = 128, 2, 256, 20, 7, 1e-5
    layer = make_audio_layer(5, d_model, ffn_dim)
    enc = np.random.default_rng(6).standard_normal(steps * d_model).astype(np.float32)
    got = o.audio_layer(enc, layer, steps, d_model, heads, ffn_dim, window, eps)

    def dense(name):
        fmt, scales, data = layer[name]
        rows = layer[name + "_bias"].size
        return o.dequantize_rows(fmt, scales, data, rows, scales.size * 32 // rows).astype(np.float64)

    def ln(x, prefix):
        mean = x.mean(axis=1, keepdims=True)
        var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
        return (x - mean) / np.sqrt(var + eps) * layer[prefix + "_weight"] + layer[prefix + "_bias"]

    x = enc.reshape(steps, d_model).astype(np.float64)
    n = ln(x, "attention_norm")
    q, k, v = (n @ dense(p).T + layer[p + "_bias"] for p in ("q", "k", "v"))
    att = windowed_attention_f64(q, k, v, steps, window, heads, d_model // heads).reshape(steps, d_model)
    x = x + att @ dense("o").T + layer["o_bias"]
    n = ln(x, "final_norm")
    h = n @ dense("ffn_in").T + layer["ffn_in_bias"]
    h = 0.5 * h * (1 + erf64(h / math.sqrt(2)))
    x = x + h @ dense("ffn_out").T + layer["ffn_out_bias"]
    want = x.reshape(-1)
    assert np.max(np.abs(got - want)) <= 1e-4 * (1 + np.max(np.abs(want)))


# ---------------------------------------------------------------- convolution front end
def _f16(values):
    return np.array([o.to_f16(float(v)) for v in np.asarray(values, np.float32).reshape(-1)], np.uint16)


def test_conv_centre_tap_known_answer():
    # kernels.zig:973-997: a 3x3 input, one output channel whose kernel picks
    # the centre: the outputs are gelu of input positions (0,0), (0,2), (2,0),
    # (2,2).
    w = _f16([0, 0, 0, 0, 1, 0, 0, 0, 0])
    out = o.conv3x3s2_gelu(np.arange(1, 10, dtype=np.float32), w, [0.0], 1, 1, 3, 3).reshape(-1)
    for got, x in zip(out, (1.0, 3.0, 7.0, 9.0)):
        assert abs(got - o.gelu(x)) <= 1e-5


def test_conv_reduces_over_channels_in_weight_order():
    # kernels.zig:999-1041: channel zero's centre tap plus channel one's
    # top-left tap, which lands inside the input only for the last output
    # position (reading 50): gelu(1), gelu(3), gelu(7), gelu(9 + 50).
    w = _f16([0, 0, 0, 0, 1, 0, 0, 0, 0] + [1, 0, 0, 0, 0, 0, 0, 0, 0])
    x = np.concatenate([np.arange(1, 10), 10 * np.arange(1, 10)]).astype(np.float32)
    out = o.conv3x3s2_gelu(x, w, [0.0], 1, 2, 3, 3).reshape(-1)
    for got, v in zip(out, (1.0, 3.0, 7.0, 59.0)):
        assert abs(got - o.gelu(v)) <= 1e-5


def _conv_f64(x, w, b, cout, cin, h, wd):
    oh, ow = (h - 1) // 2 + 1, (wd - 1) // 2 + 1
    xp = np.zeros((cin, h + 2, wd + 2))
    xp[:, 1:h + 1, 1:wd + 1] = x.reshape(cin, h, wd)
    w = w.reshape(cout, cin, 3, 3)
    out = np.zeros((cout, oh, ow))
    for i in range(3):
        for j in range(3):
            patch = xp[:, i:i + 2 * oh:2, j:j + 2 * ow:2]
            out += np.einsum("oc,chw->ohw", w[:, :, i, j], patch)
    out += np.asarray(b, np.float64)[:, None, None]
    return out


@pytest.mark.parametrize("cout,cin,h,w", [(5, 3, 9, 11), (4, 1, 16, 8), (2, 7, 4, 5), (3, 2, 1, 1), (6, 6, 2, 3)])
def test_conv_against_f64_brute_force(cout, cin, h, w):
    x = normal(cin * h * w, 51, cin)
    wv = normal(cout * cin * 9, 52, cout, 0.3)
    wb = _f16(wv)
    wf = np.array([o.from_f16(int(v)) for v in wb], np.float64)
    b = normal(cout, 53, 0, 0.1)
    got = o.conv3x3s2_gelu(x, wb, b, cout, cin, h, w)
    pre = _conv_f64(x.astype(np.float64), wf, b, cout, cin, h, w)
    want = 0.5 * pre * (1.0 + erf64(pre / math.sqrt(2.0)))
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_post_convolution_steps():
    # model_config.zig:431 and the three (n - 1) / 2 + 1 halvings.
    assert o.post_convolution_steps(3000) == 375
    assert o.post_convolution_steps(0) == 0
    assert o.post_convolution_steps(1) == 1
    assert o.post_convolution_steps(100) == 13
    assert o.post_convolution_steps(128) == 16


def test_sinusoidal_position_known_answers():
    # model.zig:1136-1170.
    row = o.add_sinusoidal_position(np.zeros(64, np.float32), 0)
    assert np.all(row[:32] == 0.0) and np.allclose(row[32:], 1.0, atol=1e-6)
    row = o.add_sinusoidal_position(np.zeros(64, np.float32), 1)
    assert np.all(np.abs(row) <= 1.0) and np.all(np.isfinite(row))
    assert abs(row[0] - math.sin(1.0)) <= 1e-6 and abs(row[32] - math.cos(1.0)) <= 1e-6
    assert abs(row[1]) > abs(row[30]) and abs(row[62]) > abs(row[32])
    assert abs(row[62] - 1.0) <= 1e-4
    seeded = o.add_sinusoidal_position(np.full(64, 0.25, np.float32), 0)
    assert np.allclose(seeded[:32], 0.25, atol=1e-6) and np.allclose(seeded[32:], 1.25, atol=1e-6)
    # Against float64 at a later step and another width.
    row = o.add_sinusoidal_position(np.zeros(896, np.float32), 12)
    half = 448
    inv = np.exp(-math.log(10000.0) / (half - 1) * np.arange(half))
    assert np.allclose(row, np.concatenate([np.sin(12 * inv), np.cos(12 * inv)]), atol=1e-7)


def _frontend_weights(seed, downsample, mel_bins, d_model, fmt=o.Q4):
    bins = o.post_convolution_steps(mel_bins)
    w = {}
    for i, (name, cin) in enumerate((("conv1", 1), ("conv2", downsample), ("conv3", downsample))):
        w[name + "_weight"] = _f16(normal(downsample * cin * 9, seed, 10 + i, 0.4))
        w[name + "_bias"] = normal(downsample, seed, 20 + i, 0.1)
    features = downsample * bins
    vals = normal(d_model * features, seed, 30, 0.05).reshape(d_model, features)
    s, d = o.quantize_rows(fmt, vals)
    w["conv_out"] = (fmt, s, d)
    return w


def _frontend_f64(log_mel, mel_bins, frames, n_window, w, downsample, d_model):
    """model.zig:509-644 in float64 (the reference's erf fit replaced by the
    exact erf; chunks, flatten, projection and positions written out)."""
    chunk = 2 * n_window
    bins = o.post_convolution_steps(mel_bins)
    fmt, s, d = w["conv_out"]
    proj = o.dequantize_rows(fmt, s, d, d_model, downsample * bins).astype(np.float64)
    rows = []
    for start in range(0, frames, chunk):
        valid = min(frames - start, chunk)
        x = np.zeros((mel_bins, chunk))
        x[:, :valid] = log_mel[:, start:start + valid]
        h, wd, cin = mel_bins, chunk, 1
        for stage in ("conv1", "conv2", "conv3"):
            wf = np.array([o.from_f16(int(v)) for v in w[stage + "_weight"]], np.float64)
            pre = _conv_f64(x, wf, w[stage + "_bias"], downsample, cin, h, wd)
            x = 0.5 * pre * (1.0 + erf64(pre / math.sqrt(2.0)))
            h, wd, cin = (h - 1) // 2 + 1, (wd - 1) // 2 + 1, downsample
        half = d_model // 2
        inv = np.exp(-math.log(10000.0) / (half - 1) * np.arange(half))
        for step in range(min(o.post_convolution_steps(chunk), o.post_convolution_steps(valid))):
            row = proj @ x[:, :, step].reshape(-1)
            rows.append(row + np.concatenate([np.sin(step * inv), np.cos(step * inv)]))
    return np.stack(rows)


def test_frontend_composition_against_f64():
    # Two full chunks and a ragged third (3 frames), so the zero-filled tail
    # and the per-chunk step count both matter.
    mel_bins, n_window, downsample, d_model, frames = 32, 4, 16, 8, 19  # 16 x 4 = 64 features
    w = _frontend_weights(61, downsample, mel_bins, d_model)
    log_mel = normal(mel_bins * frames, 62).reshape(mel_bins, frames)
    got = o.audio_frontend(log_mel, mel_bins, frames, n_window, w, downsample, d_model)
    want = _frontend_f64(log_mel, mel_bins, frames, n_window, w, downsample, d_model)
    expected_steps = 2 * o.post_convolution_steps(8) + o.post_convolution_steps(3)
    assert got.shape == (expected_steps, d_model) == want.shape
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.abs(want).max())
