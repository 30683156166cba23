"""GPU parity of the audio tower's convolution front end (kernels.zig:302-427
conv3x3Stride2Gelu; model.zig:509-644 convolveAndPack / projectConvStep with
:751-763 addSinusoidalPosition) against the oracle: the reference's
known answers, the convolution at the Qwen3-ASR stage shapes and at ragged
edges, and the whole front end at the Qwen3-ASR-0.6B shape (128 mel bins,
chunks of 100 frames, 480 channels, d_model 896) over two whole chunks and a
ragged one. 1e-3 relative, the output rms as the floor near zero."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, normal

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))


def f16(values):
    return np.array([o.to_f16(float(v)) for v in np.asarray(values, np.float32).reshape(-1)], np.uint16)


def f16_fast(values):
    # numpy's float16 cast is round-to-nearest-even, as half_float.toF16
    # (test_oracle pins the two against each other).
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def run_conv(ctx, x, w, b, batch, cout, cin, h, wd):
    oh, ow = (h - 1) // 2 + 1, (wd - 1) // 2 + 1
    bufs = [ctx.to_device(np.ascontiguousarray(v)) for v in (x, w, b)]
    out = ctx.buffer(batch * cout * oh * ow * 4)
    ctx.conv3x3s2_gelu(out.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, batch, cout, cin, h, wd)
    got = out.download(np.float32).reshape(batch, cout, oh, ow)
    for v in bufs + [out]:
        v.free()
    return got


def test_conv_known_answers(ctx):
    # kernels.zig:973-1041: the centre tap of a 3x3 input; two channels whose
    # second one's top-left tap reaches the input only at the last position.
    got = run_conv(ctx, np.arange(1, 10, dtype=np.float32), f16([0, 0, 0, 0, 1, 0, 0, 0, 0]),
                   np.zeros(1, np.float32), 1, 1, 1, 3, 3).reshape(-1)
    assert np.allclose(got, [o.gelu(v) for v in (1.0, 3.0, 7.0, 9.0)], atol=1e-5)
    x = np.concatenate([np.arange(1, 10), 10 * np.arange(1, 10)]).astype(np.float32)
    got = run_conv(ctx, x, f16([0, 0, 0, 0, 1, 0, 0, 0, 0] + [1, 0, 0, 0, 0, 0, 0, 0, 0]), np.zeros(1, np.float32),
                   1, 1, 2, 3, 3).reshape(-1)
    assert np.allclose(got, [o.gelu(v) for v in (1.0, 3.0, 7.0, 59.0)], atol=1e-5)


@pytest.mark.parametrize("batch,cout,cin,h,w", [
    (2, 480, 1, 128, 100),    # conv1 of Qwen3-ASR
    (1, 480, 480, 64, 50),    # conv2
    (2, 480, 480, 32, 25),    # conv3
    (3, 70, 13, 17, 9),       # channel counts off the tiles, odd planes
    (1, 5, 3, 1, 1),          # a single input position
    (2, 65, 9, 2, 31),
    # The matrix-core form (input channels a multiple of 16): output
    # channels and positions off its 128 x 32 tiles, a one-row output, a
    # two-column output (a 32-position tile spans 16 output rows), and a
    # plane too wide for its LDS patch (the f32 kernel).
    (3, 70, 16, 17, 9),
    (2, 130, 32, 2, 31),
    (1, 200, 48, 40, 3),
    (1, 8, 16, 4, 300),
])
def test_conv_against_oracle(ctx, batch, cout, cin, h, w):
    x = normal(batch * cin * h * w, 71, cin)
    wb = f16_fast(normal(cout * cin * 9, 72, cout, 1.0 / np.sqrt(9 * cin)))
    b = normal(cout, 73, 0, 0.1)
    got = run_conv(ctx, x, wb, b, batch, cout, cin, h, w)
    for i in range(batch):
        want = o.conv3x3s2_gelu(x[i * cin * h * w:(i + 1) * cin * h * w], wb, b, cout, cin, h, w)
        assert_close(got[i], want, what=f"conv {cout}x{cin} {h}x{w} image {i}")


def frontend_weights(ctx, seed, downsample, mel_bins, d_model, fmt):
    bins = o.post_convolution_steps(mel_bins)
    host, keep = {}, []
    for i, (name, cin) in enumerate((("conv1", 1), ("conv2", downsample), ("conv3", downsample))):
        host[name + "_weight"] = f16_fast(normal(downsample * cin * 9, seed, 10 + i, 1.0 / np.sqrt(9 * cin)))
        host[name + "_bias"] = normal(downsample, seed, 20 + i, 0.1)
    features = downsample * bins
    values = normal(d_model * features, seed, 30, 0.02).reshape(d_model, features)
    if fmt == o.F16:  # the converter's unquantized form: f16 elements, no scales
        s, d = None, values.astype(np.float16).view(np.uint16)
    else:
        s, d = o.quantize_rows(fmt, values)
    host["conv_out"] = (fmt, s, d)
    w = qa.AudioFrontendWeights()
    for name in ("conv1_weight", "conv2_weight", "conv3_weight", "conv1_bias", "conv2_bias", "conv3_bias"):
        buf = ctx.to_device(host[name])
        keep.append(buf)
        setattr(w, name, buf.ptr)
    w.conv_out = ctx.matrix_upload(fmt, d_model, features, s, d)
    return host, w, keep


@pytest.mark.parametrize("mel_bins,frames,n_window,downsample,d_model,fmt", [
    (128, 250, 50, 480, 896, o.Q4),    # Qwen3-ASR-0.6B: two whole chunks and 50 frames
    (32, 19, 4, 16, 64, o.Q8),         # ragged third chunk of 3 frames, q8 projection
    (64, 8, 4, 64, 128, o.Q5),         # exactly one chunk, q5 projection
    (128, 250, 50, 480, 896, o.F16),   # the 0.6B shape with an f16 projection (7680-wide rows)
])
def test_frontend_against_oracle(ctx, mel_bins, frames, n_window, downsample, d_model, fmt):
    host, w, keep = frontend_weights(ctx, 81, downsample, mel_bins, d_model, fmt)
    log_mel = normal(mel_bins * frames, 82)
    want = o.audio_frontend(log_mel.reshape(mel_bins, frames), mel_bins, frames, n_window, host, downsample, d_model)
    mel = ctx.to_device(log_mel)
    rows = want.shape[0]
    enc = ctx.buffer((rows + 1) * d_model * 4)
    try:
        steps = ctx.audio_frontend(w, mel.ptr, mel_bins, frames, n_window, downsample, d_model, enc.ptr, rows + 1)
        assert steps == rows
        got = enc.download(np.float32)[: rows * d_model].reshape(rows, d_model)
        assert_close(got, want, what=f"front end {mel_bins} bins {frames} frames")
        with pytest.raises(qa.QwhError, match="limit_exceeded"):
            ctx.audio_frontend(w, mel.ptr, mel_bins, frames, n_window, downsample, d_model, enc.ptr, rows - 1)
    finally:
        ctx.matrix_release(w.conv_out)
        for b in keep + [mel, enc]:
            b.free()
