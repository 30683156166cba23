"""The whole device path of a transcription, chained as transcribe.zig:120-219
runs it, against the oracle at a small shape: the convolution front end
(model.zig:509-644), the audio layers (model.zig:646-693) and their final
LayerNorm, the projector (model.zig:707-735), the prompt prefill with the
projected rows in the audio pads (decoder.zig:308-333) and greedy steps
(decoder.zig:336-339).

Each stage's output is compared with the oracle's on the same input (the
encoder rows and projected rows within 1e-3); the decoder part then runs on
the device's projected rows on both sides, teacher-forced as in
tests/test_gpu_prefill.py, so the token ids compare the prefill and the steps
rather than the audio stages' rounding."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from test_gpu_audio import make_layer
from test_gpu_frontend import frontend_weights
from test_gpu_prefill import PAD, make_pair, prompt, teacher_forced
from util import assert_close, normal, quantized_matrix

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

DECODER = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
               max_positions=128, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("fmt", [qa.FORMAT_Q8, qa.FORMAT_Q4])
def test_clip_end_to_end(ctx, fmt):
    mel_bins, frames, n_window, downsample = 32, 200, 50, 32   # two chunks of 100 frames: 26 steps
    d_model, heads, ffn_dim, layers, window, eps = 128, 2, 256, 2, 13, 1e-5
    hidden = DECODER["hidden"]
    keep, release = [], []
    fhost, fw, fkeep = frontend_weights(ctx, 91, downsample, mel_bins, d_model, fmt)
    keep += fkeep
    release.append(fw.conv_out)
    tower = [make_layer(ctx, fmt, d_model, ffn_dim, 92 + i) for i in range(layers)]
    for _, w, k in tower:
        keep += k
        release += [getattr(w, name) for name in qa.AudioLayerWeights.MATRICES]
    ln_w, ln_b = np.float32(1.0) + normal(d_model, 93, 0, 0.1), normal(d_model, 93, 1, 0.1)
    _, pis, pid = quantized_matrix(fmt, d_model, d_model, 94, 0, 0.05)
    _, pos_, pod = quantized_matrix(fmt, hidden, d_model, 94, 1, 0.05)
    p_in_b, p_out_b = normal(d_model, 94, 2, 0.1), normal(hidden, 94, 3, 0.1)
    p_in = ctx.matrix_upload(fmt, d_model, d_model, pis, pid)
    p_out = ctx.matrix_upload(fmt, hidden, d_model, pos_, pod)
    release += [p_in, p_out]
    log_mel = normal(mel_bins * frames, 95)
    gpu = ref = None
    try:
        # The audio stages, each against the oracle on the device's input.
        mel = ctx.to_device(log_mel)
        keep.append(mel)
        want = o.audio_frontend(log_mel.reshape(mel_bins, frames), mel_bins, frames, n_window, fhost, downsample,
                                d_model)
        steps = want.shape[0]
        enc = ctx.buffer(steps * d_model * 4)
        keep.append(enc)
        assert ctx.audio_frontend(fw, mel.ptr, mel_bins, frames, n_window, downsample, d_model, enc.ptr,
                                  steps) == steps == 26
        assert_close(enc.download(np.float32).reshape(steps, d_model), want, what="front end")
        for i, (host, w, _) in enumerate(tower):
            x = enc.download(np.float32)
            ctx.audio_layer(w, enc.ptr, steps, d_model, heads, ffn_dim, window, eps)
            assert_close(enc.download(np.float32), o.audio_layer(x, host, steps, d_model, heads, ffn_dim, window, eps),
                         what=f"audio layer {i}")
        x = enc.download(np.float32)
        lw, lb = ctx.to_device(ln_w), ctx.to_device(ln_b)
        pib, pob = ctx.to_device(p_in_b), ctx.to_device(p_out_b)
        keep += [lw, lb, pib, pob]
        ctx.layer_norm(enc.ptr, enc.ptr, lw.ptr, lb.ptr, d_model, steps, eps)
        normed = o.layer_norm(x, ln_w, ln_b, d_model, eps)
        assert_close(enc.download(np.float32), normed, rtol=1e-4, atol_rms=1e-4, what="final layer norm")
        proj = ctx.buffer(steps * hidden * 4)
        keep.append(proj)
        ctx.audio_projector(p_in, pib.ptr, p_out, pob.ptr, enc.ptr, steps, proj.ptr)
        rows = proj.download(np.float32).reshape(steps, hidden)
        assert_close(rows, o.audio_projector(enc.download(np.float32), (fmt, pis, pid), p_in_b, (fmt, pos_, pod),
                                             p_out_b, steps, d_model, hidden).reshape(steps, hidden),
                     what="projector")

        # The prompt with one pad per encoder step, prefilled from the device's
        # projected rows; then greedy steps.
        gpu, ref = make_pair(ctx, DECODER, 1, 96, fmt, "q8", [0])
        tokens = prompt(steps + 9, DECODER["vocab"], range(4, 4 + steps), 97)
        got = gpu.prefill(0, tokens, PAD, proj.ptr, steps)
        want_id = teacher_forced(ctx, gpu, ref, 0, tokens, rows, 0, DECODER, "q8")
        assert_close(gpu.logits(0), ref.logits(0), what="prefill logits (teacher-forced)")
        if got != want_id:
            expected = ref.logits(0)
            assert float(np.max(expected)) - float(expected[got]) <= 2e-3 * float(np.abs(expected).max()), (got, want_id)
        token = want_id
        for step in range(8):
            ids = gpu.step([token])
            nxt = ref.step(0, token)
            assert int(ids[0]) == nxt, step
            token = nxt
        assert gpu.position(0) == steps + 9 + 8
    finally:
        for d in (gpu, ref):
            if d is not None:
                d.close()
        for m in release:
            ctx.matrix_release(m)
        for b in keep:
            b.free()
