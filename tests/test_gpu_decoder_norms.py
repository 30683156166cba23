"""GPU parity of the decoder step with learned-looking RMSNorm weights
(decoder.zig:165-172 attention norm, :180-193 per-head q / k norms, :259-265
ffn norm, :277-284 final norm) against the oracle holding the same vectors.
Every device path that reads a norm weight is covered: the fused RMSNorm GEMV
prologue (batch 1), the attention kernels' q / k norms, the batch prep's
x * w with the GEMV's per-token 1 / rms (batch 3: one token tile; batch 18:
two), the separate rmsnorm kernel (unfused), and the unsplit batch GEMV."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, random_norms, set_norms

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
            max_positions=64, eps=1e-6, theta=1e6)
ODD = dict(hidden=320, layers=2, heads=5, kv_heads=5, head_dim=64, ffn=448, vocab=500,
           max_positions=64, eps=1e-6, theta=1e6)


def make_pair(ctx, config, batch, seed, norm_seed):
    gpu = qa.Decoder(ctx, batch=batch, **config)
    ref = o.Decoder(seed, batch, **config)
    gpu.init_synthetic(seed)
    norms = random_norms(config, norm_seed)
    set_norms(gpu, norms, config["layers"])
    set_norms(ref, norms, config["layers"])
    for b in range(batch):
        n = (5 * b + 3) % 29
        gpu.prefill_random(b, n, seed)
        ref.prefill_random(b, n)
    return gpu, ref


@pytest.mark.parametrize("batch,config,env", [
    (1, TINY, ()),                                             # fused RMSNorm GEMV prologue
    (3, TINY, ()),                                             # prep x * w, per-token 1 / rms in the MFMA GEMV
    (18, TINY, ()),                                            # two token tiles
    (3, TINY, ("QWH_DECODER_NO_SPLIT",)),                      # unsplit forms add their own slices
    (3, ODD, ()),                                              # unsplit kernel, factor in its epilogue
    (2, TINY, ("QWH_DECODER_PER_TOKEN", "QWH_DECODER_UNFUSED")),  # separate rmsnorm kernel
])
def test_norm_weights_teacher_forced_and_greedy(ctx, batch, config, env, monkeypatch):
    for name in env:
        monkeypatch.setenv(name, "1")
    seed = 17
    gpu, ref = make_pair(ctx, config, batch, seed, 41)
    try:
        vocab = config["vocab"]
        for step in range(5):
            tokens = [(step * 53 + b * 97 + 11) % vocab for b in range(batch)]
            gpu.forward(tokens, True)
            for b in range(batch):
                ref.forward(b, tokens[b], True)
                assert_close(gpu.logits(b), ref.logits(b), what=f"{env} batch {batch} step {step} seq {b}")
        start = [int(o.argmax(ref.logits(b))) for b in range(batch)]
        ids = gpu.generate(start, 10)
        for b in range(batch):
            t = start[b]
            expected = []
            for _ in range(10):
                t = ref.step(b, t)
                expected.append(t)
            assert ids[:, b].tolist() == expected, (b, batch, env)
    finally:
        gpu.close()
        ref.close()
