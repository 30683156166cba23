"""GPU parity of the decoder step with q5, q8, f16 and f32 weights and with
the f32 key/value cache, against the oracle holding the same model.

kernels.zig:182-206 (Matrix.apply runs whatever format a matrix holds; the
converter writes every matrix in one format, layout.zig:49-53),
decoder.zig:68-106 / :220-253 (the f32 and q8 caches), and the stop rules of
wasm/model.zig:423-451 decodeStep (:495-499 endsSequence) for the device
greedy loop."""
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
CACHE = {"q8": o.CACHE_Q8, "f32": o.CACHE_F32}


def make_pair(ctx, config, batch, seed, fmt, cache, norms=True):
    gpu = qa.Decoder(ctx, batch=batch, cache_format=CACHE[cache], **config)
    ref = o.Decoder(seed, batch, fmt, CACHE[cache], **config)
    gpu.init_synthetic(seed, fmt)
    if norms:
        n = random_norms(config, seed + 100)
        set_norms(gpu, n, config["layers"])
        set_norms(ref, n, config["layers"])
    for b in range(batch):
        count = (7 * b + 2) % 31
        gpu.prefill_random(b, count, seed)
        ref.prefill_random(b, count)
    return gpu, ref


def oracle_greedy(ref, b, token, steps):
    out = []
    for _ in range(steps):
        token = ref.step(b, token)
        out.append(token)
    return out


@pytest.mark.parametrize("fmt,cache,batch,config,env", [
    (o.Q8, "q8", 1, TINY, ()),      # byte-plane GEMV, fused RMSNorm prologue, pairs epilogue
    (o.Q8, "q8", 3, TINY, ()),      # q8 on the matrix-core batch GEMV (split form)
    (o.Q8, "q8", 18, TINY, ()),     # two token tiles
    (o.Q8, "q8", 3, ODD, ()),       # unsplit matrix-core form (an odd number of groups) and the generic GEMV
    (o.Q8, "q8", 3, TINY, ("QWH_DECODER_NO_SPLIT",)),
    (o.Q5, "q8", 1, TINY, ()),      # q5 byte-plane GEMV
    (o.Q5, "q8", 3, TINY, ()),      # q5 on the matrix-core batch GEMV (split form)
    (o.Q5, "q8", 2, ODD, ()),
    (o.Q4, "f32", 1, TINY, ()),     # f32 cache
    (o.Q4, "f32", 3, TINY, ()),
    (o.Q4, "f32", 18, TINY, ()),
    (o.Q8, "f32", 2, TINY, ()),
    (o.Q5, "f32", 1, ODD, ()),      # head_dim 64, one query head per kv head
    (o.F16, "q8", 1, TINY, ()),     # f16 weights (--quantization none): the dense GEMV
    (o.F16, "q8", 3, TINY, ()),     # a group of three tokens per pass over the weights
    (o.F16, "q8", 18, TINY, ()),    # four-token groups and a tail of two
    (o.F32, "f32", 2, ODD, ()),     # f32 weights and cache, head_dim 64
])
def test_formats_teacher_forced_and_greedy(ctx, fmt, cache, batch, config, env, monkeypatch):
    for name in env:
        monkeypatch.setenv(name, "1")
    seed = 23
    gpu, ref = make_pair(ctx, config, batch, seed, fmt, cache)
    try:
        vocab = config["vocab"]
        for step in range(4):
            tokens = [(step * 71 + b * 13 + 5) % vocab for b in range(batch)]
            gpu.forward(tokens, True)
            for b in range(batch):
                ref.forward(b, tokens[b], True)
                assert_close(gpu.logits(b), ref.logits(b), what=f"fmt {fmt} cache {cache} step {step} seq {b}")
        start = [int(o.argmax(ref.logits(b))) for b in range(batch)]
        ids = gpu.generate(start, 10)
        for b in range(batch):
            assert ids[:, b].tolist() == oracle_greedy(ref, b, start[b], 10), (fmt, cache, batch, b)
        for b in range(batch):
            assert gpu.position(b) == ref.position(b)
    finally:
        gpu.close()
        ref.close()


def test_f32_cache_prefill_holds_the_rows(ctx):
    # decoder.zig:77-83: the f32 cache stores each row as it is; the prefilled
    # rows are the generator's values, bit for bit.
    gpu = qa.Decoder(ctx, batch=2, cache_format=qa.CACHE_F32, **TINY)
    try:
        gpu.prefill_random(1, 9, 5)
        kvw = TINY["kv_heads"] * TINY["head_dim"]
        for layer in range(TINY["layers"]):
            ks, kc, vs, vc = gpu.cache_planes(1, layer)
            assert ks is None and vs is None
            for base, kv in ((kc, 0), (vc, 1)):
                got = np.empty(9 * kvw, np.float32)
                ctx._check(ctx.lib.qwh_download(ctx.handle, got.ctypes.data, base, got.nbytes))
                want = o.normal(9 * kvw, 5, 0x10000 + 0x100 * 1 + 2 * layer + kv)
                assert np.array_equal(got, want)
    finally:
        gpu.close()


def test_matrices_rebound_in_another_format(ctx):
    # Bound one by one through set_matrix: q8 planes replace a q4 synthetic
    # model (each fused block re-created in q8, then every member bound).
    seed, c = 29, TINY
    qw, kvw = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
    gpu = qa.Decoder(ctx, batch=1, **c)
    ref = o.Decoder(seed, 1, o.Q8, o.CACHE_Q8, **c)
    handles = []
    try:
        gpu.init_synthetic(seed)

        def bind(kind, layer, rows, cols, stream):
            s, d = o.quantize_rows(o.Q8, o.normal(rows * cols, seed, stream, 0.02).reshape(rows, cols))
            h = ctx.matrix_upload(qa.FORMAT_Q8, rows, cols, s, d)
            handles.append(h)
            gpu.set_matrix(kind, layer, h)

        bind(qa.T_EMBED, 0, c["vocab"], c["hidden"], 1)
        bind(qa.T_LM_HEAD, 0, c["vocab"], c["hidden"], 2)
        for layer in range(c["layers"]):
            base = 16 + 16 * layer
            for kind, rows, cols, k in ((qa.T_Q, qw, c["hidden"], 0), (qa.T_K, kvw, c["hidden"], 1),
                                        (qa.T_V, kvw, c["hidden"], 2), (qa.T_O, c["hidden"], qw, 3),
                                        (qa.T_GATE, c["ffn"], c["hidden"], 4), (qa.T_UP, c["ffn"], c["hidden"], 5),
                                        (qa.T_DOWN, c["hidden"], c["ffn"], 6)):
                bind(kind, layer, rows, cols, base + k)
        gpu.prefill_random(0, 6, seed)
        ref.prefill_random(0, 6)
        for t in (3, 400, 999):
            gpu.forward([t], True)
            ref.forward(0, t, True)
            assert_close(gpu.logits(0), ref.logits(0), what=f"rebound q8 token {t}")
    finally:
        for h in handles:
            ctx.matrix_release(h)
        gpu.close()
        ref.close()


def oracle_until(ref, b, token, max_tokens, stops):
    """wasm/model.zig:423-451 decodeStep looped to the end of the sequence."""
    emitted = []
    while True:
        if token in stops or len(emitted) >= max_tokens:
            return emitted
        emitted.append(token)
        if len(emitted) >= max_tokens:
            return emitted
        token = ref.step(b, token)


@pytest.mark.parametrize("batch", [1, 4])
def test_generate_until_stop_tokens_and_budget(ctx, batch):
    seed = 31
    config = TINY
    # A free run of the oracle picks stop tokens that some sequences meet
    # midway (a different step for each).
    probe = o.Decoder(seed, batch, **config)
    for b in range(batch):
        probe.prefill_random(b, 4 + b)
    start = [(97 * b + 11) % config["vocab"] for b in range(batch)]
    runs = [oracle_greedy(probe, b, start[b], 12) for b in range(batch)]
    probe.close()
    stops = [runs[0][5]]
    if batch > 1:
        stops.append(runs[1][2])
        stops.append(start[2])    # sequence 2's first token: it ends before emitting anything
    max_tokens = 10
    gpu = qa.Decoder(ctx, batch=batch, **config)
    ref = o.Decoder(seed, batch, **config)
    try:
        gpu.init_synthetic(seed)
        for b in range(batch):
            gpu.prefill_random(b, 4 + b, seed)
            ref.prefill_random(b, 4 + b)
        ids, counts = gpu.generate_until(start, max_tokens, stops)
        for b in range(batch):
            want = oracle_until(ref, b, start[b], max_tokens, stops)
            assert counts[b] == len(want), (b, counts[b], want)
            assert ids[: counts[b], b].tolist() == want, b
            assert np.all(ids[counts[b]:, b] == 0)
            assert gpu.position(b) == ref.position(b), b
        # The decoder continues with plain steps afterwards.
        nxt = gpu.step([int(ids[max(counts[b], 1) - 1, b]) if counts[b] else start[b] for b in range(batch)])
        assert len(nxt) == batch
    finally:
        gpu.close()
        ref.close()


def test_generate_until_budget_zero_and_one(ctx):
    gpu = qa.Decoder(ctx, batch=2, **TINY)
    try:
        gpu.init_synthetic(3)
        ids, counts = gpu.generate_until([5, 6], 0, [])
        assert ids.shape == (0, 2) and counts.tolist() == [0, 0]
        ids, counts = gpu.generate_until([5, 6], 1, [6])
        assert counts.tolist() == [1, 0] and ids[0, 0] == 5
        assert gpu.position(0) == 0 and gpu.position(1) == 0   # no forward for a budget of one
        with pytest.raises(qa.QwhError):
            gpu.generate_until([5, 6], 3, [1, 2, 3, 4])       # at most three stop tokens
    finally:
        gpu.close()
