"""GPU parity of the decoder step (decoder.zig:133-339) against the oracle's
restatement, on synthetic q4 models with a q8 cache."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, normal

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
            max_positions=64, eps=1e-6, theta=1e6)


def cache_hash(ctx, dec, seq, config):
    """FNV-1a over a sequence's key planes then value planes, all layers, in
    the decoder.zig:58-65 layout (as the oracle's qwref_decoder_cache_hash)."""
    kvw = config["kv_heads"] * config["head_dim"]
    layer_stride = config["max_positions"] * (kvw // 64) * 2 + config["max_positions"] * kvw
    total = layer_stride * config["layers"]
    ks, _, vs, _ = dec.cache_planes(seq, 0)
    h = 0xCBF29CE484222325
    for base in (ks, vs):
        buf = np.empty(total, np.uint8)
        ctx._check(ctx.lib.qwh_download(ctx.handle, buf.ctypes.data, base, total))
        h = o.fnv1a64(buf, h)
    return h


@pytest.fixture
def tiny_pair(ctx):
    seed, batch = 9, 3
    gpu = qa.Decoder(ctx, batch=batch, **TINY)
    gpu.init_synthetic(seed)
    ref = o.Decoder(seed, batch, **TINY)
    for b, n in enumerate([0, 5, 17]):
        gpu.prefill_random(b, n, seed)
        ref.prefill_random(b, n)
    yield gpu, ref
    gpu.close()
    ref.close()


def test_prefilled_cache_is_bit_exact(ctx, tiny_pair):
    gpu, ref = tiny_pair
    for b in range(3):
        assert cache_hash(ctx, gpu, b, TINY) == ref.cache_hash(b)
        assert gpu.position(b) == ref.position(b)


def test_teacher_forced_logits(ctx, tiny_pair):
    gpu, ref = tiny_pair
    for step in range(8):
        tokens = [(step * 37 + b * 101) % TINY["vocab"] for b in range(3)]
        gpu.forward(tokens, True)
        for b in range(3):
            ref.forward(b, tokens[b], True)
            assert_close(gpu.logits(b), ref.logits(b), what=f"step {step} seq {b}")
    for b in range(3):
        assert gpu.position(b) == ref.position(b)


def device_cache_row(ctx, dec, seq, layer, position, config):
    """A q8 cache row from the device planes, in the oracle's cache_row
    layout: key scales, key codes, value scales, value codes."""
    kvw = config["kv_heads"] * config["head_dim"]
    ks, kc, vs, vc = dec.cache_planes(seq, layer)
    parts = []
    for scales, codes in ((ks, kc), (vs, vc)):
        s = np.empty(kvw // 64 * 2, np.uint8)
        c = np.empty(kvw, np.uint8)
        ctx._check(ctx.lib.qwh_download(ctx.handle, s.ctypes.data, scales + position * s.size, s.size))
        ctx._check(ctx.lib.qwh_download(ctx.handle, c.ctypes.data, codes + position * kvw, kvw))
        parts += [s, c]
    return parts


def test_appended_rows_differ_only_at_rounding_ties(ctx, tiny_pair):
    # The rows each step appends (decoder.zig:85-105, quantizeRow(.q8) of the
    # new key and value) come from the device's q/k/v products, which sum in
    # another order than the oracle's dotRow. A group's f16 scale may then
    # round to the neighbouring f16 (its largest |value| / 128 lies at a
    # rounding tie), and a code may round the other way (value / scale lies
    # within that difference of a half-integer). Pinned here: scales differ
    # by at most one f16 step, codes by at most one, and only rarely. This is
    # what makes the teacher-forced logit error of a long generation grow
    # with the step count (tests/test_gpu_decoder_golden.py measures it).
    gpu, ref = tiny_pair
    kvw = TINY["kv_heads"] * TINY["head_dim"]
    n = kvw // 64 * 2
    start = [gpu.position(b) for b in range(3)]
    steps = 40
    for step in range(steps):
        tokens = [(step * 53 + b * 211) % TINY["vocab"] for b in range(3)]
        gpu.forward(tokens, False)
        for b in range(3):
            ref.forward(b, tokens[b], False)
    scale_flips = groups = code_flips = codes = 0
    for b in range(3):
        for layer in range(TINY["layers"]):
            for p in range(start[b], start[b] + steps):
                want = np.frombuffer(ref.cache_row(b, layer, p), np.uint8)
                ks, kc, vs, vc = device_cache_row(ctx, gpu, b, layer, p, TINY)
                for kv, (sc, c) in enumerate(((ks, kc), (vs, vc))):
                    off = kv * (n + kvw)
                    ds = sc.view(np.uint16).astype(np.int32) - want[off:off + n].view(np.uint16).astype(np.int32)
                    dc = c.astype(np.int16) - want[off + n:off + n + kvw].astype(np.int16)
                    assert np.abs(ds).max() <= 1 and np.abs(dc).max() <= 1, (b, layer, p, kv)
                    scale_flips += int(np.count_nonzero(ds))
                    code_flips += int(np.count_nonzero(dc))
                    groups += ds.size
                    codes += dc.size
    print(f"appended rows against the oracle's: {scale_flips} of {groups} scales one f16 step apart, "
          f"{code_flips} of {codes} codes one apart")
    assert scale_flips * 100 <= groups and code_flips * 200 <= codes


def test_free_running_token_ids(ctx, tiny_pair):
    gpu, ref = tiny_pair
    start = [o.start_token(9, b, TINY["vocab"]) for b in range(3)]
    ids = gpu.generate(start, 30)
    for b in range(3):
        t = start[b]
        expected = []
        for _ in range(30):
            t = ref.step(b, t)
            expected.append(t)
        assert ids[:, b].tolist() == expected, b


@pytest.mark.parametrize("batch,env", [
    (1, ()),                                                   # lane-per-row GEMVs, fused inputs
    (2, ("QWH_DECODER_PER_TOKEN",)),                           # batch > 1 on the per-token GEMVs
    (2, ("QWH_DECODER_PER_TOKEN", "QWH_DECODER_UNFUSED")),     # separate norm / SiLU / digit kernels
    (1, ("QWH_NO_GRAPH",)),                                    # kernels launched one by one, no graph replay
])
def test_token_ids_on_each_gemv_path(ctx, batch, env, monkeypatch):
    # The default batch > 1 path (matrix-core GEMVs) is covered above; the
    # environment switches are read when the decoder is created.
    for name in env:
        monkeypatch.setenv(name, "1")
    seed = 13
    gpu = qa.Decoder(ctx, batch=batch, **TINY)
    ref = o.Decoder(seed, batch, **TINY)
    try:
        gpu.init_synthetic(seed)
        for b in range(batch):
            gpu.prefill_random(b, 4 + 7 * b, seed)
            ref.prefill_random(b, 4 + 7 * b)
        start = [o.start_token(seed, b, TINY["vocab"]) for b in range(batch)]
        ids = gpu.generate(start, 20)
        for b in range(batch):
            t = start[b]
            expected = []
            for _ in range(20):
                t = ref.step(b, t)
                expected.append(t)
            assert ids[:, b].tolist() == expected, (b, env)
    finally:
        gpu.close()
        ref.close()


# Widths that are not multiples of 256 (5, 7 and 15 groups): the small-batch
# GEMV has no K-split form for them and runs its unsplit kernel.
ODD = dict(hidden=320, layers=2, heads=5, kv_heads=5, head_dim=64, ffn=448, vocab=500,
           max_positions=64, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("batch,config,env", [
    (18, TINY, ()),                             # two 16-token tiles of partial sums and digit planes
    (3, TINY, ("QWH_DECODER_NO_SPLIT",)),      # o / gate|up / down add their own slices
    (3, ODD, ()),                               # unsplit kernel, RMSNorm factor in its epilogue
    (3, TINY, ("QWH_NO_GRAPH",)),              # kernels launched one by one, no graph replay
])
def test_token_ids_on_each_batched_form(ctx, batch, config, env, monkeypatch):
    for name in env:
        monkeypatch.setenv(name, "1")
    seed = 21
    gpu = qa.Decoder(ctx, batch=batch, **config)
    ref = o.Decoder(seed, batch, **config)
    try:
        gpu.init_synthetic(seed)
        for b in range(batch):
            gpu.prefill_random(b, (3 * b) % 23, seed)
            ref.prefill_random(b, (3 * b) % 23)
        start = [o.start_token(seed, b, config["vocab"]) for b in range(batch)]
        ids = gpu.generate(start, 12)
        for b in range(batch):
            t = start[b]
            expected = []
            for _ in range(12):
                t = ref.step(b, t)
                expected.append(t)
            assert ids[:, b].tolist() == expected, (b, batch, env)
    finally:
        gpu.close()
        ref.close()


def test_step_and_generate_agree(ctx):
    seed = 11
    a = qa.Decoder(ctx, batch=2, **TINY)
    b = qa.Decoder(ctx, batch=2, **TINY)
    try:
        for d in (a, b):
            d.init_synthetic(seed)
            d.prefill_random(0, 3, seed)
            d.prefill_random(1, 9, seed)
        tokens = np.array([1, 2], np.uint32)
        stepped = []
        t = tokens
        for _ in range(12):
            t = a.step(t)
            stepped.append(t.copy())
        generated = b.generate(tokens, 12)
        assert np.array_equal(np.stack(stepped), generated)
        assert a.position(0) == b.position(0) == 15
    finally:
        a.close()
        b.close()


def test_position_limit_and_token_range(ctx):
    d = qa.Decoder(ctx, batch=1, **{**TINY, "max_positions": 4})
    try:
        d.init_synthetic(1)
        d.prefill_random(0, 3, 1)
        d.step([5])
        with pytest.raises(qa.QwhError) as err:
            d.step([5])   # decoder.zig:142 PositionExceeded
        assert err.value.status == -9
        d.reset()
        with pytest.raises(qa.QwhError) as err:
            d.step([TINY["vocab"]])
        assert err.value.status == -7
    finally:
        d.close()


@pytest.mark.parametrize("batch", [1, 3])
def test_audio_rows_replace_embeddings(ctx, batch):
    # decoder.zig:133-150 / :308-333: projected audio rows spliced into
    # placeholder positions, mixed with embedded tokens, then greedy steps.
    seed = 9
    gpu = qa.Decoder(ctx, batch=batch, **TINY)
    gpu.init_synthetic(seed)
    ref = o.Decoder(seed, batch, **TINY)
    for b in range(batch):
        gpu.prefill_random(b, 3 + 4 * b, seed)
        ref.prefill_random(b, 3 + 4 * b)
    hidden = TINY["hidden"]
    for step in range(5):
        rows = normal(batch * hidden, 77, step).reshape(batch, hidden)
        mask = [(step + b) % 2 == 0 for b in range(batch)]
        tokens = [(step * 13 + b * 7) % TINY["vocab"] for b in range(batch)]
        rb = ctx.to_device(rows)
        gpu.forward_rows(tokens, rb.ptr, mask, True)
        rb.free()
        for b in range(batch):
            if mask[b]:
                ref.forward_row(b, tokens[b], rows[b], True)
            else:
                ref.forward(b, tokens[b], True)
            assert_close(gpu.logits(b), ref.logits(b), what=f"audio step {step} seq {b}")
    # Greedy steps after the splice embed their tokens again.
    tokens = [int(o.argmax(ref.logits(b))) for b in range(batch)]
    for _ in range(4):
        got = gpu.step(tokens)
        want = [ref.step(b, tokens[b]) for b in range(batch)]
        assert list(got) == want
        tokens = want
    for b in range(batch):
        assert gpu.position(b) == ref.position(b)
    gpu.close()
    ref.close()
