"""GPU parity of the batched prefill (qwh_decoder_prefill) with the
reference's prefill, decoder.zig:308-333: one forwardToken per prompt
position (audio pads taking the projected audio rows in order), then
argmaxLogits of the last position.

The device runs the prompt's positions together (each layer's products as
one batched GEMM over the prompt rows -- or, for matrices without that form,
one launch of their per-token GEMV over the rows -- the rows' attention as
causal pseudo-sequences over the one cache). Two checks per prompt:

  - against the oracle, position by position and teacher-forced on the
    device's cache rows (the oracle's forwardToken for position p reads the
    device's rows below p): each q8 row the prompt wrote differs from the
    oracle's only at rounding ties (a scale one f16 step, a code one apart,
    rarely), f32 rows within 1e-3, and the last position's logits within
    1e-3. Teacher forcing keeps one position's tie from reaching the next:
    run free, a single code that rounds the other way in an early row moves
    every later position's attention, and the logits of a long prompt then
    drift from the oracle's by about 1e-3 on this synthetic model -- the
    device's own one-position step drifts the same way;
  - against the device's one-position step on a second decoder holding the
    same model (the same products, in the same order): rows equal but at
    ties, logits within 1e-3.

Also: the next token, the other sequence left untouched, and greedy steps
after the prompt."""
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from oracle import oracle as o
from util import assert_close, normal, random_norms, set_norms

pytestmark = pytest.mark.gpu
o.set_threads(min(16, os.cpu_count() or 1))

TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000,
            max_positions=640, eps=1e-6, theta=1e6)
# The 0.6B decoder's head layout (16 query heads over 8 KV heads of 128).
WIDE = dict(hidden=1024, layers=2, heads=16, kv_heads=8, head_dim=128, ffn=3072, vocab=2000,
            max_positions=512, eps=1e-6, theta=1e6)
# Shapes without the matrix-core prefill (rows of an odd number of groups):
# 320 = 5 groups of 64 per row (q4 there has no fused GEMV either, so a
# q4 prompt runs position by position), and 192 = 3 groups (q4 fused: the
# rows form).
ODD = dict(hidden=320, layers=2, heads=5, kv_heads=5, head_dim=64, ffn=448, vocab=1000,
           max_positions=64, eps=1e-6, theta=1e6)
Q4ROWS = dict(hidden=192, layers=2, heads=3, kv_heads=3, head_dim=64, ffn=192, vocab=1000,
              max_positions=128, eps=1e-6, theta=1e6)
PAD = 997
CACHE = {"q8": o.CACHE_Q8, "f32": o.CACHE_F32}


def make_pair(ctx, config, batch, seed, fmt, cache, starts):
    gpu = qa.Decoder(ctx, batch=batch, cache_format=CACHE[cache], **config)
    ref = o.Decoder(seed, batch, fmt, CACHE[cache], **config)
    gpu.init_synthetic(seed, fmt)
    norms = random_norms(config, seed + 100)
    set_norms(gpu, norms, config["layers"])
    set_norms(ref, norms, config["layers"])
    for b, n in enumerate(starts):
        gpu.prefill_random(b, n, seed)
        ref.prefill_random(b, n)
    return gpu, ref


def prompt(count, vocab, pads, seed):
    """`count` token ids (none of them PAD) with PAD at the indices `pads`."""
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, vocab - 1, count).astype(np.uint32)
    tokens[tokens == PAD] = PAD + 1
    tokens[list(pads)] = PAD
    return tokens


def device_rows(ctx, dec, seq, layer, first, count, config, f32):
    """Cache rows [first, first + count) of one layer from the device planes:
    (key scales, key codes, value scales, value codes) as byte arrays (the
    scale planes empty for an f32 cache)."""
    kvw = config["kv_heads"] * config["head_dim"]
    ks, kc, vs, vc = dec.cache_planes(seq, layer)
    out = []
    for scales, codes in ((ks, kc), (vs, vc)):
        if f32:
            s = np.empty(0, np.uint8)
            c = np.empty(count * kvw * 4, np.uint8)
            ctx._check(ctx.lib.qwh_download(ctx.handle, c.ctypes.data, codes + first * kvw * 4, c.size))
        else:
            s = np.empty(count * kvw // 64 * 2, np.uint8)
            c = np.empty(count * kvw, np.uint8)
            ctx._check(ctx.lib.qwh_download(ctx.handle, s.ctypes.data, scales + first * kvw // 64 * 2, s.size))
            ctx._check(ctx.lib.qwh_download(ctx.handle, c.ctypes.data, codes + first * kvw, c.size))
        out += [s, c]
    return out


def compare_planes(got, want, kvw, count, f32, what):
    """Two sets of cache rows (device_rows layout). f32: within 1e-3. q8: a
    group's f16 scale at most one step apart and a code at most one apart
    (a summation order moved a value across a rounding tie). Returns the
    (scale, code) difference counts and totals."""
    flips = np.zeros(4, np.int64)
    for kv in range(2):
        gs, gc, ws, wc = got[2 * kv], got[2 * kv + 1], want[2 * kv], want[2 * kv + 1]
        if f32:
            assert_close(gc.view(np.float32), wc.view(np.float32), what=f"{what} kv {kv}")
            continue
        ds = gs.view(np.uint16).astype(np.int32) - ws.view(np.uint16).astype(np.int32)
        dc = gc.astype(np.int16) - wc.astype(np.int16)
        assert np.abs(ds).max(initial=0) <= 1 and np.abs(dc).max(initial=0) <= 1, (what, kv)
        flips += [np.count_nonzero(ds), ds.size, np.count_nonzero(dc), dc.size]
    return flips


def oracle_planes(ref, seq, layer, first, count, kvw, f32):
    """The oracle's cache rows in device_rows' layout."""
    n = 0 if f32 else kvw // 64 * 2
    width = kvw * 4 if f32 else kvw
    rows = [np.frombuffer(ref.cache_row(seq, layer, first + p), np.uint8) for p in range(count)]
    out = []
    for kv in range(2):
        off = kv * (n + width)
        out.append(np.concatenate([r[off:off + n] for r in rows]) if n else np.empty(0, np.uint8))
        out.append(np.concatenate([r[off + n:off + n + width] for r in rows]))
    return out


def check_rows(ctx, gpu, want_fn, seq, first, count, config, cache, what):
    kvw = config["kv_heads"] * config["head_dim"]
    flips = np.zeros(4, np.int64)
    for layer in range(config["layers"]):
        got = device_rows(ctx, gpu, seq, layer, first, count, config, cache == "f32")
        flips += compare_planes(got, want_fn(layer), kvw, count, cache == "f32", f"{what} layer {layer}")
    if cache == "q8":
        print(f"prompt rows against {what}: {flips[0]} of {flips[1]} scales one f16 step apart, "
              f"{flips[2]} of {flips[3]} codes one apart")
        assert flips[0] * 100 <= flips[1] and flips[2] * 200 <= flips[3]


def row_bytes(planes, p, kvw, f32):
    """Prompt row p of device_rows() planes as cache_row bytes."""
    n = 0 if f32 else kvw // 64 * 2
    width = kvw * 4 if f32 else kvw
    ks, kc, vs, vc = planes
    return (ks[p * n:(p + 1) * n].tobytes() + kc[p * width:(p + 1) * width].tobytes()
            + vs[p * n:(p + 1) * n].tobytes() + vc[p * width:(p + 1) * width].tobytes())


def teacher_forced(ctx, gpu, ref, seq, tokens, rows, first, config, cache):
    """Every prompt position against the oracle's forwardToken
    (decoder.zig:133-287) reading the device's cache rows below it: the
    oracle's cache takes the device's prompt rows, then for each position p
    the oracle runs p's token (or audio row) at position first + p and its
    new row is compared with the device's row p, which is then put back. No
    difference carries from one position to the next, so each row is held to
    the bound of one step, and the last position's logits (the oracle's, on
    the device's rows) to 1e-3. Returns the oracle's greedy next token."""
    f32 = cache == "f32"
    kvw = config["kv_heads"] * config["head_dim"]
    layers = config["layers"]
    count = len(tokens)
    dev = [device_rows(ctx, gpu, seq, layer, first, count, config, f32) for layer in range(layers)]
    for layer in range(layers):
        for p in range(count):
            ref.set_cache_row(seq, layer, first + p, row_bytes(dev[layer], p, kvw, f32))
    flips = np.zeros(4, np.int64)
    used = 0
    for p, t in enumerate(tokens):
        ref.set_position(seq, first + p)
        last = p + 1 == count
        if t == PAD:
            ref.forward_row(seq, int(t), rows[used], last)
            used += 1
        else:
            ref.forward(seq, int(t), last)
        for layer in range(layers):
            want = oracle_planes(ref, seq, layer, first + p, 1, kvw, f32)
            got = [x[p * (x.size // count):(p + 1) * (x.size // count)] for x in dev[layer]]
            flips += compare_planes(got, want, kvw, 1, f32, f"layer {layer} position {first + p}")
            ref.set_cache_row(seq, layer, first + p, row_bytes(dev[layer], p, kvw, f32))
    assert used == len(rows) and ref.position(seq) == first + count
    if not f32:
        print(f"prompt rows against the oracle's, teacher-forced: {flips[0]} of {flips[1]} scales one f16 "
              f"step apart, {flips[2]} of {flips[3]} codes one apart")
        assert flips[0] * 100 <= flips[1] and flips[2] * 200 <= flips[3]
    return int(o.argmax(ref.logits(seq)))


def device_per_token(ctx, dec, tokens, rows, hidden):
    """The prompt through the device's step on sequence 1 of a batch-2
    decoder (forward, forward_rows for the audio pads), one position at a
    time, as the reference's prefill runs it; sequence 0 steps beside it."""
    staged = np.zeros((2, hidden), np.float32)
    buf = ctx.to_device(staged)
    used = 0
    try:
        for i, t in enumerate(tokens):
            last = i + 1 == len(tokens)
            ids = [0, int(t)]
            if t == PAD:
                staged[1] = rows[used]
                used += 1
                buf.upload(staged)
                dec.forward_rows(ids, buf.ptr, [False, True], last)
            else:
                dec.forward(ids, last)
    finally:
        buf.free()


@pytest.mark.parametrize("name,config,fmt,cache,count,start,pads", [
    ("pads interleaved", TINY, o.Q4, "q8", 37, 0, range(1, 37, 3)),
    ("two chunks, audio block", TINY, o.Q4, "q8", 300, 5, range(9, 109)),   # 256 + 44 positions
    ("three chunks", TINY, o.Q4, "q8", 600, 0, range(3, 403)),
    ("text only, f32 cache", TINY, o.Q4, "f32", 20, 3, ()),
    ("q8 weights", TINY, o.Q8, "q8", 40, 2, range(5, 25)),
    ("q5 weights", TINY, o.Q5, "q8", 30, 1, range(3, 13)),
    ("q5 weights, f32 cache", TINY, o.Q5, "f32", 18, 4, range(2, 8)),
    ("one position", TINY, o.Q4, "q8", 1, 7, ()),
    ("one audio position", TINY, o.Q4, "q8", 1, 0, (0,)),
    ("0.6B head layout", WIDE, o.Q4, "q8", 150, 11, range(4, 124)),
    # The rows form: each projection one launch of the matrix's per-token
    # GEMV over the chunk's rows.
    ("f16 weights", TINY, o.F16, "q8", 40, 2, range(5, 25)),
    ("f16 weights, two chunks", TINY, o.F16, "q8", 300, 5, range(9, 109)),
    ("f32 weights and cache", TINY, o.F32, "f32", 20, 3, ()),
    ("q8, 320-wide rows", ODD, o.Q8, "q8", 30, 2, range(3, 13)),
    ("q4, 192-wide rows", Q4ROWS, o.Q4, "q8", 40, 1, range(2, 12)),
])
def test_prefill_matches_per_token_reference(ctx, name, config, fmt, cache, count, start, pads):
    seed = 9
    pads = list(pads)
    kvw = config["kv_heads"] * config["head_dim"]
    gpu, ref = make_pair(ctx, config, 2, seed, fmt, cache, [13, start])
    # The same model through the device's own per-position step.
    twin, _ = make_pair(ctx, config, 2, seed, fmt, cache, [13, start])
    try:
        tokens = prompt(count, config["vocab"], pads, seed + count)
        rows = normal(len(pads) * config["hidden"], 77, count).reshape(len(pads), config["hidden"])
        rb = ctx.to_device(rows) if pads else None
        try:
            got = gpu.prefill(1, tokens, PAD, rb.ptr if rb else 0, len(pads))
        finally:
            if rb:
                rb.free()
        want = teacher_forced(ctx, gpu, ref, 1, tokens, rows, start, config, cache)
        device_per_token(ctx, twin, tokens, rows, config["hidden"])
        assert gpu.position(1) == start + count == twin.position(1)
        assert gpu.position(0) == 13
        f32 = cache == "f32"
        check_rows(ctx, gpu, lambda layer: device_rows(ctx, twin, 1, layer, start, count, config, f32),
                   1, start, count, config, cache, "the device step's")
        logits, expected = gpu.logits(1), ref.logits(1)
        assert_close(logits, expected, what=f"{name}: against the oracle (teacher-forced)")
        # Same products, summed in the same order: the per-position device
        # step agrees within the same bar.
        assert_close(logits, twin.logits(1), what=f"{name}: against the device step")
        if got != want:
            # The device may pick another id only where the oracle's logits
            # of the two ids lie within twice this test's measured logit
            # error of each other (each of the two carries at most that
            # error).
            err = float(np.max(np.abs(logits.astype(np.float64) - expected)))
            best = float(np.max(expected))
            assert best - float(expected[got]) <= 2 * err, (got, want, best - float(expected[got]), err)
        # Greedy steps after the prompt (the other sequence steps beside it).
        tokens = [o.start_token(seed, 0, config["vocab"]), want]
        for step in range(4):
            ids = gpu.step(tokens)
            expect = [ref.step(b, tokens[b]) for b in range(2)]
            assert list(ids) == expect, (name, step)
            tokens = expect
    finally:
        gpu.close()
        twin.close()
        ref.close()


def test_prefill_then_prefill_again(ctx):
    # A second prompt continues the sequence from where the first left it
    # (decoder.zig:308 feeds tokens at the sequence's current position). The
    # audio rows here are at the embeddings' scale (the synthetic embedding
    # values are N(0, 0.02)), as projected audio rows stand in for embeddings.
    seed, hidden = 21, TINY["hidden"]
    gpu, ref = make_pair(ctx, TINY, 2, seed, o.Q4, "q8", [6, 0])
    twin, _ = make_pair(ctx, TINY, 2, seed, o.Q4, "q8", [6, 0])
    try:
        first = prompt(50, TINY["vocab"], range(2, 12), 1)
        rows = normal(10 * hidden, 78, 0, 0.02).reshape(10, hidden)
        rb = ctx.to_device(rows)
        try:
            gpu.prefill(1, first, PAD, rb.ptr, 10)
        finally:
            rb.free()
        teacher_forced(ctx, gpu, ref, 1, first, rows, 0, TINY, "q8")
        second = prompt(30, TINY["vocab"], (), 2)
        got = gpu.prefill(1, second)
        want = teacher_forced(ctx, gpu, ref, 1, second, np.zeros((0, hidden), np.float32), 50, TINY, "q8")
        device_per_token(ctx, twin, np.concatenate([first, second]), rows, hidden)
        assert gpu.position(1) == 80 == twin.position(1) and gpu.position(0) == 6
        check_rows(ctx, gpu, lambda layer: device_rows(ctx, twin, 1, layer, 0, 80, TINY, False),
                   1, 0, 80, TINY, "q8", "the device step's")
        assert_close(gpu.logits(1), ref.logits(1), what="second prompt against the oracle (teacher-forced)")
        assert_close(gpu.logits(1), twin.logits(1), what="second prompt against the device step")
        assert got == want
    finally:
        gpu.close()
        twin.close()
        ref.close()


def test_prefill_position_by_position(ctx):
    # q4 rows of 320 values have neither a matrix-core nor a fused per-token
    # GEMV: at batch 1 the prompt runs through the step one position at a
    # time (decoder.zig:319-331 as written), the same checks hold; batch 2 is
    # refused (the step would advance the other sequence too). At this K the
    # q4 step takes the generic GEMV (a wavefront per row, per gate / up row
    # pair for siluMul).
    seed, fmt = 33, o.Q4
    gpu, ref = make_pair(ctx, ODD, 1, seed, fmt, "q8", [3])
    try:
        tokens = prompt(20, ODD["vocab"], range(4, 10), 5)
        rows = normal(6 * ODD["hidden"], 79, 0, 0.02).reshape(6, ODD["hidden"])
        rb = ctx.to_device(rows)
        try:
            got = gpu.prefill(0, tokens, PAD, rb.ptr, 6)
        finally:
            rb.free()
        want = teacher_forced(ctx, gpu, ref, 0, tokens, rows, 3, ODD, "q8")
        assert_close(gpu.logits(0), ref.logits(0), what="odd shape, last position (teacher-forced)")
        assert got == want and gpu.position(0) == 23
    finally:
        gpu.close()
        ref.close()
    d = qa.Decoder(ctx, batch=2, **ODD)
    try:
        d.init_synthetic(seed, fmt)
        with pytest.raises(qa.QwhError) as err:
            d.prefill(0, prompt(5, ODD["vocab"], (), 6))
        assert err.value.status == -3 and d.position(0) == 0
    finally:
        d.close()


def test_prefill_errors_leave_the_sequence_alone(ctx):
    # decoder.zig:316-317 (UnexpectedShape: an empty prompt), :322 / :331
    # (PromptMismatch: audio pads and rows not one to one) and :142
    # (PositionExceeded). The reference maps PromptMismatch and
    # UnexpectedShape to shape_mismatch at its ABI; here every prompt is
    # checked before any position runs, so a refused prompt changes nothing.
    d = qa.Decoder(ctx, batch=1, **{**TINY, "max_positions": 40})
    try:
        d.init_synthetic(3)
        d.prefill_random(0, 10, 3)
        rows = ctx.to_device(np.zeros((4, TINY["hidden"]), np.float32))
        try:
            cases = [
                (np.zeros(0, np.uint32), 0, -7),                     # empty
                (prompt(8, TINY["vocab"], (1, 2, 3), 5), 4, -7),     # 3 pads, 4 rows
                (prompt(8, TINY["vocab"], (1, 2, 3, 4, 5), 5), 4, -7),  # 5 pads, 4 rows
                (np.array([1, TINY["vocab"]], np.uint32), 0, -7),    # token out of range
                (prompt(31, TINY["vocab"], (), 5), 0, -9),           # 10 + 31 > 40 positions
            ]
            for tokens, steps, status in cases:
                with pytest.raises(qa.QwhError) as err:
                    d.prefill(0, tokens, PAD, rows.ptr if steps else 0, steps)
                assert err.value.status == status, (len(tokens), steps)
                assert d.position(0) == 10
            # 10 + 30 = 40 positions fit exactly.
            d.prefill(0, prompt(30, TINY["vocab"], (0, 1, 2, 3), 6), PAD, rows.ptr, 4)
            assert d.position(0) == 40
        finally:
            rows.free()
    finally:
        d.close()
