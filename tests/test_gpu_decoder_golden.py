"""The configs[4] decoder shape (Qwen3-ASR-1.7B: 28 layers, hidden 2048,
16 / 8 heads of 128, SwiGLU 6144, vocab 151936, q4 weights, q8 cache
prefilled to 4096 positions, seed 4) against the CPU oracle:

  - teacher-forced logits of every sequence at steps 0, 1, 64, 127 and 255
    against tests/golden/decoder_1p7b_logits.json (the 16 largest, a fixed
    sample across the vocabulary), within 1e-3 relative and within the
    per-step error bound below;
  - 256 greedy steps per sequence against the oracle's ids in
    tests/golden/decoder_1p7b_ids.json (tests/golden/make_decoder_ids.py):
    at batch 1 all 256 identical; at batch 16 at least 15 of the 16
    sequences and 3967 of the 4096 steps identical (the one sequence that
    differs takes the oracle's runner-up at step 127, inside the tie window
    the error bound gives; 44 of the fixture's 4096 steps lie inside it);
    the q8-weight fixture identical in full at both batches.

decoder.zig:133-339 (forwardToken, step, argmaxLogits)."""
import json
import os

import numpy as np
import pytest

import qwenscriber_amd as qa
from util import assert_close

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
IDS = os.path.join(HERE, "decoder_1p7b_ids.json")
LOGITS = os.path.join(HERE, "decoder_1p7b_logits.json")

# Teacher-forced logit error against the oracle, as a fraction of the step's
# largest logit, bounded per recorded step: twice the worst measured over the
# 16 sequences at batch 1 and batch 16 (measured: step 0 8.1e-6, step 1
# 2.0e-5, step 64 9.8e-5, step 127 1.56e-4, step 255 1.97e-4). The error
# grows with the step: each step appends key and value rows whose q8 codes
# may round the other way at a tie (the device's products sum in another
# order; test_gpu_decoder.py pins that those rows differ from the oracle's
# only there), and later steps attend to more of those rows.
ERROR_BOUND = {0: 2e-5, 1: 4e-5, 64: 2e-4, 127: 3.2e-4, 255: 4e-4}


def tie_window(step):
    """The largest gap between the oracle's two best logits (as a fraction
    of the best) at which the device may pick the runner-up: the two logits
    each carry at most the error bound of the first recorded step at or after
    `step`."""
    return 2 * ERROR_BOUND[min(s for s in ERROR_BOUND if s >= step)]


def load(path):
    if not os.path.exists(path):
        pytest.skip(f"golden file {os.path.basename(path)} not generated")
    with open(path) as f:
        return json.load(f)


def make_decoder(ctx, golden, batch):
    dec = qa.Decoder(ctx, batch=batch, **golden["config"])
    dec.init_synthetic(golden["seed"], golden.get("format", qa.FORMAT_Q4))
    for b in range(batch):
        dec.prefill_random(b, golden["prefill"], golden["seed"])
    return dec


def run(ctx, golden, batch):
    dec = make_decoder(ctx, golden, batch)
    try:
        start = np.array([golden["ids"][b][0] for b in range(batch)], np.uint32)
        return dec.generate(start, golden["steps"])
    finally:
        dec.close()


def check(ids, golden, batch, min_sequences, min_steps):
    """Every sequence matches the oracle's greedy ids, but for a near tie: at
    the first differing step the GPU took the oracle's runner-up, and the
    oracle's two best logits lie within tie_window(step) of each other. From
    there the sequence continues from another token, so its comparison ends;
    the other sequences are still compared in full. At least min_sequences
    sequences and min_steps steps (summed up to each sequence's first
    difference) must be identical: a flip inside the window still counts
    against them."""
    same_seqs = same_steps = 0
    for b in range(batch):
        expected = golden["ids"][b][1:]
        got = ids[:, b].tolist()
        first = next((i for i, (x, y) in enumerate(zip(got, expected)) if x != y), None)
        if first is None:
            same_seqs += 1
            same_steps += len(expected)
            continue
        same_steps += first
        msg = f"sequence {b}: first difference at step {first}: {got[first]} != {expected[first]}"
        top, second = golden["top"][b][first], golden["second"][b][first]
        assert got[first] == golden["runner_up"][b][first], f"{msg} (runner-up {golden['runner_up'][b][first]})"
        assert top - second <= tie_window(first) * abs(top), \
            f"{msg}: oracle logits {top} and {second} are not a near tie"
        print(f"{msg}: the oracle's runner-up, {(top - second) / abs(top):.2e} below its best")
    print(f"identical: {same_seqs} of {batch} sequences, {same_steps} of {batch * golden['steps']} steps")
    assert same_seqs >= min_sequences and same_steps >= min_steps, \
        f"identical {same_seqs} sequences / {same_steps} steps, fewer than {min_sequences} / {min_steps}"


def check_logits(ctx, golden, ref, batch):
    """Teacher-forced steps 0 .. the last recorded one; at each recorded
    step the device logits at the fixture's indices within 1e-3 relative.
    Returns the worst error relative to the largest logit, per recorded
    step."""
    dec = make_decoder(ctx, golden, batch)
    steps = ref["steps"]
    worst = {s: 0.0 for s in steps}
    sample = list(range(0, ref["sample_stride"] * ref["samples"], ref["sample_stride"]))
    try:
        for s in range(steps[-1] + 1):
            dec.forward([golden["ids"][b][s] for b in range(batch)], s in worst)
            if s not in worst:
                continue
            i = steps.index(s)
            for b in range(batch):
                rec = ref["records"][b][i]
                logits = dec.logits(b)
                idx = np.array(rec["top_index"] + sample)
                want = np.array(rec["top_value"] + rec["sample"], np.float32)
                got = logits[idx]
                assert_close(got, want, what=f"teacher-forced step {s} sequence {b}")
                worst[s] = max(worst[s], float(np.max(np.abs(got - want)) / np.max(np.abs(want))))
    finally:
        dec.close()
    print("teacher-forced logits, worst error / largest logit per step: " +
          ", ".join(f"{s}: {w:.2e}" for s, w in worst.items()))
    for s, w in worst.items():
        assert w <= ERROR_BOUND[s], f"step {s}: error {w:.2e} above its bound {ERROR_BOUND[s]:.1e}"
    return worst


def test_batch1_teacher_forced_logits(ctx):
    golden, ref = load(IDS), load(LOGITS)
    check_logits(ctx, golden, ref, 1)


def test_batch16_teacher_forced_logits(ctx):
    golden, ref = load(IDS), load(LOGITS)
    check_logits(ctx, golden, ref, len(ref["records"]))


def test_batch1_greedy_ids_match_oracle(ctx):
    # Batch 1 runs the lane-per-row GEMVs with fused activation forms.
    golden = load(IDS)
    check(run(ctx, golden, 1), golden, 1, 1, golden["steps"])


def test_batch16_greedy_ids_match_oracle(ctx):
    # Batch 16 runs the matrix-core GEMVs; every sequence has its own cache.
    golden = load(IDS)
    batch = len(golden["ids"])
    if batch < 2:
        pytest.skip("golden file holds one sequence")
    # Measured: 15 of 16 sequences, 3967 of 4096 steps (sequence 11 takes
    # the runner-up at step 127, 1.9e-5 below the best logit).
    check(run(ctx, golden, batch), golden, batch, batch - 1, 3967)


def test_q8_model_greedy_ids_match_oracle(ctx):
    # The same synthetic model with every matrix in q8 (the format the
    # reference's status page finds transcribing where q4 does not), at
    # batch 1 (byte-plane GEMV) and at the fixture's batch (q8 on the matrix
    # cores).
    golden = load(os.path.join(HERE, "decoder_1p7b_q8_ids.json"))
    steps = golden["steps"]
    check(run(ctx, golden, 1), golden, 1, 1, steps)
    batch = len(golden["ids"])
    if batch > 1:
        check(run(ctx, golden, batch), golden, batch, batch, batch * steps)
