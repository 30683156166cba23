#!/usr/bin/env python3
"""Writes tests/golden/decoder_1p7b_ids.json: greedy token ids of the CPU
oracle (oracle/qwref.c, a restatement of decoder.zig:133-339) for the
configs[4] decoder shape -- 28 layers, hidden 2048, 16 / 8 heads of 128,
SwiGLU 6144, vocab 151936, RMSNorm eps 1e-6, RoPE theta 1e6, q4 weights from
the synthetic generator under seed 4, each sequence's q8 cache prefilled with
4096 random rows, then 256 greedy steps from the synthetic start token.
Each step also records the oracle's runner-up token and the two largest
logits, so that a consumer can tell a flip between near-tied tokens (float
summation order) from a wrong result.

Usage: python3 tests/golden/make_decoder_ids.py [--batch 16] [--steps 256]
                [--format 16|17|18]
(the oracle is single-sequence at a time; about 0.3 s per step on 8 threads).
--format quantizes every matrix of the same synthetic model to q4 (16, the
default: decoder_1p7b_ids.json), q5 (17) or q8 (18: decoder_1p7b_q8_ids.json).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as o  # noqa: E402

CONFIG = dict(hidden=2048, layers=28, heads=16, kv_heads=8, head_dim=128, ffn=6144, vocab=151936,
              max_positions=4352, eps=1e-6, theta=1e6)
SEED = 4
PREFILL = 4096


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--format", type=int, default=o.Q4, choices=(o.Q4, o.Q5, o.Q8))
    ap.add_argument("--out", default=None)
    args = ap.parse_args()
    suffix = {o.Q4: "", o.Q5: "_q5", o.Q8: "_q8"}[args.format]
    out = args.out or os.path.join(os.path.dirname(os.path.abspath(__file__)), f"decoder_1p7b{suffix}_ids.json")
    o.set_threads(args.threads)
    t0 = time.time()
    dec = o.Decoder(SEED, args.batch, args.format, **CONFIG)
    print(f"model built in {time.time() - t0:.0f} s", flush=True)
    ids, runner_up, top, second = [], [], [], []
    for b in range(args.batch):
        dec.prefill_random(b, PREFILL)
        t = o.start_token(SEED, b, CONFIG["vocab"])
        seq, ru, l1, l2 = [t], [], [], []
        for s in range(args.steps):
            t = dec.step(b, t)
            logits = dec.logits(b)
            rest = logits.copy()
            rest[t] = -np.inf
            r = int(np.argmax(rest))
            seq.append(t)
            ru.append(r)
            l1.append(float(logits[t]))
            l2.append(float(logits[r]))
        ids.append(seq)
        runner_up.append(ru)
        top.append(l1)
        second.append(l2)
        print(f"sequence {b}: {args.steps} steps, {time.time() - t0:.0f} s", flush=True)
        with open(out, "w") as f:
            json.dump({"config": CONFIG, "seed": SEED, "prefill": PREFILL, "steps": args.steps, "format": args.format,
                       "note": "ids[b][0] is the start token; ids[b][1:] the greedy steps; "
                               "runner_up[b][s], top[b][s], second[b][s]: the second-best token of "
                               "step s and the two largest logits",
                       "ids": ids, "runner_up": runner_up, "top": top, "second": second}, f)
    dec.close()


if __name__ == "__main__":
    main()
