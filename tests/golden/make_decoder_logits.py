#!/usr/bin/env python3
"""Writes tests/golden/decoder_1p7b_logits.json: teacher-forced logits of the
CPU oracle (oracle/qwref.c, decoder.zig:133-287) at the configs[4] decoder
shape, at chosen steps of every sequence of decoder_1p7b_ids.json (same
model, seed, prefill and start tokens). Step s feeds ids[b][s] (after steps
0 .. s-1 fed theirs) and records, of the resulting 151936 logits: the 16
largest (index and value), every 1187th value (128 values: a fixed sample
across the vocabulary) and the rms of all of them.

Usage: python3 tests/golden/make_decoder_logits.py [--steps 0,1,64,127,255] [--batch 16]
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

HERE = os.path.dirname(os.path.abspath(__file__))
SAMPLE_STRIDE = 1187
SAMPLES = 128
TOP = 16


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", default="0,1,64,127,255")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--out", default=os.path.join(HERE, "decoder_1p7b_logits.json"))
    args = ap.parse_args()
    with open(os.path.join(HERE, "decoder_1p7b_ids.json")) as f:
        golden = json.load(f)
    cfg, seed, prefill = golden["config"], golden["seed"], golden["prefill"]
    steps = sorted(int(v) for v in args.steps.split(","))
    o.set_threads(args.threads)
    t0 = time.time()
    dec = o.Decoder(seed, args.batch, **cfg)
    print(f"model built in {time.time() - t0:.0f} s", flush=True)
    records = []
    for b in range(args.batch):
        dec.prefill_random(b, prefill)
        seq = []
        for s in range(steps[-1] + 1):
            dec.forward(b, golden["ids"][b][s], s in steps)
            if s not in steps:
                continue
            logits = dec.logits(b)
            top = np.argsort(-logits, kind="stable")[:TOP]
            seq.append({"step": s, "top_index": [int(i) for i in top], "top_value": [float(logits[i]) for i in top],
                        "sample": [float(v) for v in logits[::SAMPLE_STRIDE][:SAMPLES]],
                        "rms": float(np.sqrt(np.mean(logits.astype(np.float64) ** 2)))})
        records.append(seq)
        print(f"sequence {b}: {time.time() - t0:.0f} s", flush=True)
    with open(args.out, "w") as f:
        json.dump({"config": cfg, "seed": seed, "prefill": prefill, "steps": steps,
                   "sample_stride": SAMPLE_STRIDE, "samples": SAMPLES,
                   "note": "records[b][i]: logits after feeding ids[b][steps[i]] of decoder_1p7b_ids.json at "
                           "position prefill + steps[i], every earlier id fed before it (teacher forced)",
                   "records": records}, f)
    dec.close()


if __name__ == "__main__":
    main()
