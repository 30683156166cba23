"""The untrusted-byte parsers (shard.cpp: container.zig File.parse, find,
verifyChecksum; config.cpp: model_config.parse) built for the host with
AddressSanitizer and UndefinedBehaviorSanitizer (qwenscriber_amd/Makefile
`sanitize`, g++, no device code) and run over valid shards and
configurations and thousands of deterministic mutations of each (flipped
bytes, extreme length and offset fields, truncation, trailing bytes). The
run fails on any sanitizer report. No device is needed."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import model_config as mc
from oracle import oracle as o
from oracle import shard as sh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "qwenscriber_amd", "build", "parsers_sanitized")


def inputs(tmp):
    files = []

    def write(name, data):
        path = os.path.join(tmp, name)
        with open(path, "wb") as f:
            f.write(data)
        files.append(path)

    for fmt, rows, cols in ((o.Q4, 64, 64), (o.Q5, 64, 128), (o.Q8, 2, 64)):
        vals = o.normal(rows * cols, 7, fmt, 0.02).reshape(rows, cols)
        s, d = o.quantize_rows(fmt, vals)
        write(f"one_{fmt}.qw", sh.build([dict(kind=sh.KIND_AUDIO_CONV1_WEIGHT, layer=0, format=fmt, dims=(rows, cols),
                                              payload=sh.quantized_payload(fmt, s, d))]))
    # Several tensors over layers, element formats and ranks.
    tensors = []
    for layer in range(3):
        s, d = o.quantize_rows(o.Q4, o.normal(64 * 64, 8, layer, 0.02).reshape(64, 64))
        tensors.append(dict(kind=33, layer=layer + 1, format=o.Q4, dims=(64, 64),
                            payload=sh.quantized_payload(o.Q4, s, d)))
        tensors.append(dict(kind=37, layer=layer + 1, format=0, dims=(64,),
                            payload=np.ones(64, np.float32).tobytes()))
    write("many.qw", sh.build(tensors))
    write("0p6b.bin", mc.pack(mc.CONFIG_0P6B))
    write("1p7b.bin", mc.pack(mc.CONFIG_1P7B))
    write("empty.bin", b"")
    return files


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_parsers_under_asan_and_ubsan(tmp_path):
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "qwenscriber_amd"), "sanitize"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([HARNESS, "4000", *inputs(str(tmp_path))], capture_output=True, text=True, env=env,
                         timeout=600)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-4000:]
    assert "checked" in run.stdout
