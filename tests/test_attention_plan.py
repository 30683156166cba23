"""The decode attention's scratch sizing (qwenscriber_amd/csrc/
attention_plan.h) on the CPU: qwenscriber_amd/sanitize/plan_check.cpp, built
with g++ (Makefile `plan_check`, no device code), walks the head layouts the
kernels are built for, device sizes, capacities and batches, and checks that
the bytes each caller allocates before it knows the launch form (the
decoder at create, the prefill per chunk, the attention entry points) hold
the records of every range the launch then writes. A buffer sized for the
plain form's ranges but launched in the decoder form is the fault this pins
(its range records ran past the buffer's end)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "qwenscriber_amd", "build", "plan_check")


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_scratch_holds_every_launched_range():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "qwenscriber_amd"), "plan_check"], check=True)
    run = subprocess.run([CHECK], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-2000:]
    assert " 0 failures" in run.stdout, run.stdout
