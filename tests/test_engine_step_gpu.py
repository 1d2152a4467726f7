"""The boundary driven from native code on the GPU: tests/c/engine_step.cpp
runs a Qwen3-TTS-style decode step (row builder, rotary + K/V scatter, paged
attention) over the C ABI with no Python in the loop, captures the step once
as a HIP graph and replays it for later steps, and checks every replay
against an eager run (bit-identical) and the CPU oracle (to the tolerance).
tests/c/engine_prefill.cpp does the same for a chunked ragged prefill (host
prefill plan, MFMA prefill with and without the plan's exact_p, and decode
on the same rows) and a HiDream step
(M-RoPE into the K/V caches, DiT attention replayed as a HIP graph with a
changed key count)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "c", "bin")


def _run(name):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):  # built by __graft_entry__.build(); build here if it is missing
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "c"), "engine"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and f"{name}: ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_engine_step_graph_per_bucket():
    _run("engine_step")


def test_engine_prefill_and_dit_step():
    _run("engine_prefill")
