"""omni_qwen3_attend_noalloc (the allocation-free decode entry point, static
per-GPU scratch) against omni_qwen3_attend with a caller workspace, through
the C ABI: two calls in a row on one GPU, the second with fewer rows and
shorter rows (the scratch keeps the first call's partials), each compared
bit for bit (the same kernels on the same inputs), and both with the oracle.
Also the size limit: a plan above the scratch is rejected before launch, and
the first call of a process made under HIP graph capture."""
import ctypes

import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import DevPaged, assert_close, host_bits

pytestmark = pytest.mark.gpu


def _both(case, chunk):
    d = DevPaged(case)
    want = d.decode(chunk=chunk)
    c = case
    plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, int(c.lens().max()), chunk)
    assert plan.splits > 1 and plan.workspace_bytes <= (16 << 20)
    out = torch.full((c.rows, c.hq * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend_noalloc(d.qkv, d.kv, d.pos, d.seq, c.ragged, d.indptr, d.pages, c.page, out, c.hq, c.hk, c.scale,
                            plan)
    torch.cuda.synchronize()
    return host_bits(out), want


# First in this file on purpose: in a process that has made no allocation-free
# call yet, this one makes the library look up its static scratch while the
# stream is being captured.
def test_noalloc_first_call_inside_graph_capture():
    """The entry point's advertised use: captured into a HIP graph (here its
    first call in the process, so the per-device scratch lookup happens under
    capture), replayed twice with eager work in between, each replay equal
    bit for bit to omni_qwen3_attend with a caller workspace."""
    c = W.paged_decode_case(24, 16, 8, 100, 1500, seed=73)
    d = DevPaged(c)
    plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, int(c.lens().max()), 256)
    assert plan.splits > 1
    want = d.decode(chunk=256)
    out = torch.full((c.rows, c.hq * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        oa.qwen3_attend_noalloc(d.qkv, d.kv, d.pos, d.seq, c.ragged, d.indptr, d.pages, c.page, out, c.hq, c.hk,
                                c.scale, plan)
    for rep in range(2):
        out.fill_(float("nan"))
        d.decode(chunk=256)  # eager work (the workspace call) between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host_bits(out), want), f"replay {rep} differs from the workspace call"


def test_noalloc_matches_workspace_call_twice(oracle):
    big = W.paged_decode_case(48, 16, 8, 200, 2400, seed=71)
    small = W.paged_decode_case(5, 32, 8, 30, 700, seed=72)
    for c, chunk in ((big, 256), (small, 128)):
        got, want = _both(c, chunk)
        assert np.array_equal(got, want), f"noalloc differs from the workspace call ({c.rows} rows)"
        ref = oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                                  nthreads=16)
        assert_close(got, ref, what=f"noalloc vs oracle ({c.rows} rows)")


def test_noalloc_rejects_plans_above_the_scratch():
    plan = oa.decode_plan(4096, 32, 32, 16, 65536, 128)
    assert plan.workspace_bytes > (16 << 20)
    fake = ctypes.c_void_p(256)
    rc = oa.load().omni_qwen3_attend_noalloc(fake, fake, fake, None, 0, fake, fake, 16, fake, 32, 32, 0.1,
                                             ctypes.byref(plan), None)
    assert rc == oa.EWORKSPACE
    assert "static scratch" in oa.load().omni_attn_last_error().decode()
