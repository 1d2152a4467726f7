"""A whole step captured once in a HIP graph, as the engines capture one per
batch bucket, and replayed with new positions, slots, key counts and inputs:
rotary + K/V scatter then attention (bf16 qwen3 decode, FP8 lm decode, and the
HiDream DiT step with the tail-split workspace). Every replay must equal the
same step run eagerly, bit for bit (the same kernels on the same inputs), with
eager work and synchronisations between replays."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import dev_i32

pytestmark = pytest.mark.gpu


def _positions(c, rng):
    """New decode positions inside each row's pages, and the slot of each."""
    cap = (c.indptr[1:] - c.indptr[:-1]) * c.page
    pos = np.minimum(rng.integers(0, 1000, c.rows), cap - 1).astype(np.int32)
    slots = np.array([c.pages[c.indptr[n] + p // c.page] * c.page + p % c.page for n, p in enumerate(pos)], np.int32)
    return pos, slots


def test_qwen3_step_graph_replays():
    hq, hk, rows = 16, 8, 12
    c = W.paged_decode_case(rows, hq, hk, 200, 1000, seed=3, values=None, slack_pages=2)
    gen = torch.Generator(device="cuda").manual_seed(1)
    src = torch.randn(rows, (hq + 2 * hk) * 128, device="cuda", generator=gen).to(torch.bfloat16)
    kv0 = torch.randn(c.num_pages * 16, 2 * hk * 128, device="cuda", generator=gen).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)
    qkv, kv = torch.empty_like(src), kv0.clone()
    out = torch.zeros(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    pos, slots = dev_i32(np.zeros(rows, np.int32)), dev_i32(np.zeros(rows, np.int32))
    seq, indptr, pages = dev_i32(np.arange(rows)), dev_i32(c.indptr), dev_i32(c.pages)
    plan = oa.decode_plan(rows, hq, hk, 16, 1000, 256)
    ws = oa.workspace_for(plan)

    def step(s):
        qkv.copy_(src)
        oa.qwen3_rope(qkv, qn, kn, pos, slots, kv, rows, hq, hk, 1e-6, 1e6, s)
        oa.qwen3_attend(qkv, kv, pos, seq, 0, indptr, pages, 16, out, hq, hk, 128 ** -0.5, plan, ws, s)

    rng = np.random.default_rng(7)
    p0, s0 = _positions(c, rng)
    pos.copy_(dev_i32(p0)), slots.copy_(dev_i32(s0))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)  # warm
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s)
    for rep in range(4):
        p, sl = _positions(c, rng)
        src.copy_(torch.randn(src.shape, device="cuda", generator=gen).to(torch.bfloat16))
        pos.copy_(dev_i32(p)), slots.copy_(dev_i32(sl))
        kv.copy_(kv0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_out, got_kv, got_q = out.clone(), kv.clone(), qkv.clone()
        kv.copy_(kv0)
        out.zero_()
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got_out.view(torch.int16), out.view(torch.int16)), f"replay {rep}: attention output"
        assert torch.equal(got_kv.view(torch.int16), kv.view(torch.int16)), f"replay {rep}: K/V scatter"
        assert torch.equal(got_q.view(torch.int16), qkv.view(torch.int16)), f"replay {rep}: rotated q"


def test_lm_fp8_step_graph_replays():
    heads, rows = 8, 10
    c = W.paged_decode_case(rows, heads, heads, 200, 1000, seed=4, values=None, slack_pages=2)
    gen = torch.Generator(device="cuda").manual_seed(2)
    src = torch.randn(rows, 3 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    kv0 = torch.randint(0, 120, (c.num_pages * 16, W.fp8_slot_bytes(heads)), dtype=torch.uint8, device="cuda")
    kv0[:, 2 * heads * 128:] = torch.full((heads * 2,), 0.01, device="cuda").view(torch.uint8).repeat(len(kv0), 1)
    qkv, kv = torch.empty_like(src), kv0.clone()
    out = torch.zeros(rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    pos, slots = dev_i32(np.zeros(rows, np.int32)), dev_i32(np.zeros(rows, np.int32))
    seq, indptr, pages = dev_i32(np.arange(rows)), dev_i32(c.indptr), dev_i32(c.pages)
    plan = oa.decode_plan(rows, heads, heads, 16, 1000, 256)
    ws = oa.workspace_for(plan)
    coef = float(np.float32(-np.log(10000.0) * 2.0 / 128))

    def step(s):
        qkv.copy_(src)
        oa.lm_rope(qkv, pos, slots, kv, rows, heads, coef, s)
        oa.lm_attend_fp8(qkv, kv, pos, seq, 0, indptr, pages, 16, out, heads, 128 ** -0.5, 3000, plan, ws, s)

    rng = np.random.default_rng(8)
    p0, s0 = _positions(c, rng)
    pos.copy_(dev_i32(p0)), slots.copy_(dev_i32(s0))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s)
    for rep in range(4):
        p, sl = _positions(c, rng)
        src.copy_(torch.randn(src.shape, device="cuda", generator=gen).to(torch.bfloat16))
        pos.copy_(dev_i32(p)), slots.copy_(dev_i32(sl))
        kv.copy_(kv0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_out, got_kv = out.clone(), kv.clone()
        kv.copy_(kv0)
        out.zero_()
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got_out.view(torch.int16), out.view(torch.int16)), f"replay {rep}: attention output"
        assert torch.equal(got_kv, kv), f"replay {rep}: FP8 scatter"


def test_dit_step_graph_replays():
    """HiDream's rotary + K/V write then the batched attention with the tail
    split (workspace + merge), captured once and replayed with new inputs and
    new key counts through *kv_len_at, as the diffusion loop replays one graph
    per step."""
    hq, hk, rows, text = 32, 8, 300, 100
    slots_n = text + rows
    c = W.rope_case("hidream", rows, hq, hk, seed=5, pos_hi=4352)
    gen = torch.Generator(device="cuda").manual_seed(2)
    ld = c.ld
    src = torch.randn(rows, ld, device="cuda", generator=gen).to(torch.bfloat16)
    k0 = torch.randn(slots_n, hk * 128, device="cuda", generator=gen).to(torch.bfloat16)
    v0 = torch.randn(slots_n, hk * 128, device="cuda", generator=gen).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)
    qkv, kc, vc = torch.empty_like(src), k0.clone(), v0.clone()
    out = torch.zeros(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    pos = dev_i32(c.pos)
    slots = dev_i32(text + np.arange(rows, dtype=np.int32))  # image rows after the text keys
    kvl = dev_i32(np.array([slots_n], np.int32))
    ws = oa.hidream_workspace()
    scale_log2 = 128 ** -0.5 * 1.4426950408889634

    def step(s):
        qkv.copy_(src)
        oa.hidream_qk_rope(qkv, ld, qn, kn, pos, slots, kc, vc, rows, hq, hk, 20, 1e-6, 1e4, s)
        oa.hidream_attend_ws(qkv, kc, vc, out, rows, kvl, ld, 0, scale_log2, hq, hk, 1, rows * ld,
                             slots_n * hk * 128, rows * hq * 128, ws, s)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)  # warm
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s)
    for rep, n_keys in enumerate((slots_n, 350, 257, 129)):
        src.copy_(torch.randn(src.shape, device="cuda", generator=gen).to(torch.bfloat16))
        kvl.copy_(dev_i32(np.array([n_keys], np.int32)))
        kc.copy_(k0), vc.copy_(v0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_out, got_k, got_q = out.clone(), kc.clone(), qkv.clone()
        kc.copy_(k0), vc.copy_(v0)
        out.zero_()
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got_out.view(torch.int16), out.view(torch.int16)), f"replay {rep}: attention output"
        assert torch.equal(got_k.view(torch.int16), kc.view(torch.int16)), f"replay {rep}: K cache"
        assert torch.equal(got_q.view(torch.int16), qkv.view(torch.int16)), f"replay {rep}: rotated q"


def test_lm_bf16_head_group_graph_replays():
    """The headline's kernel (MHA over bf16 slots, two heads per workgroup)
    captured once and replayed with new positions and inputs, each replay
    equal bit for bit to the same call run eagerly."""
    heads, rows = 8, 12
    c = W.paged_decode_case(rows, heads, heads, 200, 1500, seed=6, values=None, slack_pages=2)
    gen = torch.Generator(device="cuda").manual_seed(3)
    qkv = torch.randn(rows, 3 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    kv = torch.randn(c.num_pages * 16, 2 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    out = torch.zeros(rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    pos = dev_i32(np.zeros(rows, np.int32))
    seq, indptr, pages = dev_i32(np.arange(rows)), dev_i32(c.indptr), dev_i32(c.pages)
    plan = oa.decode_plan(rows, heads, heads, 16, 1500, 256)
    plan.group_heads = 2
    ws = oa.workspace_for(plan)

    def step(s):
        oa.lm_attend(qkv, kv, pos, seq, 0, indptr, pages, 16, out, heads, 128 ** -0.5, 1200, plan, ws, s)

    rng = np.random.default_rng(9)
    pos.copy_(dev_i32(_positions(c, rng)[0]))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s)
    for rep in range(4):
        pos.copy_(dev_i32(_positions(c, rng)[0]))
        qkv.copy_(torch.randn(qkv.shape, device="cuda", generator=gen).to(torch.bfloat16))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        out.zero_()
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), out.view(torch.int16)), f"replay {rep}: attention output"
