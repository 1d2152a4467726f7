"""omni_qwen3_rope_attend (qwen3_rope + qwen3_attend in one launch) against
the two separate calls on the GPU, through the C ABI: the attention output
and the whole K/V cache after the call are bit-identical (the fused kernel
computes the rotary with the same device code, and takes the row's new key
from registers where the separate path reads back what qwen3_rope wrote),
and qkv is left as it was. The chain is also held to the oracle's chain
(oracle qwen3_rope, then oracle paged attention) at config 2's full size.
The new key's slot is filled with NaN before each call, so a kernel that
read it instead of the registers would not return finite values. For MHA
both paths run one K/V head per workgroup (the separate call could pick two,
a different summation order)."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits
from refs import bits_to_f64

pytestmark = pytest.mark.gpu
EPS, THETA = 1e-6, 1e6


def slots_of(c):
    """The page-table slot of each row's new key (position pos[n])."""
    return np.array([c.pages[c.indptr[n] + p // c.page] * c.page + p % c.page for n, p in enumerate(c.pos)],
                    np.int32)


def norms(seed):
    rng = np.random.default_rng(seed)
    return [W.f32_to_bf16_bits(1.0 + 0.2 * rng.standard_normal(128, dtype=np.float32)) for _ in range(2)]


def run_both(c, chunk=0, seed=0):
    """(separate: out, kv, qkv after), (fused: out, kv, qkv after), slots."""
    hq, hk = c.hq, c.hk
    qn, kn = norms(seed)
    slots = slots_of(c)
    kv0 = c.kv.copy()
    kv0.reshape(kv0.shape[0], -1)[slots] = 0x7FC0  # NaN where the new keys go
    plan = oa.decode_plan(c.rows, hq, hk, c.page, int(c.pos.max()) + 1, chunk)
    # The fused kernel takes one K/V head per workgroup; for MHA the separate
    # call may otherwise pick two (a different summation order), so both run one.
    plan.group_heads = 1 if hq == hk else 0
    ws = oa.workspace_for(plan)
    pos, sl, seq = dev_i32(c.pos), dev_i32(slots), dev_i32(c.seq)
    indptr, pages = dev_i32(c.indptr), dev_i32(c.pages)
    dqn, dkn = dev_bits(qn), dev_bits(kn)
    res = []
    for fused in (False, True):
        qkv, kv = dev_bits(c.qkv), dev_bits(kv0)
        out = torch.full((c.rows, hq * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        if fused:
            oa.qwen3_rope_attend(qkv, dqn, dkn, pos, sl, kv, indptr, pages, c.page, out, hq, hk, EPS, THETA, c.scale,
                                 plan, ws)
        else:
            oa.qwen3_rope(qkv, dqn, dkn, pos, sl, kv, c.rows, hq, hk, EPS, THETA)
            oa.qwen3_attend(qkv, kv, pos, seq, 0, indptr, pages, c.page, out, hq, hk, c.scale, plan, ws)
        torch.cuda.synchronize()
        res.append((host_bits(out), host_bits(kv), host_bits(qkv)))
    return res[0], res[1], (qn, kn, slots, kv0, plan)


def check_identical(c, chunk=0, seed=0, what=""):
    (o_s, kv_s, _), (o_f, kv_f, q_f), extra = run_both(c, chunk, seed)
    assert np.all(np.isfinite(bits_to_f64(o_f))), f"{what}: non-finite output"
    assert np.array_equal(o_f, o_s), f"{what}: output differs from qwen3_rope + qwen3_attend"
    assert np.array_equal(kv_f, kv_s), f"{what}: K/V cache differs"
    assert np.array_equal(q_f, c.qkv), f"{what}: qkv was written"
    return o_f, kv_f, extra


@pytest.mark.parametrize("hq,hk", [(16, 8), (32, 8), (8, 8)])
@pytest.mark.parametrize("page", [16, 12, 1])
def test_fused_equals_separate(hq, hk, page):
    """Lengths 1 .. 700 (splits of 128 keys: the new key in the first and in
    later splits, at every position of a 32-key tile)."""
    c = W.paged_decode_case(40, hq, hk, 1, 700, page=page, seed=hq * 100 + page, slack_pages=4)
    cap = (c.indptr[1:] - c.indptr[:-1]) * page
    c.pos[:4] = np.minimum([0, 31, 32, 127], cap[:4] - 1)  # one key; tile ends; a split's last key
    check_identical(c, chunk=128, seed=page, what=f"{hq}/{hk} page {page}")


@pytest.mark.parametrize("chunk", [0, 1024])
def test_fused_one_split_and_plan_chunk(chunk):
    """The plan's own chunk, and one split per row (no combine)."""
    c = W.paged_decode_case(24, 16, 8, 100, 1000, seed=5 + chunk, slack_pages=2)
    check_identical(c, chunk=chunk, seed=3, what=f"chunk {chunk}")


def test_fused_config2_full_size_vs_oracle(oracle):
    """Config 2 (64 rows, 16q/8kv, U[200, 2400] keys): fused = separate bit for
    bit, and both within tolerance of the oracle's rotary + attention chain,
    with the new keys' V bytes exact and the untouched slots unchanged."""
    c = W.config_case(2)
    o_f, kv_f, (qn, kn, slots, kv0, plan) = check_identical(c, what="config 2")
    q_want, kv_want = oracle.qwen3_rope(c.qkv, qn, kn, c.pos, slots, kv0, c.hq, c.hk, EPS, THETA)
    want = oracle.paged_attend(q_want, kv_want, c.pos, c.seq, 0, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                               nthreads=16)
    assert_close(o_f, want, what="config 2 fused vs oracle chain")
    untouched = np.setdiff1d(np.arange(kv_f.shape[0]), slots)
    assert np.array_equal(kv_f[untouched], kv0[untouched])
    v3g = kv_f.reshape(-1, 2 * c.hk, 128)[slots, c.hk:]
    v3w = kv_want.reshape(-1, 2 * c.hk, 128)[slots, c.hk:]
    assert np.array_equal(v3g, v3w)


def test_fused_rejects_head_group_plans():
    c = W.paged_decode_case(4, 16, 16, 50, 100, seed=1, slack_pages=1)
    plan = oa.decode_plan(4, 16, 16, 16, 100)
    plan.group_heads = 2
    qn, kn = norms(0)
    out = torch.zeros(4, 16 * 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(oa.OmniAttnError):
        oa.qwen3_rope_attend(dev_bits(c.qkv), dev_bits(qn), dev_bits(kn), dev_i32(c.pos), dev_i32(slots_of(c)),
                             dev_bits(c.kv), dev_i32(c.indptr), dev_i32(c.pages), 16, out, 16, 16, EPS, THETA, c.scale,
                             plan, oa.workspace_for(plan))


def test_fused_step_graph_replays():
    """The fused step captured once as a HIP graph and replayed with new
    positions, slots and inputs: each replay equals the eager call bit for bit."""
    hq, hk, rows = 16, 8, 12
    c = W.paged_decode_case(rows, hq, hk, 200, 1000, seed=3, slack_pages=2)
    qn, kn = (dev_bits(x) for x in norms(1))
    src, kv0 = dev_bits(c.qkv), dev_bits(c.kv)
    kv = kv0.clone()
    out = torch.zeros(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    pos, sl = dev_i32(c.pos), dev_i32(slots_of(c))
    indptr, pages = dev_i32(c.indptr), dev_i32(c.pages)
    plan = oa.decode_plan(rows, hq, hk, 16, 1000, 256)
    ws = oa.workspace_for(plan)

    def step(s):
        oa.qwen3_rope_attend(src, qn, kn, pos, sl, kv, indptr, pages, 16, out, hq, hk, EPS, THETA, c.scale, plan, ws,
                             s)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s)
    rng = np.random.default_rng(7)
    cap = (c.indptr[1:] - c.indptr[:-1]) * 16
    for rep in range(3):
        p = np.minimum(rng.integers(0, 1000, rows), cap - 1).astype(np.int32)
        c.pos = p
        pos.copy_(dev_i32(p)), sl.copy_(dev_i32(slots_of(c)))
        src.copy_(torch.randn(src.shape, device="cuda").to(torch.bfloat16))
        kv.copy_(kv0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got_out, got_kv = out.clone(), kv.clone()
        kv.copy_(kv0)
        out.zero_()
        step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(got_out.view(torch.int16), out.view(torch.int16)), f"replay {rep}: output"
        assert torch.equal(got_kv.view(torch.int16), kv.view(torch.int16)), f"replay {rep}: K/V"


PAGES = [1, 2, 3, 4, 8, 12, 16, 20, 24, 32, 48, 64]


@pytest.mark.parametrize("case", range(16))
def test_fused_sweep(case):
    """Seeded random shapes: GQA ratio, page size (powers of two and not),
    rows, lengths and split size drawn per case; fused = separate bit for bit."""
    rng = np.random.default_rng(3000 + case)
    hq, hk = [(16, 8), (32, 8), (8, 8), (32, 32), (16, 4), (8, 2)][rng.integers(0, 6)]
    page = int(rng.choice(PAGES))
    rows = int(rng.integers(1, 49))
    lo = int(rng.integers(1, 600))
    hi = lo + int(rng.integers(0, 1200))
    chunk = int(rng.choice([0, 128, 256, 512]))
    c = W.paged_decode_case(rows, hq, hk, lo, hi, page=page, seed=case, slack_pages=3)
    check_identical(c, chunk=chunk, seed=case,
                    what=f"fused case {case}: {hq}/{hk} page {page} rows {rows} len [{lo}, {hi}] chunk {chunk}")


# ------------------------------------------------------ FP8 ring (PersonaPlex)

COEF = float(np.float32(-np.log(10000.0) * 2.0 / 128))


def ring_slots_of(c):
    """The page-table slot of each row's ring index pos[n] % context."""
    out = []
    for n, p in enumerate(c.pos):
        t = int(p) % c.context
        out.append(c.pages[c.indptr[n] + t // c.page] * c.page + t % c.page)
    return np.asarray(out, np.int32)


def run_both_fp8(c, chunk=0, group_heads=0, fp8_plan=False):
    heads = c.hq
    slots = ring_slots_of(c)
    kv0 = c.kv.copy()
    kv0[slots] = 0x7F  # E4M3 NaN in K and V, NaN scales, where the new keys go
    plan = (oa.decode_plan_fp8(c.rows, heads, c.page, int(c.lens().max()), chunk) if fp8_plan else
            oa.decode_plan(c.rows, heads, heads, c.page, int(c.lens().max()), chunk))
    plan.group_heads = group_heads
    ws = oa.workspace_for(plan)
    pos, sl, seq = dev_i32(c.pos), dev_i32(slots), dev_i32(c.seq)
    indptr, pages = dev_i32(c.indptr), dev_i32(c.pages)
    res = []
    for fused in (False, True):
        qkv = dev_bits(c.qkv)
        kv = torch.from_numpy(np.ascontiguousarray(kv0)).cuda()
        out = torch.full((c.rows, heads * 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        if fused:
            oa.lm_rope_attend_fp8(qkv, pos, sl, kv, indptr, pages, c.page, out, heads, COEF, c.scale, c.context, plan,
                                  ws)
        else:
            oa.lm_rope(qkv, pos, sl, kv, c.rows, heads, COEF)
            oa.lm_attend_fp8(qkv, kv, pos, seq, 0, indptr, pages, c.page, out, heads, c.scale, c.context, plan, ws)
        torch.cuda.synchronize()
        res.append((host_bits(out), kv.cpu().numpy(), host_bits(qkv)))
    return res[0], res[1], (slots, kv0)


def check_identical_fp8(c, chunk=0, group_heads=0, what="", fp8_plan=False):
    (o_s, kv_s, _), (o_f, kv_f, q_f), extra = run_both_fp8(c, chunk, group_heads, fp8_plan)
    assert np.all(np.isfinite(bits_to_f64(o_f))), f"{what}: non-finite output"
    assert np.array_equal(o_f, o_s), f"{what}: output differs from lm_rope + lm_attend_fp8"
    assert np.array_equal(kv_f, kv_s), f"{what}: FP8 cache differs"
    assert np.array_equal(q_f, c.qkv), f"{what}: qkv was written"
    return o_f, kv_f, extra


@pytest.mark.parametrize("heads,page,gh", [(8, 16, 0), (8, 12, 2), (8, 1, 1), (32, 16, 0), (32, 16, 8), (16, 4, 4)])
def test_fused_fp8_equals_separate(heads, page, gh):
    """Rows of 1 .. 900 tokens over a 600-slot ring: rows past the ring take
    their new key at ring index pos % 600, in the middle of their keys; the
    others at their last key."""
    c = W.fp8_ring_case(40, heads, 1, 900, 600, page=page, seed=heads + page + gh, slack_pages=4)
    check_identical_fp8(c, chunk=128, group_heads=gh, what=f"fp8 {heads} heads page {page} gh {gh}")


def test_fused_fp8_config3_full_size_vs_oracle(oracle):
    """Config 3's shape over FP8 slots (128 rows, 32 heads, U[100, 3000], ring
    3000) on the FP8 plan (768-key splits, 8 heads per workgroup): fused =
    separate bit for bit, and within tolerance of the oracle's lm_rope +
    lm_attend_fp8 chain; the scatter's bytes equal the oracle's."""
    c = W.fp8_ring_case(128, 32, 100, 3000, 3000, seed=3000, slack_pages=4)
    o_f, kv_f, (slots, kv0) = check_identical_fp8(c, what="config 3 fp8", fp8_plan=True)
    q_want, kv_want = oracle.lm_rope(c.qkv, c.pos, slots, kv0, 32, COEF)
    want = oracle.lm_attend_fp8(q_want, kv_want, c.pos, c.seq, 0, c.indptr, c.pages, 16, 32, c.scale, 3000,
                                nthreads=16)
    assert_close(o_f, want, what="config 3 fp8 fused vs oracle chain")
    untouched = np.setdiff1d(np.arange(kv_f.shape[0]), slots)
    assert np.array_equal(kv_f[untouched], kv0[untouched])


@pytest.mark.parametrize("case", range(12))
def test_fused_fp8_sweep(case):
    rng = np.random.default_rng(4000 + case)
    heads = int(rng.choice([2, 4, 8, 16, 32]))
    page = int(rng.choice(PAGES))
    rows = int(rng.integers(1, 41))
    lo = int(rng.integers(1, 600))
    hi = lo + int(rng.integers(0, 1200))
    context = int(rng.integers(1, hi + 1))
    chunk = int(rng.choice([0, 128, 256, 512]))
    c = W.fp8_ring_case(rows, heads, lo, hi, context, page=page, seed=case, slack_pages=3)
    check_identical_fp8(c, chunk=chunk, what=f"fp8 fused case {case}: {heads} heads page {page} rows {rows} "
                        f"len [{lo}, {hi}] ctx {context} chunk {chunk}")
