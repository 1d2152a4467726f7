"""Seeded random sweeps of every attention kernel against the CPU oracle:
shapes, GQA ratios, page sizes (powers of two and not), lengths, splits and modes drawn per case
(ragged prefill rows also through the split-K decode kernel)
from a generator seeded by the case number, so any failure names a case
that reruns exactly. Sizes stay small enough for the oracle to finish in
well under a second per case."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits

pytestmark = pytest.mark.gpu

CASES = range(24)
# Page sizes drawn: powers of two (shift-and-mask kernels) and others (the
# multiply-high division kernels; 12, 24 and 48 keep the scalar page-id paths
# of the decode, FP8 and prefill loaders, 3 and 20 the per-lane ones).
PAGES = [1, 2, 3, 4, 8, 12, 16, 20, 24, 32, 48, 64]


def _paged_oracle(oracle, c):
    return oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                               context=c.context, nthreads=16)


@pytest.mark.parametrize("case", CASES)
def test_decode_sweep(oracle, case):
    rng = np.random.default_rng(1000 + case)
    lm = bool(rng.integers(0, 4) == 0)  # lm_attend: MHA with a ring cap
    if lm:
        hq = hk = int(rng.choice([4, 8, 32]))
    else:
        hq, hk = [(16, 8), (32, 8), (8, 8), (32, 32), (16, 4), (8, 2)][rng.integers(0, 6)]
    page = int(rng.choice(PAGES))
    rows = int(rng.integers(1, 49))
    lo = int(rng.integers(1, 600))
    hi = lo + int(rng.integers(0, 1200))
    context = int(rng.integers(1, hi + 1)) if lm else 0
    chunk = int(rng.choice([0, 128, 256, 512]))
    c = W.paged_decode_case(rows, hq, hk, lo, hi, page=page, seed=case, context=context, slack_pages=3)
    what = f"decode case {case}: {hq}/{hk} page {page} rows {rows} len [{lo}, {hi}] ctx {context} chunk {chunk}"
    plan = oa.decode_plan(rows, hq, hk, page, int(c.lens().max()), chunk)
    out = torch.zeros(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    args = (dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 0, dev_i32(c.indptr), dev_i32(c.pages),
            page, out)
    if lm:
        oa.lm_attend(*args, hq, c.scale, context, plan, oa.workspace_for(plan))
    else:
        oa.qwen3_attend(*args, hq, hk, c.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(host_bits(out), _paged_oracle(oracle, c), what=what)


@pytest.mark.parametrize("case", CASES)
def test_fp8_decode_sweep(oracle, case):
    rng = np.random.default_rng(2000 + case)
    heads = int(rng.choice([2, 4, 8, 16, 32]))
    page = int(rng.choice(PAGES))
    rows = int(rng.integers(1, 41))
    lo = int(rng.integers(1, 500))
    hi = lo + int(rng.integers(0, 1000))
    context = int(rng.integers(1, hi + 1))
    chunk = int(rng.choice([0, 128, 512]))
    gh = int(rng.choice([g for g in (0, 1, 2, 4, 8) if g == 0 or heads % g == 0]))
    c = W.fp8_ring_case(rows, heads, lo, hi, context, page=page, seed=case, slack_pages=2)
    what = f"fp8 case {case}: heads {heads} page {page} rows {rows} len [{lo}, {hi}] ctx {context} chunk {chunk} gh {gh}"
    plan = oa.decode_plan(rows, heads, heads, page, int(c.lens().max()), chunk)
    plan.group_heads = gh
    out = torch.zeros(rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    oa.lm_attend_fp8(dev_bits(c.qkv), torch.from_numpy(np.ascontiguousarray(c.kv)).cuda(), dev_i32(c.pos),
                     dev_i32(c.seq), 0, dev_i32(c.indptr), dev_i32(c.pages), page, out, heads, c.scale, context, plan,
                     oa.workspace_for(plan))
    torch.cuda.synchronize()
    want = oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, page, heads, c.scale, context,
                                nthreads=16)
    assert_close(host_bits(out), want, what=what)


@pytest.mark.parametrize("case", CASES)
def test_prefill_sweep(oracle, case):
    rng = np.random.default_rng(3000 + case)
    hk = int(rng.choice([1, 2, 4, 8]))
    hq = hk * int(rng.choice([1, 2, 4, 8]))
    page = int(rng.choice(PAGES))
    nseq = int(rng.integers(1, 5))
    new_hi = int(rng.integers(1, 300))
    cached_hi = int(rng.integers(0, 300))
    c = W.ragged_prefill_case(nseq, hq, hk, 1, new_hi, 0, cached_hi, page=page, seed=case, slack_pages=2)
    what = f"prefill case {case}: {hq}/{hk} page {page} seqs {nseq} new <= {new_hi} cached <= {cached_hi}"
    pf = oa.prefill_plan(c.rows, hq, hk, page, c.seq, c.pos)
    out = torch.zeros(c.rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.prefill_run(pf, dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), dev_i32(c.indptr),
                   dev_i32(c.pages), out, c.scale)
    torch.cuda.synchronize()
    want = _paged_oracle(oracle, c)
    assert_close(host_bits(out), want, what=what)
    if hq // hk <= 4:  # the same ragged rows through the split-K decode kernel (qwen3_attend, ragged = 1)
        plan = oa.decode_plan(c.rows, hq, hk, page, int(c.pos.max()) + 1, int(rng.choice([0, 128, 256])))
        out2 = torch.zeros_like(out)
        oa.qwen3_attend(dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 1, dev_i32(c.indptr),
                        dev_i32(c.pages), page, out2, hq, hk, c.scale, plan, oa.workspace_for(plan))
        torch.cuda.synchronize()
        assert_close(host_bits(out2), want, what=f"{what} (decode kernel, chunk {plan.chunk})")
    # The plan's exact_p on the same rows: within tolerance of the oracle, and
    # (f32-P numerics) nearer to it on average than P rounded to bf16.
    pf_x = oa.prefill_plan(c.rows, hq, hk, page, c.seq, c.pos, exact_p=True)
    out3 = torch.zeros_like(out)
    oa.prefill_run(pf_x, dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), dev_i32(c.indptr),
                   dev_i32(c.pages), out3, c.scale)
    torch.cuda.synchronize()
    _, mean_x = assert_close(host_bits(out3), want, what=f"{what} (exact_p)")
    _, mean_r = assert_close(host_bits(out), want, what=what)
    assert mean_x <= mean_r * 1.05 + 1e-7, (what, mean_x, mean_r)


@pytest.mark.parametrize("case", CASES)
def test_dit_sweep(oracle, case):
    rng = np.random.default_rng(4000 + case)
    hk = int(rng.choice([1, 2, 4, 8]))
    hq = hk * int(rng.choice([1, 2, 4, 8]))
    q_len = int(rng.integers(1, 400))
    kv_len = int(rng.integers(1, 500))
    causal = int(rng.integers(0, 2))
    batch = int(rng.integers(1, 4))
    use_ws = bool(rng.integers(0, 2))
    c = W.dense_case(hq, hk, q_len, kv_len, causal, batch=batch, seed=case)
    what = f"dit case {case}: {hq}/{hk} q {q_len} kv {kv_len} causal {causal} batch {batch} ws {use_ws}"
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(batch, q_len, hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([kv_len], np.int32))
    strides = (q_len * c.q_stride, kv_len * hk * 128, q_len * hq * 128)
    if use_ws:
        oa.hidream_attend_ws(q, k, v, out, q_len, kvl, c.q_stride, causal, c.scale_log2, hq, hk, batch, *strides,
                             oa.hidream_workspace())
    else:
        oa.hidream_attend_batched(q, k, v, out, q_len, kvl, c.q_stride, causal, c.scale_log2, hq, hk, batch, *strides)
    torch.cuda.synchronize()
    got = host_bits(out)
    for b in range(batch):
        want = oracle.dense_attend(np.ascontiguousarray(c.q[b]), np.ascontiguousarray(c.k[b]),
                                   np.ascontiguousarray(c.v[b]), q_len, kv_len, c.q_stride, hq, hk, causal,
                                   c.scale_log2, nthreads=16)
        assert_close(got[b], want, what=f"{what} (batch {b})")
