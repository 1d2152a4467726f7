"""Paged decode on the GPU against the CPU oracle (qwen3_attend / lm_attend
semantics), plus the bit-exact page-table properties."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import DevPaged, assert_close, dev_bits, dev_i32, host_bits

pytestmark = pytest.mark.gpu


def oracle_out(oracle, c, threads=8):
    return oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                               context=c.context, nthreads=threads)


@pytest.mark.parametrize("chunk", [0, 128, 256])
def test_config1_parity(oracle, chunk):
    c = W.config_case(1)
    got = DevPaged(c).decode(chunk=chunk)
    assert_close(got, oracle_out(oracle, c), what=f"config1 chunk={chunk}")


@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 4), (16, 4), (32, 32)])
@pytest.mark.parametrize("lo,hi", [(1, 40), (1, 1), (500, 1300)])
def test_head_shapes_and_lengths(oracle, hq, hk, lo, hi):
    c = W.paged_decode_case(7, hq, hk, lo, hi, seed=hq + hk + lo, slack_pages=3)
    got = DevPaged(c).decode(chunk=128)
    assert_close(got, oracle_out(oracle, c), what=f"{hq}/{hk} len[{lo},{hi}]")


def test_single_key_rows_are_exact(oracle):
    c = W.paged_decode_case(6, 8, 4, 1, 1, seed=3)
    assert np.array_equal(DevPaged(c).decode(), oracle_out(oracle, c))


def test_ragged_rows(oracle):
    c = W.ragged_prefill_case(4, 16, 8, 1, 70, 0, 600, seed=11)
    got = DevPaged(c).decode(chunk=128)
    assert_close(got, oracle_out(oracle, c), what="ragged")


def test_lm_ring_cap(oracle):
    c = W.paged_decode_case(9, 8, 8, 100, 3000, seed=12, context=700)
    past = c.pos + 1 >= 700  # rows whose pages already hold a full ring move past it
    c.pos = np.where(past, c.pos + np.random.default_rng(1).integers(0, 5000, c.rows), c.pos).astype(np.int32)
    got = DevPaged(c).decode(lm=True, max_len=700)
    assert_close(got, oracle_out(oracle, c), what="ring")


def test_rows_longer_than_plan_bound(oracle):
    c = W.paged_decode_case(5, 8, 4, 600, 900, seed=13)
    got = DevPaged(c).decode(chunk=128, max_len=256)  # the last split absorbs the overflow
    assert_close(got, oracle_out(oracle, c), what="overflow")


def test_lastlen_encoding_is_identical():
    c = W.paged_decode_case(8, 16, 8, 1, 500, seed=14)
    d = DevPaged(c)
    a = d.decode(chunk=128)
    last = ((c.pos % 16) + 1).astype(np.int32)
    plan = oa.decode_plan(c.rows, 16, 8, 16, int(c.lens().max()), 128)
    ws = oa.workspace_for(plan)
    d.out.zero_()
    oa.decode_lastlen(d.qkv, d.kv, dev_i32(last), d.seq, 0, d.indptr, d.pages, 16, d.out, 16, 8, c.scale, plan, ws)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(d.out), a)


@pytest.mark.parametrize("page", [16, 1, 3, 12, 24, 48])
def test_gather_bit_exact(oracle, page):
    """The page-table gather is byte-equal to the oracle's, for power-of-two
    pages and for the sizes only the division path serves."""
    c = W.paged_decode_case(6, 8, 4, 1, 700, page=page, seed=15, slack_pages=5)
    d = DevPaged(c)
    lens = c.lens().astype(np.int32)
    ids = np.array([3, 0, 5, 1], np.int32)
    sel = lens[ids]
    out_indptr = np.concatenate([[0], np.cumsum(sel)]).astype(np.int32)
    out = torch.zeros(int(out_indptr[-1]), 2 * c.hk * 128, dtype=torch.bfloat16, device="cuda")
    oa.gather_kv(d.kv, c.hk, d.indptr, d.pages, page, dev_i32(ids), dev_i32(sel), dev_i32(out_indptr), out)
    torch.cuda.synchronize()
    got = host_bits(out)
    for j, s in enumerate(ids):
        want = oracle.gather_kv(c.kv, c.hk, c.indptr, c.pages, page, int(s), int(sel[j]))
        assert np.array_equal(got[out_indptr[j]:out_indptr[j + 1]], want)


@pytest.mark.parametrize("page", [12, 24])
def test_page_permutation_is_bit_identical_any_page(page):
    """Non-power-of-two pages: permuting the physical pages (and the table with
    them) leaves the decode output bit-identical."""
    c = W.paged_decode_case(6, 16, 8, 50, 900, page=page, seed=16, slack_pages=9)
    a = DevPaged(c).decode(chunk=256)
    perm = np.random.default_rng(2).permutation(c.num_pages).astype(np.int32)
    kv2 = np.empty_like(c.kv)
    kv2.reshape(c.num_pages, page, -1)[perm] = c.kv.reshape(c.num_pages, page, -1)
    c.kv, c.pages = kv2, perm[c.pages].copy()
    assert np.array_equal(DevPaged(c).decode(chunk=256), a)


def test_page_permutation_is_bit_identical():
    c = W.paged_decode_case(6, 16, 8, 50, 900, seed=16, slack_pages=9)
    a = DevPaged(c).decode(chunk=256)
    perm = np.random.default_rng(2).permutation(c.num_pages).astype(np.int32)
    kv2 = np.empty_like(c.kv)
    src = c.kv.reshape(c.num_pages, 16, -1)
    kv2.reshape(c.num_pages, 16, -1)[perm] = src
    c.kv, c.pages = kv2, perm[c.pages].copy()
    assert np.array_equal(DevPaged(c).decode(chunk=256), a)


def test_row_output_independent_of_neighbours():
    c = W.paged_decode_case(8, 8, 4, 10, 900, seed=17)
    a = DevPaged(c).decode(chunk=128, max_len=900)
    c2 = W.paged_decode_case(8, 8, 4, 10, 900, seed=18)
    # Row 3 keeps its query, pages and K/V; every other row changes.
    c2.kv = np.concatenate([c2.kv, c.kv])
    off = c2.num_pages
    s = 3
    n3 = c.indptr[s + 1] - c.indptr[s]
    pages3 = c.pages[c.indptr[s]:c.indptr[s + 1]] + off
    pages = np.concatenate([c2.pages[: c2.indptr[s]], pages3, c2.pages[c2.indptr[s + 1]:]]).astype(np.int32)
    indptr = c2.indptr.copy()
    indptr[s + 1:] += n3 - (c2.indptr[s + 1] - c2.indptr[s])
    c2.pages, c2.indptr, c2.num_pages = pages, indptr, c2.num_pages + c.num_pages
    c2.pos[s] = c.pos[s]
    c2.qkv[s] = c.qkv[s]
    b = DevPaged(c2).decode(chunk=128, max_len=900)
    assert np.array_equal(a[s], b[s])


def test_graph_replay_with_new_lengths(oracle):
    c = W.paged_decode_case(16, 16, 8, 10, 1200, seed=19)
    d = DevPaged(c)
    plan = oa.decode_plan(c.rows, 16, 8, 16, 1200, 128)
    ws = oa.workspace_for(plan)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        oa.qwen3_attend(d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, 16, d.out, 16, 8, c.scale, plan, ws, s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        oa.qwen3_attend(d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, 16, d.out, 16, 8, c.scale, plan, ws, s)
    rng = np.random.default_rng(5)
    for rep in range(4):
        # New positions inside each row's pages; same buffers.
        cap = (c.indptr[1:] - c.indptr[:-1]) * 16
        c.pos = np.minimum(rng.integers(0, 1200, c.rows), cap - 1).astype(np.int32)
        d.pos.copy_(dev_i32(c.pos))
        d.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_close(host_bits(d.out), oracle_out(oracle, c), what=f"replay {rep}")


def _device_values(c, seed):
    """Full-size values drawn on the device, copied back for the oracle."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    qkv = torch.randn(c.rows, (c.hq + 2 * c.hk) * 128, device="cuda", generator=gen).to(torch.bfloat16)
    kv = torch.randn(c.num_pages * c.page, 2 * c.hk * 128, device="cuda", generator=gen).to(torch.bfloat16)
    c.qkv, c.kv = host_bits(qkv), host_bits(kv)
    return qkv, kv


@pytest.mark.parametrize("cfg", [2, 3])
def test_full_config_parity(oracle, cfg):
    c = W.config_case(cfg, values=None)
    qkv, kv = _device_values(c, cfg)
    d = DevPaged.__new__(DevPaged)
    d.c, d.qkv, d.kv = c, qkv, kv
    d.pos, d.seq, d.indptr, d.pages = dev_i32(c.pos), dev_i32(c.seq), dev_i32(c.indptr), dev_i32(c.pages)
    d.out = torch.zeros(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    max_len = W.CONFIGS[cfg]["len_hi"]
    got = d.decode(max_len=max_len, lm=cfg == 3)
    want = oracle_out(oracle, c, threads=16)
    assert_close(got, want, what=f"config{cfg}")


@pytest.mark.parametrize("chunk", [0, 128])
def test_reads_no_slot_past_the_keys(oracle, chunk):
    """Every slot no row reads holds NaN (the rest of each last page and the
    pool's slack): clamped tail keys must not bring them into P.V."""
    from gpu_util import seen_slots

    c = W.paged_decode_case(9, 16, 8, 1, 300, seed=31, slack_pages=4)
    seen = seen_slots(c)
    assert (~seen).any()
    c.kv = c.kv.copy()
    c.kv[~seen] = 0x7FC0  # bf16 NaN
    assert_close(DevPaged(c).decode(chunk=chunk), oracle_out(oracle, c), what=f"NaN past the keys chunk={chunk}")


@pytest.mark.parametrize("chunk", [0, 1024])
def test_long_contexts(oracle, chunk):
    """Rows of 20k-64k keys: many splits per row (the plan's chunk, or 1024),
    far past the configs' 3000-key bound."""
    c = W.paged_decode_case(3, 8, 2, 20000, 65536, seed=15)  # 8q/2kv: a 1 KiB slot keeps the pool small
    assert_close(DevPaged(c).decode(chunk=chunk), oracle_out(oracle, c), what=f"long contexts chunk {chunk}")


@pytest.mark.parametrize("splits", [3, 5, 6, 7])
def test_every_split_written_once(oracle, splits):
    """Split counts that are not powers of two (the rotated slot -> split map
    has a period of 8 units there): the workspace starts as NaN, so a split
    the kernel skipped or a partial left from an earlier call would show up
    in the output. Rows of every length up to the plan's bound, MHA and GQA."""
    for hq, hk in ((8, 8), (16, 8)):
        max_len = 128 * splits
        c = W.paged_decode_case(37, hq, hk, 1, max_len, seed=100 + splits, slack_pages=2)
        d = DevPaged(c)
        plan = oa.decode_plan(c.rows, hq, hk, 16, max_len, 128)
        assert plan.splits == splits
        ws = oa.workspace_for(plan)
        ws.view(torch.float32).fill_(float("nan"))
        oa.qwen3_attend(d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, 16, d.out, hq, hk, c.scale, plan, ws)
        torch.cuda.synchronize()
        assert_close(host_bits(d.out), oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, 16, hq,
                                                           hk, c.scale, nthreads=16),
                     what=f"{hq}/{hk} splits {splits}")


@pytest.mark.parametrize("gh", [0, 1, 2, 4])
@pytest.mark.parametrize("page", [1, 3, 12, 16])
def test_mha_heads_per_workgroup(oracle, gh, page):
    """MHA over bf16 slots with one head per workgroup (decode_split<1>) or 2
    and 4 adjacent heads (decode_split_mh<H>, whose load instructions read
    4 / H keys x H heads), with and without the ring cap, over pages smaller
    and larger than a load's key group, powers of two and not."""
    for lm in (True, False):
        c = W.paged_decode_case(7, 8, 8, 1, 900, page=page, seed=gh * 31 + page, context=600 if lm else 0,
                                slack_pages=2)
        d = DevPaged(c)
        plan = oa.decode_plan(c.rows, 8, 8, page, int(c.lens().max()), 128)
        plan.group_heads = gh
        ws = oa.workspace_for(plan)
        args = (d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, page, d.out)
        if lm:
            oa.lm_attend(*args, 8, c.scale, c.context, plan, ws)
        else:
            oa.qwen3_attend(*args, 8, 8, c.scale, plan, ws)
        torch.cuda.synchronize()
        assert_close(host_bits(d.out), oracle_out(oracle, c), what=f"mha gh {gh} page {page} lm {lm}")


def test_mha_head_groups_agree_with_one_head_kernel(oracle):
    """The headline's shape class (MHA, 32 heads, 96 rows of up to 3000 keys,
    ring 3000, 1024-key splits): the 2-head kernel the plan picks there and the
    one-head kernel give the same rows to the tolerance, and both meet the
    oracle."""
    c = W.paged_decode_case(96, 32, 32, 100, 3000, seed=33, context=3000)
    d = DevPaged(c)
    outs = []
    for gh in (0, 1):
        plan = oa.decode_plan(c.rows, 32, 32, 16, 3000, 1024)
        plan.group_heads = gh
        d.out.zero_()
        oa.lm_attend(d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, 16, d.out, 32, c.scale, 3000, plan,
                     oa.workspace_for(plan))
        torch.cuda.synchronize()
        outs.append(host_bits(d.out))
    assert_close(outs[0], outs[1], what="2-head vs 1-head kernel")
    assert_close(outs[0], oracle_out(oracle, c, threads=16), what="2-head kernel vs oracle")


@pytest.mark.parametrize("hq,hk,gh", [(16, 8, 2), (16, 8, 4), (32, 8, 2), (8, 4, 2)])
@pytest.mark.parametrize("page", [16, 12])
def test_gqa_head_groups(oracle, hq, hk, gh, page):
    """GQA rows through the head-group kernel a plan's group_heads selects
    (two or four K/V heads per workgroup, each with its G query heads)."""
    c = W.paged_decode_case(9, hq, hk, 1, 1300, page=page, seed=hq + hk + gh + page, slack_pages=2)
    d = DevPaged(c)
    plan = oa.decode_plan(c.rows, hq, hk, page, int(c.lens().max()), 256)
    plan.group_heads = gh
    oa.qwen3_attend(d.qkv, d.kv, d.pos, d.seq, 0, d.indptr, d.pages, page, d.out, hq, hk, c.scale, plan,
                    oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(host_bits(d.out), oracle_out(oracle, c), what=f"gqa {hq}/{hk} gh {gh} page {page}")


@pytest.mark.parametrize("gh", [2, 4])
def test_head_groups_ragged_and_last_page_lengths(oracle, gh):
    """The head-group kernel on ragged prefill rows (qwen3_attend, ragged = 1)
    and with per-sequence last-page lengths (decode_run_lastlen) in place of
    positions."""
    p = W.ragged_prefill_case(3, 8, 8, 1, 200, 0, 300, seed=50 + gh, slack_pages=2)
    plan = oa.decode_plan(p.rows, 8, 8, 16, int(p.pos.max()) + 1, 128)
    plan.group_heads = gh
    out = torch.zeros(p.rows, 8 * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend(dev_bits(p.qkv), dev_bits(p.kv), dev_i32(p.pos), dev_i32(p.seq), 1, dev_i32(p.indptr),
                    dev_i32(p.pages), 16, out, 8, 8, p.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(host_bits(out), oracle_out(oracle, p, threads=16), what=f"ragged rows gh {gh}")

    c = W.paged_decode_case(8, 8, 8, 1, 500, seed=60 + gh)
    d = DevPaged(c)
    want = d.decode(chunk=128, group_heads=gh)
    last = ((c.pos % 16) + 1).astype(np.int32)
    plan = oa.decode_plan(c.rows, 8, 8, 16, int(c.lens().max()), 128)
    plan.group_heads = gh
    d.out.zero_()
    oa.decode_lastlen(d.qkv, d.kv, dev_i32(last), d.seq, 0, d.indptr, d.pages, 16, d.out, 8, 8, c.scale, plan,
                      oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(d.out), want)
    assert_close(want, oracle_out(oracle, c), what=f"gh {gh} vs oracle")


def test_calls_on_two_streams_overlap_safely(oracle):
    """Calls are reentrant per stream: two decode problems (one MHA over the
    head-group kernel, one GQA) issued alternately on two streams, each with
    its own workspace, equal their serial results bit for bit."""
    a = W.paged_decode_case(40, 8, 8, 100, 2000, seed=201)
    b = W.paged_decode_case(24, 16, 8, 100, 2000, seed=202)
    da, db = DevPaged(a), DevPaged(b)
    want_a = da.decode(chunk=256, group_heads=2)
    want_b = db.decode(chunk=256)
    pa = oa.decode_plan(a.rows, 8, 8, 16, int(a.lens().max()), 256)
    pa.group_heads = 2
    pb = oa.decode_plan(b.rows, 16, 8, 16, int(b.lens().max()), 256)
    wa, wb = oa.workspace_for(pa), oa.workspace_for(pb)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    da.out.zero_(), db.out.zero_()
    torch.cuda.synchronize()
    for _ in range(3):
        oa.qwen3_attend(da.qkv, da.kv, da.pos, da.seq, 0, da.indptr, da.pages, 16, da.out, 8, 8, a.scale, pa, wa, sa)
        oa.qwen3_attend(db.qkv, db.kv, db.pos, db.seq, 0, db.indptr, db.pages, 16, db.out, 16, 8, b.scale, pb, wb, sb)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(da.out), want_a)
    assert np.array_equal(host_bits(db.out), want_b)
