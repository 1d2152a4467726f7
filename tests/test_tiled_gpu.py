"""MFMA prefill (ragged causal over the paged cache) and HiDream DiT
attention on the GPU against the CPU oracle."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits
from refs import bits_to_f64

pytestmark = pytest.mark.gpu


def run_prefill(c, exact_p=False):
    pf = oa.prefill_plan(c.rows, c.hq, c.hk, c.page, c.seq, c.pos, exact_p=exact_p)
    out = torch.zeros(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.prefill_run(pf, dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), dev_i32(c.indptr),
                   dev_i32(c.pages), out, c.scale)
    torch.cuda.synchronize()
    return host_bits(out)


def oracle_paged(oracle, c, threads=16):
    return oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                               nthreads=threads)


@pytest.mark.parametrize("hq,hk", [(32, 8), (16, 16), (16, 8), (64, 8)])
def test_prefill_parity(oracle, hq, hk):
    c = W.ragged_prefill_case(3, hq, hk, 1, 300, 0, 200, seed=hq + hk)
    assert_close(run_prefill(c), oracle_paged(oracle, c), what=f"prefill {hq}/{hk}")


@pytest.mark.parametrize("page", [3, 12, 24, 48, 80])
def test_prefill_any_page(oracle, page):
    """Pages that are not powers of two: 48 and 80 (multiples of a wave's 16
    tile rows) take the one-page-id-per-wave loader with a multiply-high
    division, 3, 12 and 24 the per-key loader."""
    c = W.ragged_prefill_case(3, 32, 8, 1, 300, 0, 200, page=page, seed=page, slack_pages=3)
    assert_close(run_prefill(c), oracle_paged(oracle, c), what=f"prefill page {page}")


def test_prefill_single_rows_and_odd_lengths(oracle):
    c = W.ragged_prefill_case(6, 32, 8, 1, 3, 0, 70, seed=3)
    assert_close(run_prefill(c), oracle_paged(oracle, c), what="short")


def test_prefill_matches_decode_kernel(oracle):
    """The same rows through the split-K decode kernel: two kernels, one answer."""
    c = W.ragged_prefill_case(4, 32, 8, 50, 200, 0, 300, seed=4)
    a = run_prefill(c)
    plan = oa.decode_plan(c.rows, 32, 8, 16, int(c.pos.max()) + 1, 128)
    out = torch.zeros(c.rows, 32 * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend(dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 1, dev_i32(c.indptr),
                    dev_i32(c.pages), 16, out, 32, 8, c.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(a, host_bits(out), what="prefill vs decode")


def test_prefill_config4_subset(oracle):
    """Config 4's construction (new U[512,4096], cached U[0,1024]) on 2 requests."""
    c = W.ragged_prefill_case(2, 32, 8, 512, 4096, 0, 1024, seed=4000)
    assert_close(run_prefill(c), oracle_paged(oracle, c), what="config4 subset")


def test_prefill_config4_own_draw(oracle):
    """Config 4's own seeded draw (B = 8, seed 4000: 25,499 rows, up to 4,563
    keys), the workload bench.py times, so its work-list order (longest tiles
    first, XCD ranges, the 8 sequences' items) is the one checked: every row
    against the oracle (about 895 GFLOP, 10-20 s on 16 host threads), and
    every row against the split-K decode kernel (the reference's f32 P)."""
    c = W.config_case(4)
    assert c.rows == 25499 and len(c.extra["new"]) == 8
    got = run_prefill(c)
    want = oracle_paged(oracle, c)
    mx, mn = assert_close(got, want, what=f"config4 all {c.rows} rows vs oracle")
    print(f"config4 vs oracle: max-abs {mx:.3g} mean-abs {mn:.3g}")
    plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, int(c.pos.max()) + 1)
    out = torch.zeros(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend(dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 1, dev_i32(c.indptr),
                    dev_i32(c.pages), c.page, out, c.hq, c.hk, c.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(got, host_bits(out), what="config4 prefill vs decode, every row")
    # The plan's exact_p (P as bf16 hi + lo, the reference's f32-P numerics):
    # every row against the oracle and, nearly bit for bit, the decode kernel.
    ex = run_prefill(c, exact_p=True)
    mx, mn = assert_close(ex, want, what=f"config4 exact_p all {c.rows} rows vs oracle")
    print(f"config4 exact_p vs oracle: max-abs {mx:.3g} mean-abs {mn:.3g}")
    same = float(np.mean(ex == host_bits(out)))
    assert same >= 0.99, f"exact_p prefill and the f32-P decode kernel agree on {same:.4f} of elements"


def run_dense(c, b_all=True):
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(c.batch, c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([c.kv_len], np.int32))
    if c.batch == 1:
        oa.hidream_attend(q, k, v, out, c.q_len, kvl, c.q_stride, c.causal, c.scale_log2, c.hq, c.hk)
    else:
        oa.hidream_attend_batched(q, k, v, out, c.q_len, kvl, c.q_stride, c.causal, c.scale_log2, c.hq, c.hk, c.batch,
                                  c.q_len * c.q_stride, c.kv_len * c.hk * 128, c.q_len * c.hq * 128)
    torch.cuda.synchronize()
    return host_bits(out)


def oracle_dense(oracle, c, b=0, kv_len=None):
    return oracle.dense_attend(np.ascontiguousarray(c.q[b]), np.ascontiguousarray(c.k[b]),
                               np.ascontiguousarray(c.v[b]), c.q_len, kv_len or c.kv_len, c.q_stride, c.hq, c.hk,
                               c.causal, c.scale_log2, nthreads=16)


# On a 256-CU GPU the workspace-free call runs the last round's items as row
# halves when they fill at most half of it: every case below but the
# 1100-query one (144 items, all whole) runs as halves only. (16, 8, 65) and
# (4, 4, 1) have second halves with one and no rows.
@pytest.mark.parametrize("hq,hk,q_len,kv_len,causal", [
    (32, 8, 300, 300, 1), (32, 8, 257, 333, 0), (8, 8, 100, 130, 0), (4, 4, 1, 1, 0), (16, 8, 65, 64, 1),
    (32, 4, 40, 500, 0), (32, 8, 1100, 300, 1),
])
def test_dit_parity(oracle, hq, hk, q_len, kv_len, causal):
    c = W.dense_case(hq, hk, q_len, kv_len, causal, seed=q_len)
    assert_close(run_dense(c)[0], oracle_dense(oracle, c), what=f"dit {hq}/{hk} {q_len}x{kv_len} c{causal}")


def test_dit_kv_len_read_from_device(oracle):
    c = W.dense_case(32, 8, 200, 400, 0, seed=7)
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([259], np.int32))
    oa.hidream_attend(q, k, v, out, c.q_len, kvl, c.q_stride, 0, c.scale_log2, c.hq, c.hk)
    torch.cuda.synchronize()
    assert_close(host_bits(out), oracle_dense(oracle, c, kv_len=259), what="kv_len 259")


def test_dit_batched_pair(oracle):
    c = W.dense_case(32, 8, 130, 130, 0, batch=2, seed=8)
    got = run_dense(c)
    for b in range(2):
        assert_close(got[b], oracle_dense(oracle, c, b), what=f"batch {b}")


def test_dit_config5_subset(oracle):
    """Config 5's shape (4352 keys, 32q/8kv, RMS-normed q/k) on the first 256 queries."""
    c = W.dense_case(32, 8, 4352, 4352, 0, seed=5000)
    got = run_dense(c)[0]
    sub = W.DenseCase(hq=32, hk=8, q_len=256, kv_len=4352, causal=0, q_stride=c.q_stride, q=c.q, k=c.k, v=c.v)
    want = oracle_dense(oracle, sub)
    assert_close(got[:256], want, what="config5 first 256 rows")


def run_dense_ws(c, kv_len=None):
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(c.batch, c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([kv_len or c.kv_len], np.int32))
    ws = oa.hidream_workspace()
    ws.fill_(0xFF)  # stale partials must not matter
    oa.hidream_attend_ws(q, k, v, out, c.q_len, kvl, c.q_stride, c.causal, c.scale_log2, c.hq, c.hk, c.batch,
                         c.q_len * c.q_stride, c.kv_len * c.hk * 128, c.q_len * c.hq * 128, ws)
    torch.cuda.synchronize()
    return host_bits(out)


@pytest.mark.parametrize("hq,hk,q_len,kv_len,causal,batch", [
    # (with 256-row tiles, 128-key tiles and 256 resident workgroups on MI355X)
    (8, 2, 256, 256, 0, 1),     # 8 items, each split into 32 chunks of a 2-tile key range (most chunks empty)
    (32, 8, 300, 700, 1, 2),    # causal: chunk ranges differ per tile
    (32, 8, 1000, 1000, 0, 1),  # 128 items: each split in two
    (4, 4, 1, 1, 0, 1),
])
def test_dit_tail_split_parity(oracle, hq, hk, q_len, kv_len, causal, batch):
    c = W.dense_case(hq, hk, q_len, kv_len, causal, batch=batch, seed=q_len + kv_len)
    got = run_dense_ws(c)
    for b in range(batch):
        assert_close(got[b], oracle_dense(oracle, c, b), what=f"ws dit {hq}/{hk} {q_len}x{kv_len} c{causal} b{b}")


@pytest.mark.parametrize("hk,seed", [(8, 5000), (32, 5032)])
def test_dit_config5_full_size(oracle, hk, seed):
    """Config 5 at its full size, the CFG pair of 4352 queries and keys, 32
    q heads over hk = 8 (the reference's shape) and hk = 32 (the MHA variant
    bench.py also times). On a 256-CU GPU its 1088 items run as 1024 whole
    and 64 split into 4 key chunks with a workspace (the kernels bench.py
    times), and as row halves without one. Every row of both batch halves
    meets the oracle in both forms (2 x 310 GFLOP, about 10 s on 16 host
    threads), and the two forms agree on every row."""
    c = W.dense_case(32, hk, 4352, 4352, 0, batch=2, seed=seed)
    got, ref = run_dense_ws(c), run_dense(c)
    for b in range(2):
        want = oracle_dense(oracle, c, b)
        mx, mn = assert_close(got[b], want, what=f"config5 hk {hk} batch {b} (workspace) vs oracle")
        print(f"config5 hk {hk} batch {b} vs oracle: max-abs {mx:.3g} mean-abs {mn:.3g}")
        assert_close(ref[b], want, what=f"config5 hk {hk} batch {b} (no workspace) vs oracle")
        assert_close(got[b], ref[b], what=f"config5 hk {hk} batch {b}: workspace vs row halves")


@pytest.mark.parametrize("causal", [0, 1])
def test_dit_row_halves_match_split(oracle, causal):
    """544 items: on a 256-CU GPU the last 32 (kv head 7, queries 2304..)
    run as row halves without a workspace and as 8 key chunks with one. Both
    agree with each other everywhere and with the oracle on the last 128
    queries (whole tiles for heads 0..27, halves for 28..31)."""
    c = W.dense_case(32, 8, 4352, 1024, causal, seed=31 + causal)
    got, split = run_dense(c)[0], run_dense_ws(c)[0]
    assert_close(got, split, what="halves vs split")
    # Queries 4224.. see all 1024 keys, causal or not.
    want = oracle.dense_attend(np.ascontiguousarray(c.q[0, -128:]), np.ascontiguousarray(c.k[0]),
                               np.ascontiguousarray(c.v[0]), 128, 1024, c.q_stride, 32, 8, 0, c.scale_log2,
                               nthreads=16)
    assert_close(got[-128:], want, what=f"halves tail vs oracle c{causal}")


@pytest.mark.parametrize("causal", [0, 1])
def test_dit_no_key_gives_nan(oracle, causal):
    """*kv_len_at = 0 (hidream.cu:337-346: l = 0, so O * (1 / l) = NaN): every
    output element is NaN through the plain call, the batched call (row halves
    for the last round) and the workspace call (key chunks, all empty), as the
    oracle gives; a second call with keys overwrites them with finite values."""
    c = W.dense_case(32, 8, 300, 300, causal, batch=2, seed=41 + causal)
    want = oracle.dense_attend(np.ascontiguousarray(c.q[0]), np.ascontiguousarray(c.k[0]), np.ascontiguousarray(c.v[0]),
                               c.q_len, 0, c.q_stride, c.hq, c.hk, causal, c.scale_log2, nthreads=16)
    assert np.isnan(bits_to_f64(want)).all()
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    zero = dev_i32(np.array([0], np.int32))
    bs = (c.q_len * c.q_stride, c.kv_len * c.hk * 128, c.q_len * c.hq * 128)
    outs = [torch.zeros(c.batch, c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    oa.hidream_attend(q, k, v, outs[0], c.q_len, zero, c.q_stride, causal, c.scale_log2, c.hq, c.hk)
    oa.hidream_attend_batched(q, k, v, outs[1], c.q_len, zero, c.q_stride, causal, c.scale_log2, c.hq, c.hk, 2, *bs)
    oa.hidream_attend_ws(q, k, v, outs[2], c.q_len, zero, c.q_stride, causal, c.scale_log2, c.hq, c.hk, 2, *bs,
                         oa.hidream_workspace())
    torch.cuda.synchronize()
    assert np.isnan(bits_to_f64(host_bits(outs[0][0]))).all(), "plain call"
    assert np.isnan(bits_to_f64(host_bits(outs[1]))).all(), "batched call"
    assert np.isnan(bits_to_f64(host_bits(outs[2]))).all(), "workspace call"
    # The same buffers with keys again: finite and equal to the oracle.
    oa.hidream_attend_ws(q, k, v, outs[2], c.q_len, dev_i32(np.array([c.kv_len], np.int32)), c.q_stride, causal,
                         c.scale_log2, c.hq, c.hk, 2, *bs, oa.hidream_workspace())
    torch.cuda.synchronize()
    assert_close(host_bits(outs[2])[1], oracle_dense(oracle, c, 1), what="keys again")


def test_dit_empty_query_launch_is_a_no_op():
    """q_len = 0 (and batch = 0) returns OK and writes nothing."""
    c = W.dense_case(32, 8, 4, 4, 0, seed=43)
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.full((4, c.hq * 128), 3.0, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([4], np.int32))
    oa.hidream_attend(q, k, v, out, 0, kvl, c.q_stride, 0, c.scale_log2, c.hq, c.hk)
    oa.hidream_attend_ws(q, k, v, out, 0, kvl, c.q_stride, 0, c.scale_log2, c.hq, c.hk, 1, 0, 0, 0,
                         oa.hidream_workspace())
    oa.hidream_attend_batched(q, k, v, out, 4, kvl, c.q_stride, 0, c.scale_log2, c.hq, c.hk, 0, 0, 0, 0)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())


@pytest.mark.parametrize("page", [1, 2, 4, 8, 64])
def test_prefill_page_sizes(oracle, page):
    """The paged tile loader at pages below a wave's 16 rows of a tile (one
    page id per key row) and from 16 up (one scalar page id per wave and tile)."""
    c = W.ragged_prefill_case(3, 32, 8, 40, 260, 0, 150, page=page, seed=page)
    assert_close(run_prefill(c), oracle_paged(oracle, c), what=f"prefill page {page}")


BF16_NAN = 0x7FC0


def test_prefill_reads_no_slot_past_its_keys(oracle):
    """Every cache slot no row may see holds NaN, including the rest of each
    sequence's last page: the tail tile must not read them into P.V."""
    c = W.ragged_prefill_case(4, 32, 8, 30, 300, 0, 150, seed=21)
    seen = np.zeros(c.kv.shape[0], bool)
    for s in range(len(c.indptr) - 1):
        rows = c.seq == s
        if not rows.any():
            continue
        keys = np.arange(int(c.pos[rows].max()) + 1)
        pg = c.pages[c.indptr[s]:c.indptr[s + 1]]
        seen[pg[keys // c.page] * c.page + keys % c.page] = True
    assert (~seen).any() and any((int(c.pos[c.seq == s].max()) + 1) % 64 for s in np.unique(c.seq))
    c.kv = c.kv.copy()
    c.kv[~seen] = BF16_NAN
    assert_close(run_prefill(c), oracle_paged(oracle, c), what="prefill with NaN past the keys")


@pytest.mark.parametrize("causal", [0, 1])
def test_dit_reads_no_key_past_kv_len(oracle, causal):
    """K and V rows past *kv_len_at hold NaN; the partial last key tile must
    not read them into P.V."""
    c = W.dense_case(32, 8, 200, 400, causal, seed=22)
    c.k, c.v = c.k.copy(), c.v.copy()
    c.k[:, 259:] = BF16_NAN
    c.v[:, 259:] = BF16_NAN
    q, k, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([259], np.int32))
    oa.hidream_attend(q, k, v, out, c.q_len, kvl, c.q_stride, causal, c.scale_log2, c.hq, c.hk)
    torch.cuda.synchronize()
    assert_close(host_bits(out), oracle_dense(oracle, c, kv_len=259), what=f"kv_len 259 with NaN past it, c{causal}")


@pytest.mark.parametrize("layout", ["gaps", "interleaved"])
def test_prefill_runs_split_at_gaps_and_interleaving(oracle, layout):
    """Rows whose positions jump inside a sequence, or whose sequences
    alternate row by row: the plan cuts them into separate runs (single rows
    when interleaved), and each row still sees keys 0..pos of its sequence."""
    base = W.ragged_prefill_case(3, 32, 8, 150, 300, 20, 200, seed=77)
    rng = np.random.default_rng(78)
    if layout == "gaps":
        keep = np.sort(rng.choice(base.rows, size=base.rows * 2 // 3, replace=False))  # drop a third of the rows
    else:
        per_seq = [np.flatnonzero(base.seq == s) for s in range(3)]
        n = min(len(x) for x in per_seq)
        keep = np.stack([x[:n] for x in per_seq], axis=1).reshape(-1)  # seq 0, 1, 2, 0, 1, 2, ...
    c = W.PagedCase(hq=32, hk=8, page=base.page, pos=base.pos[keep], seq=base.seq[keep], ragged=1,
                    indptr=base.indptr, pages=base.pages, num_pages=base.num_pages, qkv=base.qkv[keep], kv=base.kv)
    pf = oa.prefill_plan(c.rows, 32, 8, c.page, c.seq, c.pos)
    assert pf.plan.tiles > (c.rows + 63) // 64  # really cut into more, shorter runs
    assert_close(run_prefill(c), oracle_paged(oracle, c), what=f"prefill {layout}")


def test_prefill_long_sequence(oracle):
    """One sequence of 6000 new rows over 3000 cached keys: 94 tiles per kv
    head. The oracle checks the first and last 96 rows (rows are independent)."""
    c = W.ragged_prefill_case(1, 32, 8, 6000, 6000, 3000, 3000, seed=79)
    got = run_prefill(c)
    pick = np.r_[0:96, c.rows - 96:c.rows]
    sub = W.PagedCase(hq=32, hk=8, page=c.page, pos=c.pos[pick], seq=c.seq[pick], ragged=1, indptr=c.indptr,
                      pages=c.pages, num_pages=c.num_pages, qkv=c.qkv[pick], kv=c.kv)
    assert_close(got[pick], oracle_paged(oracle, sub), what="long prefill, first and last rows")


@pytest.mark.parametrize("hq,hk,page", [(32, 8, 16), (16, 16, 16), (16, 8, 12), (64, 8, 16), (8, 4, 3)])
def test_prefill_exact_p_parity(oracle, hq, hk, page):
    """The plan's exact_p (P carried as two bf16 terms through P.V) on every
    query-head group, paged through powers of two and not, against the oracle."""
    c = W.ragged_prefill_case(3, hq, hk, 1, 300, 0, 200, page=page, seed=hq + hk + page)
    assert_close(run_prefill(c, exact_p=True), oracle_paged(oracle, c), what=f"prefill exact_p {hq}/{hk} page {page}")


@pytest.mark.parametrize("seed", [29, 31])
def test_prefill_exact_p_is_the_f32_p_kernel(seed):
    """With exact_p the MFMA prefill keeps P to 16 significant bits (hi + lo
    bf16), the precision qwen3_attend(ragged = 1)'s f32 P reaches in its
    bf16 output: it agrees bit for bit with the split-K decode kernel (f32 P)
    on >= 99% of elements, differs by at most one bf16 ulp (or 2^-15 near zero)
    elsewhere, and its
    error against f64 SDPA is the decode kernel's (mean within 5%), below the
    bf16-P prefill's."""
    from refs import paged_truth
    from gpu_util import bits_f32

    c = W.ragged_prefill_case(2, 32, 8, 300, 700, 0, 200, seed=seed)
    ex, pre = run_prefill(c, exact_p=True), run_prefill(c)
    plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, int(c.pos.max()) + 1)
    out = torch.zeros(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend(dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 1, dev_i32(c.indptr),
                    dev_i32(c.pages), c.page, out, c.hq, c.hk, c.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    dec = host_bits(out)
    assert np.mean(ex == dec) >= 0.99
    fe, fd = bits_f32(ex).astype(np.float64), bits_f32(dec).astype(np.float64)
    from refs import bf16_ulp
    # Beyond the rounding step the two f32 results differ by summation order
    # and P's 17th bit, a few 2^-24 of sum p |v| / l (< 1): 2^-15 absolute
    # covers outputs near zero, where one ulp is smaller than that.
    assert np.all(np.abs(fe - fd) <= bf16_ulp(np.maximum(np.abs(fe), np.abs(fd))) + 2.0 ** -15)
    truth = paged_truth(c).reshape(c.rows, -1)
    e_ex, e_dec = np.abs(fe - truth), np.abs(fd - truth)
    e_pre = np.abs(bits_f32(pre).astype(np.float64) - truth)
    assert e_ex.mean() <= 1.05 * e_dec.mean(), (e_ex.mean(), e_dec.mean())
    assert e_ex.mean() < e_pre.mean(), (e_ex.mean(), e_pre.mean())


def test_prefill_error_against_f64_truth_is_near_the_f32_p_kernels():
    """The MFMA prefill rounds P to bf16 (an MFMA operand) where
    qwen3_attend(ragged = 1) keeps it in f32 (qwen3.cu:123-208). Against f64
    SDPA its error stays within 2.5x the mean and 2x the max of the split-K
    decode kernel (f32 P) on the same rows."""
    from refs import paged_truth
    from gpu_util import bits_f32

    c = W.ragged_prefill_case(2, 32, 8, 300, 700, 0, 200, seed=29)
    pre = run_prefill(c)
    plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, int(c.pos.max()) + 1)
    out = torch.zeros(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend(dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), 1, dev_i32(c.indptr),
                    dev_i32(c.pages), c.page, out, c.hq, c.hk, c.scale, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    truth = paged_truth(c).reshape(c.rows, -1)
    e_pre = np.abs(bits_f32(pre).astype(np.float64) - truth)
    e_dec = np.abs(bits_f32(host_bits(out)).astype(np.float64) - truth)
    assert e_pre.mean() <= 2.5 * e_dec.mean(), (e_pre.mean(), e_dec.mean())
    assert e_pre.max() <= 2.0 * e_dec.max(), (e_pre.max(), e_dec.max())
    assert e_pre.max() < 2e-2 / 4 and e_pre.mean() < 2e-3 / 4
