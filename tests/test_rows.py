"""The native host row builder (the engines' Rows::push_seq / Rows::push) on
the CPU: arrays against the closed forms, the ring rule, lease coverage
errors, and agreement with the workload generator's tables."""
import numpy as np
import pytest

import omni_attn as oa
import workloads as W


def test_push_seq_matches_the_closed_form():
    rng = np.random.default_rng(1)
    r = oa.Rows(page=16)
    leases, firsts, counts = [], [], []
    for s in range(5):
        n = int(rng.integers(1, 9))
        leases.append(rng.permutation(1000)[:n].astype(np.int32))
        firsts.append(int(rng.integers(0, n * 16 - 4)))
        counts.append(int(rng.integers(0, n * 16 - firsts[-1] + 1)))
        r.push(leases[-1], firsts[-1], counts[-1], s)
    assert r.counts() == (sum(counts), 5, sum(len(x) for x in leases))
    assert np.array_equal(r.indptr, np.concatenate([[0], np.cumsum([len(x) for x in leases])]))
    assert np.array_equal(r.pages, np.concatenate(leases))
    assert np.array_equal(r.seq, np.concatenate([np.full(c, s) for s, c in enumerate(counts)]))
    pos = np.concatenate([np.arange(f, f + c) for f, c in zip(firsts, counts)])
    assert np.array_equal(r.pos, pos)
    slot = np.concatenate([lease[np.arange(f, f + c) // 16] * 16 + np.arange(f, f + c) % 16
                           for lease, f, c in zip(leases, firsts, counts)])
    assert np.array_equal(r.slot, slot)


@pytest.mark.parametrize("page", [1, 3, 12, 24, 48])
def test_any_page_size_follows_the_slot_rule(page):
    """pages[t / page] * page + t % page for page sizes that are not powers of
    two as well (the reference's slot rule divides)."""
    r = oa.Rows(page=page, ring=0)
    lease = np.array([9, 2, 14, 5, 0], np.int32)
    count = 5 * page - 1
    r.push(lease, 1, count, 0)
    q = np.arange(1, 1 + count)
    assert np.array_equal(r.slot, lease[q // page] * page + q % page)


def test_ring_slots_wrap_at_the_context():
    r = oa.Rows(page=16, ring=40)
    lease = np.array([7, 3, 11], np.int32)  # 48 slots cover a 40-position ring
    r.push(lease, 35, 10, 0)
    q = np.arange(35, 45) % 40
    assert np.array_equal(r.pos, np.arange(35, 45))
    assert np.array_equal(r.slot, lease[q // 16] * 16 + q % 16)


def test_lease_coverage_and_arguments_are_checked():
    r = oa.Rows(page=16)
    with pytest.raises(oa.OmniAttnError) as e:
        r.push(np.array([1, 2], np.int32), 30, 3, 0)  # position 32 needs a third page
    assert e.value.code == oa.ETABLE
    with pytest.raises(oa.OmniAttnError) as e:
        r.push(np.array([1, -2], np.int32), 0, 3, 0)
    assert e.value.code == oa.ETABLE
    with pytest.raises(oa.OmniAttnError):
        oa.Rows(page=0)
    assert r.counts() == (0, 0, 0)  # failed pushes leave nothing behind
    r.push(np.array([4], np.int32), 0, 16, 0)
    r.clear()
    assert r.counts() == (0, 0, 0)


def test_builder_reproduces_the_workload_tables():
    """Decode rows (one per sequence at pos) and ragged prefill rows built from
    each sequence's pages give the generators' arrays, and pass check_table."""
    c = W.paged_decode_case(9, 16, 8, 1, 700, seed=4, values=None, slack_pages=3)
    r = oa.Rows(page=16)
    for s in range(c.rows):
        r.push(c.pages[c.indptr[s]:c.indptr[s + 1]], int(c.pos[s]), 1, s)
    assert np.array_equal(r.pos, c.pos) and np.array_equal(r.seq, c.seq)
    assert np.array_equal(r.indptr, c.indptr) and np.array_equal(r.pages, c.pages)
    oa.check_table(r.indptr, r.pages, c.num_pages, r.pos, r.seq, ragged=False, page=16)
    p = W.ragged_prefill_case(4, 32, 8, 3, 90, 0, 40, seed=5, values=None)
    r2 = oa.Rows(page=16)
    for s in range(4):
        first, n = int(p.extra["cached"][s]), int(p.extra["new"][s])
        r2.push(p.pages[p.indptr[s]:p.indptr[s + 1]], first, n, s)
    assert np.array_equal(r2.pos, p.pos) and np.array_equal(r2.seq, p.seq)
    assert np.array_equal(r2.indptr, p.indptr) and np.array_equal(r2.pages, p.pages)


def test_hidream_rows_follow_the_prompt_layout():
    """HiDream-O1's prefill rows (model.rs:123-160, prompt.rs:71-80): text row
    k at (k, k, k) in slot k; the timestep slot at text position `causal`;
    patch (i, j) at (4096, 4096 + i, 4096 + j) in raster order; generation
    slots after the text slots; the step sees causal + rows keys."""
    tp, ts, gp, gs, kv = oa.hidream_rows(3, (2, 3))
    assert tp.tolist() == [[0, 0, 0], [1, 1, 1], [2, 2, 2]] and ts.tolist() == [0, 1, 2]
    assert gp.tolist() == [[3, 3, 3],
                           [4096, 4096, 4096], [4096, 4096, 4097], [4096, 4096, 4098],
                           [4096, 4097, 4096], [4096, 4097, 4097], [4096, 4097, 4098]]
    assert gs.tolist() == [3, 4, 5, 6, 7, 8, 9] and kv == 10
    # a 64 x 64 grid at another image origin
    tp, ts, gp, gs, kv = oa.hidream_rows(200, (64, 64), image_position=10000)
    assert kv == 200 + 1 + 4096 and gs[0] == 200 and gs[-1] == kv - 1
    i, j = np.divmod(np.arange(4096), 64)
    assert np.array_equal(gp[1:], np.stack([np.full(4096, 10000), 10000 + i, 10000 + j], 1))


def test_hidream_rows_validate():
    L = oa.load()
    assert L.omni_hidream_rows(0, 2, 2, 4096, None, None, None, None, None) == oa.EINVAL
    assert L.omni_hidream_rows(3, 0, 2, 4096, None, None, None, None, None) == oa.EINVAL
    assert L.omni_hidream_rows(3, 2, 2, -1, None, None, None, None, None) == oa.EINVAL
    assert L.omni_hidream_rows(3, 2, 2, 4096, None, None, None, None, None) == oa.OK
