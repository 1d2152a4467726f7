"""The C ABI without a GPU: the library loads, exports every entry point the
header declares, and its host-side planning and validation behave as
documented (no kernel launches here)."""
import ctypes
import os
import re

import numpy as np
import pytest

import omni_attn as oa
import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "omni_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(omni_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_what_python_binds():
    assert set(declared_functions()) == set(oa.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = oa.load()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert L.omni_attn_version() >= 100


def test_decode_plan_shapes():
    p = oa.decode_plan(128, 32, 32, 16, 3000)
    assert p.splits == (3000 + p.chunk - 1) // p.chunk and p.chunk % 128 == 0
    assert p.workspace_bytes == 128 * 32 * p.splits * 129 * 4
    p1 = oa.decode_plan(4, 16, 8, 16, 100)
    assert p1.splits == 1 and p1.workspace_bytes == 0
    p2 = oa.decode_plan(4, 16, 8, 16, 1000, chunk=256)
    assert p2.chunk == 256 and p2.splits == 4


@pytest.mark.parametrize("rows,chunk", [(32, 256), (64, 384), (128, 768), (256, 1024), (1, 256)])
def test_decode_plan_fp8_picks_the_fp8_split(rows, chunk):
    """The FP8 plan's split size: the largest of 1024/768/512/384 keys giving
    >= 2048 workgroups of 8 heads at full length (rows x heads / 8 x splits),
    else 256; everything else as decode_plan with hq = hk = heads."""
    p = oa.decode_plan_fp8(rows, 32, 16, 3000)
    assert p.chunk == chunk
    splits = -(-3000 // chunk)
    assert (p.rows, p.hq, p.hk, p.page, p.max_len, p.splits) == (rows, 32, 32, 16, 3000, splits)
    wgs = [rows * 4 * -(-3000 // c) for c in (1024, 768, 512, 384)]
    assert chunk == next((c for c, w in zip((1024, 768, 512, 384), wgs) if w >= 2048), 256)
    assert p.workspace_bytes == (rows * 32 * splits * 129 * 4 if splits > 1 else 0)
    q = oa.decode_plan(rows, 32, 32, 16, 3000, chunk=chunk)
    assert bytes(p) == bytes(q)  # the same plan as the bf16 init at that chunk
    assert oa.decode_plan_fp8(rows, 32, 16, 3000, chunk=512).chunk == 512  # a hint is kept


@pytest.mark.parametrize("args,code", [
    ((4, 0, 16, 100, 0), oa.EINVAL),        # heads
    ((4, 8, 0, 100, 0), oa.EINVAL),         # page
    ((4, 8, 16, 0, 0), oa.EINVAL),          # max_len
    ((4, 8, 16, 100, 96), oa.EINVAL),       # chunk not a multiple of 128
])
def test_decode_plan_fp8_rejects(args, code):
    with pytest.raises(oa.OmniAttnError) as e:
        oa.decode_plan_fp8(*args)
    assert e.value.code == code


@pytest.mark.parametrize("args,code", [
    ((4, 16, 6, 16, 100, 0), oa.EINVAL),        # hq not a multiple of hk
    ((4, 16, 2, 16, 100, 0), oa.EUNSUPPORTED),  # G = 8 not implemented in decode
    ((4, 16, 8, 0, 100, 0), oa.EINVAL),         # page not positive
    ((4, 16, 8, -16, 100, 0), oa.EINVAL),       # page not positive
    ((4, 16, 8, 16, 0, 0), oa.EINVAL),          # max_len
    ((4, 16, 8, 16, 100, 100), oa.EINVAL),      # chunk not a multiple of 128
    ((70000, 16, 8, 16, 100, 0), oa.EINVAL),    # rows beyond grid limit
])
def test_decode_plan_rejects(args, code):
    with pytest.raises(oa.OmniAttnError) as e:
        oa.decode_plan(*args)
    assert e.value.code == code


def test_run_without_workspace_fails_before_launch():
    p = oa.decode_plan(4, 16, 8, 16, 1000, chunk=128)
    fake = ctypes.c_void_p(16)
    rc = oa.load().omni_qwen3_attend(fake, fake, fake, None, 0, fake, fake, 16, fake, 16, 8, 0.1, ctypes.byref(p),
                                     None, None)
    assert rc == oa.EWORKSPACE
    rc = oa.load().omni_qwen3_attend(fake, fake, fake, None, 0, fake, fake, 16, fake, 16, 4, 0.1, ctypes.byref(p),
                                     None, None)
    assert rc == oa.EINVAL  # plan/argument mismatch
    rc = oa.load().omni_qwen3_attend(None, fake, fake, None, 0, fake, fake, 16, fake, 16, 8, 0.1, ctypes.byref(p),
                                     fake, None)
    assert rc == oa.EINVAL


@pytest.mark.parametrize("gh,hq,hk", [(3, 8, 8), (8, 8, 8), (-1, 8, 8), (4, 16, 4), (2, 4, 1), (4, 8, 2)])
def test_bf16_group_heads_validated_before_launch(gh, hq, hk):
    """bf16 slots take 1, 2 or 4 K/V heads per workgroup dividing hk (1 or 2
    when four q heads share a K/V head)."""
    p = oa.decode_plan(4, hq, hk, 16, 1000, chunk=128)
    p.group_heads = gh
    fake = ctypes.c_void_p(16)
    rc = oa.load().omni_qwen3_attend(fake, fake, fake, None, 0, fake, fake, 16, fake, hq, hk, 0.1, ctypes.byref(p),
                                     fake, None)
    assert rc == oa.EINVAL
    assert "group_heads" in oa.load().omni_attn_last_error().decode()


@pytest.mark.parametrize("gh", [3, 16, -2, 6])
def test_fp8_group_heads_validated_before_launch(gh):
    p = oa.decode_plan(4, 8, 8, 16, 1000, chunk=128)
    p.group_heads = gh
    fake = ctypes.c_void_p(16)
    rc = oa.load().omni_lm_attend_fp8(fake, fake, fake, None, 0, fake, fake, 16, fake, 8, 0.1, 1000, ctypes.byref(p),
                                      fake, None)
    assert rc == oa.EINVAL
    assert "group_heads" in oa.load().omni_attn_last_error().decode()


def test_check_table_accepts_generated_cases():
    c = W.paged_decode_case(9, 8, 4, 1, 500, seed=1)
    oa.check_table(c.indptr, c.pages, c.num_pages, c.pos, None, False, 16)
    r = W.ragged_prefill_case(3, 8, 2, 5, 60, 0, 40, seed=2)
    oa.check_table(r.indptr, r.pages, r.num_pages, r.pos, r.seq, True, 16)


def test_check_table_rejects_bad_tables():
    c = W.paged_decode_case(4, 8, 4, 20, 100, seed=3)
    bad = c.indptr.copy()
    bad[2] = bad[3] + 1
    with pytest.raises(oa.OmniAttnError) as e:
        oa.check_table(bad, c.pages, c.num_pages, c.pos, None, False, 16)
    assert e.value.code == oa.ETABLE
    pages = c.pages.copy()
    pages[1] = c.num_pages
    with pytest.raises(oa.OmniAttnError):
        oa.check_table(c.indptr, pages, c.num_pages, c.pos, None, False, 16)
    pos = c.pos.copy()
    pos[0] = (c.indptr[1] - c.indptr[0]) * 16  # one token past its pages
    with pytest.raises(oa.OmniAttnError):
        oa.check_table(c.indptr, c.pages, c.num_pages, pos, None, False, 16)
    # ...unless the ring cap keeps it inside.
    oa.check_table(c.indptr, c.pages, c.num_pages, pos, None, False, 16, context=int(c.pos[0]) + 1)


HEADER = 16  # work-list header: entries 0..8 bound the item ranges of the 8 XCDs


def _plan_host(rows, hq, hk, seq, pos):
    L = oa.load()
    plan = oa.PrefillPlan()
    seq = np.ascontiguousarray(seq, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    rc = L.omni_attn_prefill_plan_init(rows, hq, hk, 16, seq.ctypes.data_as(ctypes.c_void_p),
                                       pos.ctypes.data_as(ctypes.c_void_p), None, 0, ctypes.byref(plan))
    assert rc == oa.EWORKSPACE
    work = np.zeros(plan.work_bytes // 4, np.int32)
    rc = L.omni_attn_prefill_plan_init(rows, hq, hk, 16, seq.ctypes.data_as(ctypes.c_void_p),
                                       pos.ctypes.data_as(ctypes.c_void_p), work.ctypes.data_as(ctypes.c_void_p),
                                       len(work), ctypes.byref(plan))
    assert rc == oa.OK
    return plan, work[:HEADER], work[HEADER:].reshape(-1, 4)


def _tiles(pos, items):
    """Distinct tiles (seq, first, rows, keys of the last row) in first-seen order."""
    out = []
    for s, first, n, _ in items:
        t = (int(s), int(first), int(n), int(pos[first + n - 1]) + 1)
        if t not in out:
            out.append(t)
    return out


def test_prefill_plan_items_cover_every_row_and_head_once():
    r = W.ragged_prefill_case(5, 32, 8, 1, 300, 0, 100, seed=4)
    plan, hdr, items = _plan_host(r.rows, 32, 8, r.seq, r.pos)
    per_tile = plan.tile_rows // 4
    covered = np.zeros((r.rows, 8), int)
    for s, first, n, h in items:
        assert 1 <= n <= per_tile and 0 <= h < 8
        assert np.all(r.seq[first:first + n] == s)
        assert np.all(np.diff(r.pos[first:first + n]) == 1)
        covered[first:first + n, h] += 1
    assert np.all(covered == 1)
    assert plan.tiles * 8 == len(items)
    # XCD ranges: increasing, covering every item, and the grid spans the widest.
    assert hdr[0] == 0 and hdr[8] == len(items) and np.all(np.diff(hdr[:9]) >= 0) and np.all(hdr[9:] == 0)
    assert plan.workgroups == 8 * int(np.diff(hdr[:9]).max())


def _dispatch_order(hdr, items):
    """Items in the order workgroups are numbered: workgroup i runs item
    hdr[i % 8] + i // 8 (XCD i % 8); holes where an XCD's range is exhausted."""
    out = []
    for i in range(8 * int(np.diff(hdr[:9]).max())):
        x, j = i % 8, i // 8
        if hdr[x] + j < hdr[x + 1]:
            out.append(items[hdr[x] + j])
    return np.array(out)


@pytest.mark.parametrize("hk", [1, 2, 4, 8, 16])
def test_prefill_plan_runs_longest_first_and_pins_kv_heads(hk):
    r = W.ragged_prefill_case(6, 4 * hk, hk, 40, 400, 0, 200, seed=5)
    plan, hdr, items = _plan_host(r.rows, 4 * hk, hk, r.seq, r.pos)
    keys = lambda it: np.array([r.pos[f + n - 1] + 1 for _, f, n, _ in it])
    # In workgroup order: tiles by keys, most first, each with its hk kv heads in order.
    order = _dispatch_order(hdr, items)
    assert len(order) == len(items)
    assert np.all(np.diff(keys(order)) <= 0)
    tiles = order.reshape(-1, hk, 4)
    assert np.all(tiles[:, :, 3] == np.arange(hk)) and np.all(tiles[:, :, :3] == tiles[:, :1, :3])
    # Every XCD runs longest first and always sees the same kv heads.
    for x in range(8):
        mine = items[hdr[x]:hdr[x + 1]]
        assert np.all(np.diff(keys(mine)) <= 0)
        assert set(int(h) % 8 for h in mine[:, 3]) <= {x % hk if hk <= 8 else x}
    # The XCD ranges differ by at most one item.
    sizes = np.diff(hdr[:9])
    assert sizes.max() - sizes.min() <= 1 and plan.workgroups == 8 * int(sizes.max())


def test_prefill_plan_breaks_runs_at_position_gaps():
    seq = np.array([0, 0, 0, 1, 1, 0, 0], np.int32)
    pos = np.array([5, 6, 8, 0, 1, 9, 10], np.int32)
    plan, hdr, items = _plan_host(7, 4, 4, seq, pos)
    assert plan.tiles == 4
    # tiles by keys, most first: both runs of sequence 0, then sequence 1
    order = _dispatch_order(hdr, items)
    assert _tiles(pos, order) == [(0, 5, 2, 11), (0, 2, 1, 9), (0, 0, 2, 7), (1, 3, 2, 2)]
    assert [tuple(w) for w in order[:5]] == [(0, 5, 2, 0), (0, 5, 2, 1), (0, 5, 2, 2), (0, 5, 2, 3), (0, 2, 1, 0)]
    # XCD 0 takes items 0 and 8: kv head 0 of the first and third tiles
    assert [tuple(w) for w in items[hdr[0]:hdr[1]]] == [(0, 5, 2, 0), (0, 0, 2, 0)]


def test_rope_entry_points_validate_before_launch():
    L = oa.load()
    f = ctypes.c_void_p(4096)  # aligned fake device pointer: every call below fails before any launch
    bad = ctypes.c_void_p(4098)
    assert L.omni_qwen3_rope(f, f, f, f, f, f, 0, 16, 8, 1e-6, 1e6, None) == oa.OK  # no rows: nothing to do
    assert L.omni_qwen3_rope(bad, f, f, f, f, f, 4, 16, 8, 1e-6, 1e6, None) == oa.EINVAL
    assert L.omni_qwen3_rope(f, f, f, None, f, f, 4, 16, 8, 1e-6, 1e6, None) == oa.EINVAL
    assert L.omni_qwen3_rope(f, f, f, f, f, f, 4, 16, 8, 1e-6, -1.0, None) == oa.EINVAL
    assert L.omni_qwen3_rope(f, f, f, f, f, f, 4, 0, 8, 1e-6, 1e6, None) == oa.EINVAL
    assert L.omni_qwen3_rope_dense(f, f, f, f, 10, 5, 3, 7, 16, 8, 1e-6, 1e6, None) == oa.EINVAL  # base+per > span
    assert L.omni_qwen3_rope_dense(f, f, f, f, 10, 0, 3, 70, 16, 8, 1e-6, 1e6, None) == oa.EINVAL
    assert L.omni_lm_rope(f, f, f, ctypes.c_void_p(4100), 4, 32, -0.14, None) == oa.EINVAL  # kv not 8-aligned
    assert L.omni_lm_rope(f, f, f, f, 4, 32, float("nan"), None) == oa.EINVAL
    assert L.omni_hidream_qk_rope(f, 128, f, f, f, f, f, f, 4, 4, 2, 20, 1e-6, 1e6, None) == oa.EINVAL  # ld too short
    assert L.omni_hidream_qk_rope(f, 1024, f, f, f, f, f, f, 4, 4, 2, 22, 1e-6, 1e6, None) == oa.EINVAL
    assert "mrope_hw" in L.omni_attn_last_error().decode()


def test_short_entry_points_validate_before_launch():
    L = oa.load()
    f = ctypes.c_void_p(4096)
    p = oa.decode_plan(4, 16, 8, 1, 20)
    assert L.omni_qwen3_attend_dense(f, f, 5, 7, 10, f, 16, 8, 0.1, ctypes.byref(p), f, None) == oa.EINVAL
    small = oa.decode_plan(4, 16, 8, 1, 8)
    assert L.omni_qwen3_attend_dense(f, f, 5, 7, 16, f, 16, 8, 0.1, ctypes.byref(small), f, None) == oa.EINVAL
    assert L.omni_mimi_attend(f, f, f, f, f, 4, 0, 8, 0.125, 250, 1024, None) == oa.EINVAL
    assert L.omni_mimi_attend(f, f, f, f, f, 4, 2, 8, 0.125, 250, 1000, None) == oa.EINVAL  # stride not 16-aligned
    assert L.omni_codec_attention(f, f, f, f, f, 4, 1024, 8, -1.0, None) == oa.EINVAL
    assert L.omni_lm_dep_kv_attend(f, f, 8, f, 4, 16, 0.125, None) == oa.EINVAL
    assert L.omni_lm_dep_kv_attend(f, f, 0, f, 0, 16, 0.125, None) == oa.OK


def test_decode_rejects_a_plan_edited_after_init():
    """The kernels size their grid and split partials from the plan: a plan
    whose fields no longer agree (more splits than its chunk gives, a chunk
    off the 128-key grid, a workspace smaller than its splits need, rows past
    the grid limit) is refused before any launch."""
    L = oa.load()
    fake = ctypes.c_void_p(4096)

    def run(p):
        return L.omni_qwen3_attend(fake, fake, fake, None, 0, fake, fake, 16, fake, 16, 8, 0.1, ctypes.byref(p), fake,
                                   None)

    for field, value in [("splits", 9), ("chunk", 100), ("chunk", 0), ("workspace_bytes", 1024), ("rows", 70000),
                         ("max_len", 0)]:
        p = oa.decode_plan(4, 16, 8, 16, 1000, chunk=128)
        setattr(p, field, value)
        assert run(p) == oa.EINVAL, field
        assert "self-consistent" in L.omni_attn_last_error().decode()


def test_entry_points_reject_misaligned_rows():
    """Rows move in 16-byte pieces: q / qkv, k, v, kv, out at 16-byte
    alignment (FP8 slots at 8), and DiT batch strides in multiples of 8
    elements. All refused before any launch."""
    L = oa.load()
    f, odd, eight = ctypes.c_void_p(4096), ctypes.c_void_p(4098), ctypes.c_void_p(4104)
    p = oa.decode_plan(4, 16, 8, 16, 1000, chunk=128)
    assert L.omni_qwen3_attend(odd, f, f, None, 0, f, f, 16, f, 16, 8, 0.1, ctypes.byref(p), f, None) == oa.EINVAL
    assert L.omni_qwen3_attend(f, eight, f, None, 0, f, f, 16, f, 16, 8, 0.1, ctypes.byref(p), f, None) == oa.EINVAL
    assert L.omni_qwen3_attend(f, f, f, None, 0, f, f, 16, odd, 16, 8, 0.1, ctypes.byref(p), f, None) == oa.EINVAL
    p8 = oa.decode_plan(4, 8, 8, 16, 1000, chunk=128)
    assert L.omni_lm_attend_fp8(f, odd, f, None, 0, f, f, 16, f, 8, 0.1, 1000, ctypes.byref(p8), f, None) == oa.EINVAL
    kvl = ctypes.c_void_p(4096)
    for q, k, v, out in [(odd, f, f, f), (f, odd, f, f), (f, f, eight, f), (f, f, f, odd)]:
        assert L.omni_hidream_attend(q, k, v, out, 10, kvl, 6144, 0, 0.1, 32, 8, None) == oa.EINVAL
    assert L.omni_hidream_attend_batched(f, f, f, f, 10, kvl, 6144, 0, 0.1, 32, 8, 2, 61444, 0, 0, None) == oa.EINVAL
    assert L.omni_hidream_attend_batched(f, f, f, f, 10, kvl, 6144, 0, 0.1, 32, 8, 2, 0, -8, 0, None) == oa.EINVAL
    assert "batch strides" in L.omni_attn_last_error().decode()


def test_prefill_rejects_bad_rows_and_plans():
    L = oa.load()
    plan = oa.PrefillPlan()
    for seq, pos in [([0, -1], [0, 0]), ([0, 0], [2**31 - 2, 2**31 - 1])]:
        s = np.array(seq, np.int32)
        q = np.array(pos, np.int32)
        rc = L.omni_attn_prefill_plan_init(2, 32, 8, 16, s.ctypes.data_as(ctypes.c_void_p),
                                           q.ctypes.data_as(ctypes.c_void_p), None, 0, ctypes.byref(plan))
        assert rc == oa.ETABLE, (seq, pos)
    f, odd = ctypes.c_void_p(4096), ctypes.c_void_p(4098)
    good, _, _ = _plan_host(4, 32, 8, np.zeros(4, np.int32), np.arange(4, dtype=np.int32))
    bad = oa.PrefillPlan.from_buffer_copy(good)
    bad.hk = 0
    assert L.omni_attn_prefill_run(ctypes.byref(bad), f, f, f, f, f, f, f, 0.1, f, None) == oa.EINVAL
    # Fields that disagree with each other: the grid, the item count and the
    # tile shape come from the plan, so any edit is refused before a launch
    # (too few workgroups would skip items silently).
    for field, value in [("page", 0), ("workgroups", 0), ("workgroups", good.workgroups - 8),
                         ("workgroups", good.workgroups + 8), ("tiles", good.tiles + 1), ("tile_rows", 128),
                         ("hq", 8 * 16), ("hq", 8 * 3), ("work_bytes", good.work_bytes - 4),
                         ("exact_p", 2), ("exact_p", -1)]:
        bad = oa.PrefillPlan.from_buffer_copy(good)
        setattr(bad, field, value)
        assert L.omni_attn_prefill_run(ctypes.byref(bad), f, f, f, f, f, f, f, 0.1, f, None) == oa.EINVAL, field
    assert L.omni_attn_prefill_run(ctypes.byref(good), odd, f, f, f, f, f, f, 0.1, f, None) == oa.EINVAL
    assert good.exact_p == 0  # plan_init's default: P rounded to bf16


def test_rows_push_keeps_positions_and_slots_in_int32():
    r = oa.Rows(page=16)
    with pytest.raises(oa.OmniAttnError) as e:
        r.push(np.arange(8), 2**31 - 4, 8, 0)  # positions past int32
    assert e.value.code == oa.EINVAL
    with pytest.raises(oa.OmniAttnError) as e:
        r.push([2**31 // 16], 0, 4, 0)  # the page's slots pass int32
    assert e.value.code == oa.ETABLE
    r.push([2**31 // 16 - 1], 0, 16, 0)  # the last page that fits
    assert int(r.slot[-1]) == 2**31 - 1


def test_python_wrappers_refuse_a_short_workspace():
    """The C run takes no workspace size, so the binding checks it against
    the plan before the call (a shorter buffer would be written past)."""
    torch = pytest.importorskip("torch")
    p = oa.decode_plan(4, 16, 8, 16, 1000, chunk=128)
    with pytest.raises(oa.OmniAttnError) as e:
        oa._ws(p, torch.empty(int(p.workspace_bytes) - 16, dtype=torch.uint8))
    assert e.value.code == oa.EWORKSPACE and "the plan needs" in str(e.value)


def test_empty_batches_return_before_any_launch():
    """A bucket with no rows (decode, prefill) is a no-op that returns OK on any
    host, GPU or not: nothing is launched."""
    L = oa.load()
    f = ctypes.c_void_p(4096)
    p = oa.decode_plan(0, 16, 8, 16, 1000)
    assert p.rows == 0
    assert L.omni_qwen3_attend(f, f, f, None, 0, f, f, 16, f, 16, 8, 0.1, ctypes.byref(p), f, None) == oa.OK
    p8 = oa.decode_plan(0, 8, 8, 16, 1000)
    assert L.omni_lm_attend_fp8(f, f, f, None, 0, f, f, 16, f, 8, 0.1, 1000, ctypes.byref(p8), f, None) == oa.OK
    plan = oa.PrefillPlan()
    rc = L.omni_attn_prefill_plan_init(0, 32, 8, 16, None, None, None, 0, ctypes.byref(plan))
    assert rc == oa.EWORKSPACE and plan.work_bytes == 16 * 4  # the header alone
    work = np.zeros(16, np.int32)
    rc = L.omni_attn_prefill_plan_init(0, 32, 8, 16, None, None, work.ctypes.data_as(ctypes.c_void_p), 16,
                                       ctypes.byref(plan))
    assert rc == oa.OK and plan.tiles == 0
    assert L.omni_attn_prefill_run(ctypes.byref(plan), f, f, f, f, f, f, f, 0.1, f, None) == oa.OK


def test_mimi_rope_kv_and_copy_kv_validate_before_launch():
    """The two cache writers refuse bad shapes on any host, GPU or not."""
    L = oa.load()
    f, odd = ctypes.c_void_p(4096), ctypes.c_void_p(4100)
    coef = -0.28
    assert L.omni_mimi_rope_kv(f, f, f, f, 0, 2, 8, coef, 250, 64000, None) == oa.OK  # no rows: nothing to do
    assert L.omni_mimi_rope_kv(f, f, f, f, 4, 0, 8, coef, 250, 64000, None) == oa.EINVAL  # T
    assert L.omni_mimi_rope_kv(f, f, f, f, 4, 2, 8, coef, 0, 64000, None) == oa.EINVAL  # context
    assert L.omni_mimi_rope_kv(f, f, f, f, 4, 2, 8, coef, 250, 64008, None) == oa.EINVAL  # stride % 16
    assert L.omni_mimi_rope_kv(odd, f, f, f, 4, 2, 8, coef, 250, 64000, None) == oa.EINVAL  # alignment
    assert L.omni_mimi_rope_kv(f, f, f, f, 4, 2, 0, coef, 250, 64000, None) == oa.EINVAL  # heads
    assert L.omni_mimi_rope_kv(f, f, f, f, 4, 2, 8, float("nan"), 250, 64000, None) == oa.EINVAL
    assert L.omni_lm_copy_kv(None, None, None, 0, 8448, None) == oa.OK
    assert L.omni_lm_copy_kv(f, f, f, 3, 8440, None) == oa.EINVAL  # not a multiple of 16
    assert L.omni_lm_copy_kv(f, f, f, -1, 8448, None) == oa.EINVAL
    assert L.omni_lm_copy_kv(odd, f, f, 3, 8448, None) == oa.EINVAL
    assert L.omni_lm_copy_kv(f, None, f, 3, 8448, None) == oa.EINVAL
