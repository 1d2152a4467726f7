"""Pins the CPU oracle (oracle/omni_attn_oracle.c) before it is trusted as the
checker of the HIP kernels.

The reference ships no attention-level golden vector (its golden tests need
checkpoints and recorded PyTorch runs), so each oracle function is pinned by:
  * an independent f64 library computation (torch SDPA in float64) on small
    inputs, to within one bf16 ulp — a dropped key, wrong head index or wrong
    page lookup moves outputs by far more;
  * special cases with closed forms (one key -> its V row exactly; equal
    scores -> the mean of V; one dominant key -> its V row exactly);
  * invariances the reference kernels have (physical page permutation,
    GQA == MHA with replicated K/V heads, ring cap == truncated positions).
"""
import numpy as np
import pytest
import torch

import workloads as W
from refs import bf16_ulp, bits_to_f64, dense_truth, dense_weight_abs, paged_truth


def within_ulp(got_bits, want, ulps=1.0, floor=1e-6):
    got = bits_to_f64(got_bits).reshape(want.shape)
    err = np.abs(got - want)
    bound = ulps * bf16_ulp(want) + floor
    return bool(np.all(err <= bound)), float((err / bound).max())


# ------------------------------------------------------------------- bf16 rule
def test_bf16_rounding_matches_torch(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-5, 5, 10000),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 65504.0, 3.0e38, 1e-40], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(x), want)
    assert np.array_equal(W.f32_to_bf16_bits(x), want)
    assert np.array_equal(oracle.bf16_to_f32(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_normal_generator_statistics(oracle):
    v = oracle.bf16_to_f32(oracle.normal_bf16(200000, 7))
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert np.array_equal(oracle.normal_bf16(1001, 7)[:1000], oracle.normal_bf16(1000, 7))


# ------------------------------------------------------------------ page table
def test_slot_closed_form(oracle):
    case = W.paged_decode_case(5, 4, 2, 1, 100, page=16, seed=3)
    for s in range(case.rows):
        for t in (0, 1, 15, 16, 17, int(case.pos[s])):
            if t > case.pos[s]:
                continue
            want = int(case.pages[case.indptr[s] + t // 16]) * 16 + t % 16
            assert oracle.slot(case.indptr, case.pages, s, t, 16) == want


@pytest.mark.parametrize("page", [1, 16, 64])
def test_gather_is_fancy_indexing(oracle, page):
    case = W.paged_decode_case(6, 4, 2, 1, 300, page=page, seed=4)
    for s in range(case.rows):
        ln = int(case.pos[s]) + 1
        t = np.arange(ln)
        slots = case.pages[case.indptr[s] + t // page].astype(np.int64) * page + t % page
        assert np.array_equal(oracle.gather_kv(case.kv, case.hk, case.indptr, case.pages, page, s, ln), case.kv[slots])


# ------------------------------------------------------------ paged attention
@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 4), (16, 4), (16, 8)])
def test_paged_matches_f64_sdpa(oracle, hq, hk):
    case = W.paged_decode_case(6, hq, hk, 1, 300, seed=hq * 10 + hk)
    got = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, hq, hk,
                              case.scale, nthreads=4)
    ok, worst = within_ulp(got, paged_truth(case))
    assert ok, f"worst error {worst:.2f} ulp"


def test_paged_ragged_and_context(oracle):
    case = W.ragged_prefill_case(3, 8, 2, 5, 40, 0, 50, seed=5)
    got = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 1, case.indptr, case.pages, 16, 8, 2,
                              case.scale)
    ok, worst = within_ulp(got, paged_truth(case))
    assert ok, worst
    # The PersonaPlex ring: rows past the context see exactly `context` slots.
    ring = W.paged_decode_case(5, 4, 4, 200, 400, seed=6, context=150)
    got = oracle.paged_attend(ring.qkv, ring.kv, ring.pos, ring.seq, 0, ring.indptr, ring.pages, 16, 4, 4,
                              ring.scale, context=150)
    ok, worst = within_ulp(got, paged_truth(ring))
    assert ok, worst
    trunc = oracle.paged_attend(ring.qkv, ring.kv, np.full_like(ring.pos, 149), ring.seq, 0, ring.indptr, ring.pages,
                                16, 4, 4, ring.scale)
    assert np.array_equal(got, trunc)


def test_paged_single_key_is_v_row(oracle):
    case = W.paged_decode_case(4, 8, 4, 1, 1, seed=7)
    got = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 8, 4, case.scale)
    for n in range(case.rows):
        slot = int(case.pages[case.indptr[n]]) * 16
        v = case.kv[slot].reshape(8, 128)[4:]
        assert np.array_equal(got[n].reshape(8, 128), np.repeat(v, 2, axis=0))


def test_paged_equal_scores_give_mean(oracle):
    case = W.paged_decode_case(3, 4, 2, 37, 200, seed=8)
    case.qkv[:, : 4 * 128] = 0  # q = 0: every score 0, p = 1
    got = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 4, 2, case.scale)
    want = paged_truth(case)
    ok, worst = within_ulp(got, want)
    assert ok, worst
    from refs import slots_of
    for n in range(case.rows):
        v = bits_to_f64(case.kv[slots_of(case, n, int(case.pos[n]) + 1)]).reshape(-1, 4, 128)[:, 2:]
        assert np.allclose(want[n].reshape(2, 2, 128), v.mean(0)[:, None, :].repeat(2, 1).reshape(2, 2, 128))


def test_paged_dominant_key(oracle):
    case = W.paged_decode_case(2, 2, 1, 300, 300, seed=9)
    s, t_hot = 1, 211
    from refs import slots_of
    sl = slots_of(case, s, 300)
    # k of the hot key = 64 * q (in bf16): its score beats every other by far.
    q = bits_to_f64(case.qkv[s, :128])
    case.kv[sl[t_hot], :128] = W.f32_to_bf16_bits((q * 64).astype(np.float32))
    got = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 2, 1, case.scale)
    v = case.kv[sl[t_hot], 128:256]
    assert np.array_equal(got[s, :128], v) and np.array_equal(got[s, 128:], v)


def test_paged_page_permutation_invariance(oracle):
    case = W.paged_decode_case(5, 8, 4, 10, 200, seed=10, slack_pages=7)
    a = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 8, 4, case.scale)
    perm = np.random.default_rng(11).permutation(case.num_pages).astype(np.int32)
    kv2 = np.empty_like(case.kv)
    for p in range(case.num_pages):
        kv2[perm[p] * 16:(perm[p] + 1) * 16] = case.kv[p * 16:(p + 1) * 16]
    b = oracle.paged_attend(case.qkv, kv2, case.pos, case.seq, 0, case.indptr, perm[case.pages].copy(), 16, 8, 4,
                            case.scale)
    assert np.array_equal(a, b)


def test_paged_gqa_equals_replicated_mha(oracle):
    case = W.paged_decode_case(4, 8, 2, 10, 130, seed=12)
    a = oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 8, 2, case.scale)
    kv = case.kv.reshape(-1, 4, 128)
    kv_rep = np.concatenate([np.repeat(kv[:, :2], 4, 1), np.repeat(kv[:, 2:], 4, 1)], 1).reshape(len(kv), -1)
    qkv = np.concatenate([case.qkv[:, : 8 * 128], np.zeros((case.rows, 16 * 128), np.uint16)], 1)
    b = oracle.paged_attend(np.ascontiguousarray(qkv), np.ascontiguousarray(kv_rep), case.pos, case.seq, 0,
                            case.indptr, case.pages, 16, 8, 8, case.scale)
    assert np.array_equal(a, b)


def test_paged_threads_do_not_change_results(oracle):
    case = W.paged_decode_case(8, 8, 4, 10, 400, seed=13)
    args = (case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 8, 4, case.scale)
    assert np.array_equal(oracle.paged_attend(*args, nthreads=1), oracle.paged_attend(*args, nthreads=8))


def test_paged_rejects_bad_shapes(oracle):
    case = W.paged_decode_case(2, 4, 2, 10, 20, seed=14)
    with pytest.raises(ValueError):
        oracle.paged_attend(case.qkv, case.kv, case.pos, case.seq, 0, case.indptr, case.pages, 16, 5, 2, case.scale)


# ------------------------------------------------------------ dense attention
@pytest.mark.parametrize("hq,hk,q_len,kv_len,causal", [
    (4, 1, 70, 70, 1), (4, 1, 33, 130, 0), (8, 2, 65, 64, 0), (8, 8, 20, 7, 1), (4, 4, 1, 1, 0), (8, 1, 9, 200, 1),
])
def test_dense_matches_f64_sdpa(oracle, hq, hk, q_len, kv_len, causal):
    case = W.dense_case(hq, hk, q_len, kv_len, causal, seed=q_len + kv_len)
    got = oracle.dense_attend(case.q[0], case.k[0], case.v[0], q_len, kv_len, case.q_stride, hq, hk, causal,
                              case.scale_log2, nthreads=4)
    # P is rounded to bf16 before P.V (hidream.cu:321-324): each term may move
    # by 2^-9 of its weight, so the bound is 1 ulp + 2^-8 * sum p|v| / l.
    want = dense_truth(case)
    got_f = bits_to_f64(got).reshape(want.shape)
    bound = bf16_ulp(want) + 2.0 ** -8 * dense_weight_abs(case) + 1e-6
    assert np.all(np.abs(got_f - want) <= bound), float((np.abs(got_f - want) / bound).max())


def test_dense_causal_first_row_is_v0(oracle):
    case = W.dense_case(4, 1, 16, 16, 1, seed=21)
    got = oracle.dense_attend(case.q[0], case.k[0], case.v[0], 16, 16, case.q_stride, 4, 1, 1, case.scale_log2)
    assert np.array_equal(got[0].reshape(4, 128), np.repeat(case.v[0, 0][None], 4, 0))


def test_dense_kv_len_masks_tail(oracle):
    case = W.dense_case(4, 2, 10, 100, 0, seed=22)
    a = oracle.dense_attend(case.q[0], case.k[0], case.v[0], 10, 37, case.q_stride, 4, 2, 0, case.scale_log2)
    k2, v2 = case.k[0].copy(), case.v[0].copy()
    k2[37:] = 0x7F80  # +inf bits past kv_len must never be read
    v2[37:] = 0x7FC0
    b = oracle.dense_attend(case.q[0], k2, v2, 10, 37, case.q_stride, 4, 2, 0, case.scale_log2)
    assert np.array_equal(a, b)



def test_dense_no_key_gives_nan(oracle):
    """*kv_len_at = 0: no row sees a key, so l stays 0 and the reference's
    normalisation 1 / l (hidream.cu:337-346) turns O = 0 into NaN everywhere."""
    case = W.dense_case(8, 2, 5, 40, 1, seed=23)
    for causal in (0, 1):
        got = oracle.dense_attend(case.q[0], case.k[0], case.v[0], 5, 0, case.q_stride, 8, 2, causal, case.scale_log2)
        assert np.isnan(bits_to_f64(got)).all()

# ------------------------------------------------------- FP8 (E4M3) ring attention
def test_e4m3_decode_matches_torch(oracle):
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3_to_f32(int(b)) for b in codes], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], want[~nan])


def _dequant(c, heads):
    raw = c.kv[:, : 2 * heads * 128].copy()
    vals = torch.from_numpy(raw).view(torch.float8_e4m3fn).float().numpy().reshape(len(raw), 2 * heads, 128)
    sc = c.kv[:, 2 * heads * 128:].copy().view(np.float32).reshape(len(raw), 2 * heads, 1)
    return vals.astype(np.float64) * sc


@pytest.mark.parametrize("heads,ctx", [(2, 0), (4, 150)])
def test_fp8_ring_matches_f64_sdpa(oracle, heads, ctx):
    import workloads as W2

    c = W2.fp8_ring_case(6, heads, 1, 300, ctx, seed=heads + ctx)
    got = oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, 16, heads, c.scale, ctx or 0)
    deq = _dequant(c, heads)
    from refs import slots_of
    want = np.zeros((c.rows, heads, 128))
    for n in range(c.rows):
        sl = slots_of(c, n, int(c.lens()[n]))
        k = torch.from_numpy(deq[sl, :heads].transpose(1, 0, 2).copy())
        v = torch.from_numpy(deq[sl, heads:].transpose(1, 0, 2).copy())
        q = torch.from_numpy(bits_to_f64(c.qkv[n, : heads * 128]).reshape(heads, 1, 128))
        want[n] = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=c.scale)[:, 0].numpy()
    ok, worst = within_ulp(got, want)
    assert ok, worst


def test_fp8_single_key_is_scaled_v_row(oracle):
    import workloads as W2

    c = W2.fp8_ring_case(3, 2, 1, 1, 0, seed=31)
    got = oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, 16, 2, c.scale, 0)
    for n in range(c.rows):
        slot = int(c.pages[c.indptr[n]]) * 16
        v8 = torch.from_numpy(c.kv[slot, 2 * 128: 4 * 128].copy()).view(torch.float8_e4m3fn).float().numpy()
        vs = c.kv[slot, 4 * 128:].copy().view(np.float32)[2:4]
        want = W.f32_to_bf16_bits((v8.reshape(2, 128) * vs[:, None]).astype(np.float32)).reshape(-1)
        assert np.array_equal(got[n], want)
