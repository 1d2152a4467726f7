"""Properties the attention math fixes, checked on the HIP path itself (no
oracle in the loop): softmax attention is invariant to the order of its keys,
grouped-query heads equal their K/V heads replicated into MHA, and a row whose
keys are all identical outputs the mean of its V rows. Each property pairs two
runs of the kernels (or one run and a closed form) on the same seeded inputs.
The tolerance between two kernel runs is the one the path is held to against
the reference math (max-abs 2e-2, mean-abs 2e-3); the closed form is held to
the bf16 rounding of its result."""
import dataclasses

import numpy as np
import pytest
import torch

import workloads as W
from gpu_util import DevPaged, assert_close, bits_f32, dev_bits, dev_i32, host_bits

pytestmark = pytest.mark.gpu


def _slots_of_row(c, n, length):
    s = int(c.seq[n]) if c.ragged else n
    pg = c.pages[c.indptr[s]:c.indptr[s + 1]]
    t = np.arange(length)
    return pg[t // c.page] * c.page + t % c.page


@pytest.mark.parametrize("hq,hk", [(16, 8), (32, 8), (8, 2)])
def test_decode_gqa_equals_replicated_mha(hq, hk):
    """qwen3_attend with G = hq / hk query heads per K/V head against the MHA
    call (hk' = hq) whose K/V head h' is K/V head h' / G: the G > 1 and G = 1
    kernels agree."""
    c = W.paged_decode_case(6, hq, hk, 1, 1500, seed=hq * 7 + hk)
    g = hq // hk
    rows, slots = c.qkv.shape[0], c.kv.shape[0]
    qkv = np.zeros((rows, 3 * hq * 128), np.uint16)
    qkv[:, :hq * 128] = c.qkv[:, :hq * 128]
    kv3 = c.kv.reshape(slots, 2, hk, 128)
    kv_mha = np.repeat(kv3, g, axis=2).reshape(slots, 2 * hq * 128)
    m = dataclasses.replace(c, hk=hq, qkv=qkv, kv=kv_mha)
    assert_close(DevPaged(m).decode(chunk=128), DevPaged(c).decode(chunk=128), what=f"G={g} vs MHA")


@pytest.mark.parametrize("lm", [False, True])
def test_decode_key_order_invariance(lm):
    """Permuting the K/V contents of each row's keys 0..len-1 (within its own
    slots) leaves the output unchanged up to summation order."""
    c = W.paged_decode_case(7, 16, 16 if lm else 8, 2, 1300, seed=41, context=900 if lm else 0)
    a = DevPaged(c).decode(chunk=256, max_len=900 if lm else None, lm=lm)
    lens = c.lens()
    kv2 = c.kv.copy()
    rng = np.random.default_rng(3)
    for n in range(c.rows):
        sl = _slots_of_row(c, n, int(lens[n]))
        kv2[sl] = c.kv[sl[rng.permutation(len(sl))]]
    b = DevPaged(dataclasses.replace(c, kv=kv2)).decode(chunk=256, max_len=900 if lm else None, lm=lm)
    assert_close(b, a, what=f"key order lm={lm}")


@pytest.mark.parametrize("hq,hk", [(16, 8), (16, 16)])
def test_decode_identical_keys_give_mean_of_v(hq, hk):
    """Every key of a row equal: all scores are equal, so P is uniform and the
    output is the mean of the row's V rows (split and unsplit)."""
    c = W.paged_decode_case(5, hq, hk, 1, 2100, seed=5 + hq + hk)
    kv = c.kv.reshape(c.kv.shape[0], 2, hk, 128).copy()
    kv[:, 0] = kv[0, 0]  # one K row per head, in every slot
    c = dataclasses.replace(c, kv=kv.reshape(c.kv.shape[0], -1))
    lens = c.lens()
    g = hq // hk
    want = np.zeros((c.rows, hq, 128))
    v = bits_f32(kv[:, 1]).astype(np.float64)  # [slots][hk][128]
    for n in range(c.rows):
        mean = v[_slots_of_row(c, n, int(lens[n]))].mean(axis=0)  # [hk][128]
        want[n] = np.repeat(mean, g, axis=0)
    for chunk in (0, 128):
        got = bits_f32(DevPaged(c).decode(chunk=chunk)).astype(np.float64).reshape(c.rows, hq, 128)
        # bf16 keeps 8 significant bits: a correctly rounded mean is within 2^-8 relative.
        err = np.abs(got - want) - (2.0 ** -8) * np.abs(want) - 1e-6
        assert err.max() <= 0, f"chunk {chunk}: {err.max():.3g} past bf16 rounding"


@pytest.mark.parametrize("hq,hk", [(32, 8), (16, 16)])
def test_dit_key_permutation_invariance(hq, hk):
    """hidream_attend (non-causal) with its K and V rows permuted together."""
    from test_tiled_gpu import run_dense

    c = W.dense_case(hq, hk, 300, 700, 0, seed=hq + 5 * hk)
    perm = np.random.default_rng(9).permutation(700)
    p = dataclasses.replace(c, k=np.ascontiguousarray(c.k[:, perm]), v=np.ascontiguousarray(c.v[:, perm]))
    assert_close(run_dense(p), run_dense(c), what=f"DiT {hq}/{hk} key permutation")


@pytest.mark.parametrize("causal", [0, 1])
def test_dit_gqa_equals_replicated_mha(causal):
    """hidream_attend with 4 query heads per K/V head (tiled_attn<4>) against
    the MHA call on replicated K/V heads (tiled_attn<1>)."""
    from test_tiled_gpu import run_dense

    c = W.dense_case(32, 8, 260, 260, causal, seed=17 + causal)
    q = c.q.reshape(1, 260, 48, 128)[:, :, :32].reshape(1, 260, 32 * 128)
    k = np.repeat(c.k.reshape(1, 260, 8, 128), 4, axis=2).reshape(1, 260, 32 * 128)
    v = np.repeat(c.v.reshape(1, 260, 8, 128), 4, axis=2).reshape(1, 260, 32 * 128)
    m = dataclasses.replace(c, hk=32, q_stride=32 * 128, q=np.ascontiguousarray(q), k=k, v=v)
    assert_close(run_dense(m), run_dense(c), what=f"DiT GQA vs MHA causal={causal}")


def test_prefill_rows_independent_of_batch_order():
    """The MFMA prefill on two sequences, then on the same two with their row
    blocks swapped in the row list: each row's output is the same (its tile
    composition is unchanged, so bit-identical)."""
    import omni_attn as oa

    c = W.ragged_prefill_case(2, 32, 8, 300, 700, 0, 200, seed=23)
    rows = c.rows
    s0 = np.nonzero(c.seq == 0)[0]
    s1 = np.nonzero(c.seq == 1)[0]
    order = np.concatenate([s1, s0])

    def run(idx):
        qkv = dev_bits(np.ascontiguousarray(c.qkv[idx]))
        pos, seq = c.pos[idx].astype(np.int32), c.seq[idx].astype(np.int32)
        pf = oa.prefill_plan(rows, c.hq, c.hk, c.page, seq, pos)
        out = torch.zeros(rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
        oa.prefill_run(pf, qkv, dev_bits(c.kv), dev_i32(pos), dev_i32(seq), dev_i32(c.indptr), dev_i32(c.pages), out,
                       c.scale)
        torch.cuda.synchronize()
        return host_bits(out)

    a = run(np.arange(rows))
    b = run(order)
    back = np.empty_like(b)
    back[order] = b
    assert np.array_equal(back, a)
