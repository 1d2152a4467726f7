"""Scores far from N(0, 1): every kernel against the oracle when each key's K
row is scaled up with its position, so a row's running maximum keeps growing
(the decode kernels' online rescale runs every tile, and the MFMA kernels'
lazy base, which moves only when the maximum grows by more than 2^8, moves
again and again), and when scores span hundreds of log2 units (softmax close
to one-hot on the last keys).

Near one-hot rows return a single V row, so outputs here reach |o| of 2-4,
where one bf16 ulp is 0.0156-0.031: the DiT check is therefore element by
element against float64 SDPA, to the bound the oracle itself is pinned to
(bf16 rounding of the output, one ulp, plus 2^-8 sum p|v| / l for P rounded to
bf16), with one more ulp for the kernel's own rounding; the mean stays held to
2e-3 against the oracle."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import DevPaged, assert_close, compare, dev_bits, dev_i32, host_bits
from refs import bf16_ulp, bits_to_f64, dense_truth, dense_weight_abs

pytestmark = pytest.mark.gpu


def bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def key_positions(c):
    """Logical key index of every physical slot a paged case's sequences own
    (-1 for unowned slots)."""
    t_of = np.full(c.kv.shape[0], -1, np.int64)
    for s in range(len(c.indptr) - 1):
        pg = c.pages[c.indptr[s]:c.indptr[s + 1]]
        t = np.arange(len(pg) * c.page)
        t_of[pg[t // c.page] * c.page + t % c.page] = t
    return t_of


def grow(t, rate):
    return 1.0 + np.maximum(t, 0) * rate


@pytest.mark.parametrize("hq,hk,gh,lm", [(16, 8, 0, False), (8, 8, 1, True), (8, 8, 2, True), (8, 8, 4, False)])
@pytest.mark.parametrize("rate", [0.02, 0.2])
def test_decode_growing_scores(oracle, hq, hk, gh, lm, rate):
    c = W.paged_decode_case(6, hq, hk, 300, 1500, seed=70 + hq + gh, context=1200 if lm else 0, slack_pages=2)
    kv = bits_to_f32(c.kv).reshape(c.kv.shape[0], 2 * hk, 128)
    kv[:, :hk] *= grow(key_positions(c), rate)[:, None, None].astype(np.float32)
    c.kv = W.f32_to_bf16_bits(kv).reshape(c.kv.shape)
    d = DevPaged(c)
    got = d.decode(chunk=256, lm=lm, group_heads=gh)
    want = oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, c.page, hq, hk, c.scale,
                               context=c.context, nthreads=16)
    assert_close(got, want, what=f"decode {hq}/{hk} gh {gh} lm {lm} rate {rate}")


@pytest.mark.parametrize("rate", [0.02, 0.2])
def test_fp8_growing_scores(oracle, rate):
    """FP8 slots: the growth goes into the per-(slot, head) K scales."""
    heads = 8
    c = W.fp8_ring_case(6, heads, 300, 1500, 1200, seed=80, slack_pages=2)
    body = 2 * heads * 128
    sc = c.kv[:, body:].copy().view(np.float32).reshape(-1, 2 * heads)
    sc[:, :heads] *= grow(key_positions(c), rate)[:, None].astype(np.float32)
    c.kv[:, body:] = sc.reshape(len(sc), -1).view(np.uint8)
    plan = oa.decode_plan(c.rows, heads, heads, 16, int(c.lens().max()), 256)
    out = torch.zeros(c.rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    oa.lm_attend_fp8(dev_bits(c.qkv), torch.from_numpy(np.ascontiguousarray(c.kv)).cuda(), dev_i32(c.pos),
                     dev_i32(c.seq), 0, dev_i32(c.indptr), dev_i32(c.pages), 16, out, heads, c.scale, 1200, plan,
                     oa.workspace_for(plan))
    torch.cuda.synchronize()
    want = oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, 16, heads, c.scale, 1200,
                                nthreads=16)
    assert_close(host_bits(out), want, what=f"fp8 rate {rate}")


@pytest.mark.parametrize("rate", [0.02, 0.2])
def test_prefill_growing_scores(oracle, rate):
    c = W.ragged_prefill_case(3, 32, 8, 100, 400, 0, 600, seed=90, slack_pages=2)
    kv = bits_to_f32(c.kv).reshape(c.kv.shape[0], 16, 128)
    kv[:, :8] *= grow(key_positions(c), rate)[:, None, None].astype(np.float32)
    c.kv = W.f32_to_bf16_bits(kv).reshape(c.kv.shape)
    pf = oa.prefill_plan(c.rows, 32, 8, 16, c.seq, c.pos)
    out = torch.zeros(c.rows, 32 * 128, dtype=torch.bfloat16, device="cuda")
    oa.prefill_run(pf, dev_bits(c.qkv), dev_bits(c.kv), dev_i32(c.pos), dev_i32(c.seq), dev_i32(c.indptr),
                   dev_i32(c.pages), out, c.scale)
    torch.cuda.synchronize()
    want = oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, 1, c.indptr, c.pages, 16, 32, 8, c.scale, nthreads=16)
    assert_close(host_bits(out), want, what=f"prefill rate {rate}")


@pytest.mark.parametrize("rate,causal,ws", [(0.02, 0, False), (0.2, 1, False), (0.02, 1, True), (0.2, 0, True)])
def test_dit_growing_scores(oracle, rate, causal, ws):
    c = W.dense_case(32, 8, 600, 900, causal, seed=95, rmsnorm=False)
    k = bits_to_f32(c.k).reshape(1, c.kv_len, 8, 128)
    k *= grow(np.arange(c.kv_len), rate)[None, :, None, None].astype(np.float32)
    c.k = W.f32_to_bf16_bits(k).reshape(c.k.shape)
    q, kk, v = dev_bits(c.q), dev_bits(c.k), dev_bits(c.v)
    out = torch.zeros(1, c.q_len, 32 * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([c.kv_len], np.int32))
    if ws:
        oa.hidream_attend_ws(q, kk, v, out, c.q_len, kvl, c.q_stride, causal, c.scale_log2, 32, 8, 1,
                             c.q_len * c.q_stride, c.kv_len * 8 * 128, c.q_len * 32 * 128, oa.hidream_workspace())
    else:
        oa.hidream_attend(q, kk, v, out, c.q_len, kvl, c.q_stride, causal, c.scale_log2, 32, 8)
    torch.cuda.synchronize()
    want = oracle.dense_attend(np.ascontiguousarray(c.q[0]), np.ascontiguousarray(c.k[0]),
                               np.ascontiguousarray(c.v[0]), c.q_len, c.kv_len, c.q_stride, 32, 8, causal,
                               c.scale_log2, nthreads=16)
    got = host_bits(out)[0]
    what = f"dit rate {rate} causal {causal} ws {ws}"
    assert compare(got, want)[1] <= 2e-3, what
    truth = dense_truth(c).reshape(c.q_len, -1)
    bound = 2 * bf16_ulp(truth) + 2.0 ** -8 * dense_weight_abs(c).reshape(c.q_len, -1)
    err = np.abs(bits_to_f64(got).reshape(truth.shape) - truth)
    assert np.all(err <= bound), f"{what}: worst excess {float((err - bound).max()):.3g}"
