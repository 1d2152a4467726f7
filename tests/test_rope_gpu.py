"""Rotary embedding + K/V scatter on the GPU against the CPU oracle, through
the C ABI. The scatter is bit-exact: only the rows' slots change and V is
copied (bf16) or quantized (FP8, with its scale) exactly as the oracle does.
Rotated values (transcendental sin/cos, powf, expf) are mostly bit-identical
and otherwise within the rounding bound `within_ulp` states; rotated FP8 K is
within one E4M3 step."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits
from refs import bf16_ulp, bits_to_f64

pytestmark = pytest.mark.gpu
HEAD = 128


def within_ulp(got_bits, want_bits, pos=None, interleaved=False, min_equal=0.95, what=""):
    """One bf16 ulp of the output, plus (2^-8 + pos * 2^-21) of the rotary
    pair's magnitude: a rounding of the normalized input to bf16 may flip on
    a last-bit difference in rsqrt (one bf16 ulp of the pair's inputs, which
    stays that size when the rotated output cancels to a small value), and a
    1-ulp difference in a device powf / expf becomes an angle error that grows
    with the position (the reference computes pos * inv_freq in f32 too). Most
    elements must still be bit-identical."""
    g, w = bits_to_f64(got_bits), bits_to_f64(want_bits)
    assert np.all(np.isfinite(g)), f"{what}: non-finite"
    d = np.abs(g - w)
    bound = bf16_ulp(w) * 1.0001
    if pos is not None:
        w3 = w.reshape(len(pos), -1, HEAD)
        if interleaved:
            pm = np.repeat(np.maximum(np.abs(w3[..., 0::2]), np.abs(w3[..., 1::2])), 2, axis=-1)
        else:
            m = np.maximum(np.abs(w3[..., :64]), np.abs(w3[..., 64:]))
            pm = np.concatenate([m, m], axis=-1)
        p = np.asarray(pos, dtype=np.float64).reshape(len(pos), -1).max(axis=1)
        bound = bound + ((2.0 ** -8 + p[:, None, None] * 2.0 ** -21) * pm).reshape(bound.shape)
    assert np.all(d <= bound), f"{what}: worst excess {np.max(d - bound):.3g}"
    frac = np.mean(got_bits == want_bits)
    assert frac >= min_equal, f"{what}: only {frac:.4f} bit-identical"


def dev_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host_u8(t):
    return t.cpu().numpy()


# 12000 rows x 48 heads = 147 MB of qkv rows: past the 128 MiB where the kernel
# switches to nontemporal row loads.
@pytest.mark.parametrize("rows,hq,hk,theta", [(5, 4, 2, 1e6), (64, 16, 8, 1e6), (33, 32, 8, 1e4), (3, 2, 1, 5e5),
                                              (12000, 32, 8, 1e6)])
def test_qwen3_rope(oracle, rows, hq, hk, theta):
    c = W.rope_case("qwen3", rows, hq, hk, seed=rows + hq, pos_hi=40000)
    c.theta = theta
    qkv, kv = dev_bits(c.qkv), dev_bits(c.cache["kv"])
    oa.qwen3_rope(qkv, dev_bits(c.q_norm), dev_bits(c.k_norm), dev_i32(c.pos), dev_i32(c.slots), kv, rows, hq, hk,
                  c.eps, c.theta)
    torch.cuda.synchronize()
    q_want, kv_want = oracle.qwen3_rope(c.qkv, c.q_norm, c.k_norm, c.pos, c.slots, c.cache["kv"], hq, hk, c.eps,
                                        c.theta)
    q_got, kv_got = host_bits(qkv), host_bits(kv)
    within_ulp(q_got, q_want, c.pos, what="q")
    untouched = np.setdiff1d(np.arange(kv_got.shape[0]), c.slots)
    assert np.array_equal(kv_got[untouched], c.cache["kv"][untouched])
    k3g, k3w = kv_got.reshape(-1, 2 * hk, HEAD)[c.slots], kv_want.reshape(-1, 2 * hk, HEAD)[c.slots]
    within_ulp(np.ascontiguousarray(k3g[:, :hk]), np.ascontiguousarray(k3w[:, :hk]), c.pos, what="k")
    assert np.array_equal(k3g[:, hk:], k3w[:, hk:])  # V copied bit for bit


def test_qwen3_rope_dense(oracle):
    hq, hk, per, base, span, rows = 16, 8, 6, 10, 24, 30
    c = W.rope_case("dense", rows, hq, hk, seed=2, per=per, base=base, span=span)
    qkv, kv = dev_bits(c.qkv), dev_bits(c.cache["kv"])
    oa.qwen3_rope_dense(qkv, dev_bits(c.q_norm), dev_bits(c.k_norm), kv, rows, per, base, span, hq, hk, c.eps, c.theta)
    torch.cuda.synchronize()
    q_want, kv_want = oracle.qwen3_rope_dense(c.qkv, c.q_norm, c.k_norm, c.cache["kv"], rows, per, base, span, hq, hk,
                                              c.eps, c.theta)
    within_ulp(host_bits(qkv), q_want, c.pos, what="q")
    kvg, kvw = host_bits(kv).reshape(-1, 2 * hk, HEAD), kv_want.reshape(-1, 2 * hk, HEAD)
    slots = (np.arange(rows) // per) * span + c.pos
    within_ulp(np.ascontiguousarray(kvg[slots, :hk]), np.ascontiguousarray(kvw[slots, :hk]), c.pos, what="k")
    assert np.array_equal(np.delete(kvg, slots, axis=0), np.delete(kvw, slots, axis=0))
    assert np.array_equal(kvg[slots, hk:], kvw[slots, hk:])


@pytest.mark.parametrize("rows,hq,hk,mrope_hw,ld_pad", [(7, 4, 2, 20, 64), (300, 32, 8, 20, 0), (9, 8, 8, 0, 8)])
def test_hidream_qk_rope(oracle, rows, hq, hk, mrope_hw, ld_pad):
    c = W.rope_case("hidream", rows, hq, hk, seed=rows, pos_hi=4352, ld_pad=ld_pad)
    qkv, kc, vc = dev_bits(c.qkv), dev_bits(c.cache["k_cache"]), dev_bits(c.cache["v_cache"])
    oa.hidream_qk_rope(qkv, c.ld, dev_bits(c.q_norm), dev_bits(c.k_norm), dev_i32(c.pos), dev_i32(c.slots), kc, vc,
                       rows, hq, hk, mrope_hw, c.eps, c.theta)
    torch.cuda.synchronize()
    q_want, k_want, v_want = oracle.hidream_qk_rope(c.qkv, c.ld, c.q_norm, c.k_norm, c.pos, c.slots,
                                                    c.cache["k_cache"], c.cache["v_cache"], hq, hk, mrope_hw, c.eps,
                                                    c.theta)
    within_ulp(host_bits(qkv)[:, : (hq + 2 * hk) * HEAD], np.ascontiguousarray(q_want[:, : (hq + 2 * hk) * HEAD]),
               c.pos, what="q")
    assert np.array_equal(host_bits(qkv)[:, (hq + 2 * hk) * HEAD:], c.qkv[:, (hq + 2 * hk) * HEAD:])
    kg = host_bits(kc)
    within_ulp(np.ascontiguousarray(kg[c.slots]), np.ascontiguousarray(k_want[c.slots]), c.pos, what="k cache")
    assert np.array_equal(np.delete(kg, c.slots, axis=0), np.delete(k_want, c.slots, axis=0))
    assert np.array_equal(host_bits(vc), v_want)


@pytest.mark.parametrize("rows,heads", [(6, 4), (128, 32), (1, 1)])
def test_lm_rope_fp8(oracle, rows, heads):
    c = W.rope_case("lm", rows, heads, heads, seed=rows + heads, pos_hi=3000)
    qkv, kv = dev_bits(c.qkv), dev_u8(c.cache["kv"])
    oa.lm_rope(qkv, dev_i32(c.pos), dev_i32(c.slots), kv, rows, heads, c.coef)
    torch.cuda.synchronize()
    q_want, kv_want = oracle.lm_rope(c.qkv, c.pos, c.slots, c.cache["kv"], heads, c.coef)
    within_ulp(host_bits(qkv), q_want, c.pos, interleaved=True, what="q")
    kv_got = host_u8(kv)
    untouched = np.setdiff1d(np.arange(kv_got.shape[0]), c.slots)
    assert np.array_equal(kv_got[untouched], c.cache["kv"][untouched])
    body = 2 * heads * HEAD
    g, w = kv_got[c.slots], kv_want[c.slots]
    # V bytes and V scales: exact.
    assert np.array_equal(g[:, heads * HEAD:body], w[:, heads * HEAD:body])
    gs = np.ascontiguousarray(g[:, body:]).view(np.float32).reshape(rows, 2 * heads)
    ws = np.ascontiguousarray(w[:, body:]).view(np.float32).reshape(rows, 2 * heads)
    assert np.array_equal(gs[:, heads:], ws[:, heads:])
    # K: scales to f32 rounding of the rotated absmax, values to one E4M3 step.
    rel = np.abs(gs[:, :heads] - ws[:, :heads]) / ws[:, :heads]
    assert np.all(rel <= c.pos[:, None] * 2.0 ** -21 + 2.0 ** -22)

    def deq(b, s):
        v = torch.from_numpy(np.ascontiguousarray(b[:, : heads * HEAD])).view(torch.float8_e4m3fn).double().numpy()
        return v.reshape(rows, heads, HEAD) * s[:, :heads, None]

    dg, dw = deq(g, gs), deq(w, ws)
    amax = np.abs(dw).max(-1, keepdims=True)
    slack = c.pos[:, None, None] * 2.0 ** -21 * amax  # the same position-grown angle error as for q
    assert np.all(np.abs(dg - dw) <= 2.0 ** -3 * np.abs(dw) + ws[:, :heads, None] * 2.0 ** -9 * 1.0001 + slack)
    assert np.mean(g[:, : heads * HEAD] == w[:, : heads * HEAD]) >= 0.98


def test_lm_rope_then_fp8_decode_chain(oracle):
    """The FP8 cache lm_rope writes is the one lm_attend_fp8 reads: rope every
    position of 3 sessions on the GPU and on the oracle, then decode the last
    row of each; outputs agree to the attention tolerance."""
    heads, page = 4, 16
    lens = np.array([40, 17, 64])
    rng = np.random.default_rng(5)
    pages_per = (lens + page - 1) // page
    pool_pages = int(pages_per.sum()) + 2
    perm = rng.permutation(pool_pages).astype(np.int32)
    indptr = np.concatenate([[0], np.cumsum(pages_per)]).astype(np.int32)
    pages = perm[: indptr[-1]].copy()
    seq = np.concatenate([np.full(l, s) for s, l in enumerate(lens)]).astype(np.int32)
    pos = np.concatenate([np.arange(l) for l in lens]).astype(np.int32)
    slots = np.array([pages[indptr[s] + t // page] * page + t % page for s, t in zip(seq, pos)], np.int32)
    rows = len(pos)
    qkv = W.normal_bits(rng, (rows, 3 * heads * HEAD))
    kv0 = np.zeros((pool_pages * page, W.fp8_slot_bytes(heads)), np.uint8)
    coef = float(np.float32(-np.log(10000.0) * 2.0 / HEAD))
    q_o, kv_o = oracle.lm_rope(qkv, pos, slots, kv0, heads, coef)
    d_qkv, d_kv = dev_bits(qkv), dev_u8(kv0)
    oa.lm_rope(d_qkv, dev_i32(pos), dev_i32(slots), d_kv, rows, heads, coef)
    last = np.cumsum(lens) - 1
    d_last = d_qkv[torch.from_numpy(last).cuda()].contiguous()
    plan = oa.decode_plan(3, heads, heads, page, int(lens.max()))
    out = torch.zeros(3, heads * HEAD, dtype=torch.bfloat16, device="cuda")
    lpos = np.ascontiguousarray(pos[last])
    oa.lm_attend_fp8(d_last, d_kv, dev_i32(lpos), dev_i32(np.arange(3)), 0, dev_i32(indptr), dev_i32(pages), page, out,
                     heads, HEAD ** -0.5, 3000, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    want = oracle.lm_attend_fp8(np.ascontiguousarray(q_o[last]), kv_o, lpos, np.arange(3, dtype=np.int32), 0, indptr,
                                pages, page, heads, HEAD ** -0.5, 3000)
    assert_close(host_bits(out), want, what="rope -> fp8 decode")
