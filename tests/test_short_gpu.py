"""Dense (code predictor) and head-64 ring attentions on the GPU against the
CPU oracle, through the C ABI. Outputs to the attention tolerance (max-abs
2e-2, mean-abs 2e-3); ring / workspace writes: V bit-exact, rotated K to the
rotary rounding bound, every other byte untouched."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits
from refs import bf16_ulp, bits_to_f64
from test_short_oracle import codec_case, mimi_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hq,hk,per,base,span,nseq", [(16, 8, 5, 7, 16, 3), (16, 8, 16, 0, 17, 64), (8, 8, 1, 30, 40, 5)])
def test_qwen3_attend_dense(oracle, hq, hk, per, base, span, nseq):
    rows = nseq * per
    rng = np.random.default_rng(per + base)
    qkv = W.normal_bits(rng, (rows, (hq + 2 * hk) * 128))
    kv = W.normal_bits(rng, (nseq * span, 2 * hk * 128))
    want = oracle.qwen3_attend_dense(qkv, kv, per, base, span, hq, hk, 128 ** -0.5, nthreads=8)
    plan = oa.decode_plan(rows, hq, hk, 1, base + per)
    out = torch.zeros(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.qwen3_attend_dense(dev_bits(qkv), dev_bits(kv), per, base, span, out, hq, hk, 128 ** -0.5, plan,
                          oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(host_bits(out), want, what="qwen3_attend_dense")


@pytest.mark.parametrize("seed,context,pos_hi,sessions,T", [(1, 40, 60, 3, 2), (2, 250, 400, 128, 2), (3, 16, 5, 2, 1)])
def test_mimi_attend(oracle, seed, context, pos_hi, sessions, T):
    c = mimi_case(seed, sessions=sessions, T=T, heads=8, context=context, pos_hi=pos_hi)
    want = oracle.mimi_attend(c["qkv"], c["pos"], c["lines"], c["state"], c["rows"], c["T"], c["heads"], 0.125,
                              c["context"], c["stride"])
    out = torch.zeros(c["rows"], c["heads"] * 64, dtype=torch.bfloat16, device="cuda")
    state = torch.from_numpy(c["state"]).cuda()
    oa.mimi_attend(dev_bits(c["qkv"]), dev_i32(c["pos"]), dev_i32(c["lines"]), state, out, c["rows"], c["T"],
                   c["heads"], 0.125, c["context"], c["stride"])
    torch.cuda.synchronize()
    assert_close(host_bits(out), want, what="mimi_attend")


@pytest.mark.parametrize("seed,sessions,heads,pos_hi", [(4, 4, 4, 200), (5, 64, 16, 1000), (6, 3, 2, 3)])
def test_codec_attention(oracle, seed, sessions, heads, pos_hi):
    c = codec_case(seed, sessions=sessions, heads=heads, pos_hi=pos_hi)
    theta = 10000.0
    want, kv_want = oracle.codec_attention(c["qkv"], c["pos"], c["lines"], c["state"], c["rows"], c["stride"], heads,
                                           theta)
    out = torch.zeros(c["rows"], heads * 64, dtype=torch.bfloat16, device="cuda")
    kv = torch.from_numpy(c["state"]).cuda()
    oa.codec_attention(dev_bits(c["qkv"]), dev_i32(c["pos"]), dev_i32(c["lines"]), kv, out, c["rows"], c["stride"],
                       heads, theta)
    torch.cuda.synchronize()
    assert_close(host_bits(out), want, what="codec_attention")
    kv_got = kv.cpu().numpy()
    diff = kv_got != kv_want
    # Only rotated K bytes may differ (a rounding flip); V and everything else are exact.
    width = heads * 64
    for r in range(c["rows"]):
        base = int(c["lines"][r]) * c["stride"]
        f = int(c["pos"][r]) % 72
        off = base + f * width * 2
        g = bits_to_f64(kv_got[off:off + width * 2].view(np.uint16))
        w = bits_to_f64(kv_want[off:off + width * 2].view(np.uint16))
        p = int(c["pos"][r])
        # one bf16 ulp plus (2^-22 + p 2^-21) of the rotary pair's magnitude (half-split, pairs i, i + 32)
        k_in = np.abs(bits_to_f64(c["qkv"][r].reshape(3, heads, 64)[1]))
        pm = np.maximum(k_in[:, :32], k_in[:, 32:])
        pm = np.concatenate([pm, pm], -1).reshape(-1)
        assert np.all(np.abs(g - w) <= bf16_ulp(w) * 1.0001 + (2.0 ** -22 + p * 2.0 ** -21) * pm)
        diff[off:off + width * 2] = False
    assert not diff.any(), "bytes outside the rotated K frames differ"


@pytest.mark.parametrize("step", [0, 5, 7])
def test_lm_dep_kv_attend(oracle, step):
    rng = np.random.default_rng(10 + step)
    seqs, heads = 32, 16
    width = heads * 64
    qkv = W.normal_bits(rng, (seqs, 3 * width))
    ws = W.normal_bits(rng, (seqs, 8, 2, width))
    want, ws_want = oracle.lm_dep_kv_attend(qkv, ws, step, seqs, heads, 0.125)
    out = torch.zeros(seqs, width, dtype=torch.bfloat16, device="cuda")
    d_ws = dev_bits(ws)
    oa.lm_dep_kv_attend(dev_bits(qkv), d_ws, step, out, seqs, heads, 0.125)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(d_ws), ws_want)
    assert_close(host_bits(out), want, what="lm_dep_kv_attend")


def _interleaved_bound(x, p):
    """One bf16 ulp plus (2^-22 + p 2^-21) of each interleaved pair's
    magnitude: device and host sin/cos and exp may round apart by that much."""
    m = np.maximum(np.abs(x[..., 0::2]), np.abs(x[..., 1::2]))
    return np.repeat(m, 2, axis=-1) * (2.0 ** -22 + p * 2.0 ** -21)


@pytest.mark.parametrize("seed,context,pos_hi,sessions,T", [(7, 40, 60, 3, 2), (8, 250, 3000, 128, 2), (9, 16, 5, 2, 1)])
def test_mimi_rope_kv(oracle, seed, context, pos_hi, sessions, T):
    """Mimi's rotary + ring write against the oracle: rotated q (in place) and
    k (ring slot) to the rotary rounding bound, v bit-exact, every other byte
    of qkv and of the state untouched; then mimi_attend over the written rings
    against the oracle's chain."""
    c = mimi_case(seed, sessions=sessions, T=T, heads=8, context=context, pos_hi=pos_hi)
    heads, rows = c["heads"], c["rows"]
    coef = float(np.float32(-np.log(10000.0) * 2.0 / 64))
    q_want, st_want = oracle.mimi_rope_kv(c["qkv"], c["pos"], c["lines"], c["state"], rows, T, heads, coef,
                                          c["context"], c["stride"])
    qkv = dev_bits(c["qkv"])
    state = torch.from_numpy(c["state"]).cuda()
    oa.mimi_rope_kv(qkv, dev_i32(c["pos"]), dev_i32(c["lines"]), state, rows, T, heads, coef, c["context"],
                    c["stride"])
    torch.cuda.synchronize()
    q_got, st_got = host_bits(qkv), state.cpu().numpy()
    p = np.array([int(c["pos"][n // T]) * T + n % T for n in range(rows)], np.float64)
    x = bits_to_f64(c["qkv"]).reshape(rows, 3 * heads, 64)
    g = bits_to_f64(q_got).reshape(rows, 3 * heads, 64)
    w = bits_to_f64(q_want).reshape(rows, 3 * heads, 64)
    b = bf16_ulp(w[:, :heads]) * 1.0001 + _interleaved_bound(x[:, :heads], p[:, None, None])
    assert np.all(np.abs(g[:, :heads] - w[:, :heads]) <= b), "rotated q"
    assert np.array_equal(q_got.reshape(rows, 3, -1)[:, 1:], c["qkv"].reshape(rows, 3, -1)[:, 1:])
    slot_bytes = 2 * heads * 64 * 2
    diff = st_got != st_want
    for n in range(rows):
        at = int(c["lines"][n // T]) * c["stride"] + (int(p[n]) % c["context"]) * slot_bytes
        gs = bits_to_f64(st_got[at:at + slot_bytes].view(np.uint16)).reshape(2 * heads, 64)
        ws = bits_to_f64(st_want[at:at + slot_bytes].view(np.uint16)).reshape(2 * heads, 64)
        bk = bf16_ulp(ws[:heads]) * 1.0001 + _interleaved_bound(x[n, heads:2 * heads], p[n])
        assert np.all(np.abs(gs[:heads] - ws[:heads]) <= bk), f"rotated k, row {n}"
        assert np.array_equal(gs[heads:], ws[heads:]), f"v, row {n}"
        diff[at:at + slot_bytes // 2] = False
    assert not diff.any(), "bytes outside the rotated K heads differ"
    # The chain: attention over the rings just written, from the rotated q.
    out = torch.zeros(rows, heads * 64, dtype=torch.bfloat16, device="cuda")
    oa.mimi_attend(qkv, dev_i32(c["pos"]), dev_i32(c["lines"]), state, out, rows, T, heads, 0.125, c["context"],
                   c["stride"])
    torch.cuda.synchronize()
    want = oracle.mimi_attend(q_want, c["pos"], c["lines"], st_want, rows, T, heads, 0.125, c["context"],
                              c["stride"])
    assert_close(host_bits(out), want, what="mimi_rope_kv -> mimi_attend")


@pytest.mark.parametrize("slot_bytes,tokens", [(8448, 300), (16384, 64), (8448, 0), (16, 5)])
def test_lm_copy_kv(oracle, slot_bytes, tokens):
    """Prefix K/V reuse: slot dst[r] takes slot src[r]'s bytes, bit for bit,
    everything else untouched (FP8 slots of 8448 bytes, bf16 slots of 16 KiB)."""
    rng = np.random.default_rng(slot_bytes + tokens)
    slots = 2 * tokens + 17
    kv = rng.integers(0, 256, size=(slots, slot_bytes), dtype=np.uint8)
    perm = rng.permutation(slots).astype(np.int32)
    src, dst = perm[:tokens], perm[tokens:2 * tokens]
    d_kv = torch.from_numpy(kv).cuda()
    oa.lm_copy_kv(d_kv, dev_i32(src), dev_i32(dst), tokens, slot_bytes)
    torch.cuda.synchronize()
    want = oracle.lm_copy_kv(kv, src, dst, slot_bytes)
    assert np.array_equal(d_kv.cpu().numpy(), want)
