"""The dense and head-64 attention oracles pinned on the CPU:

* qwen3_attend_dense: float64 SDPA over the dense slots (n / per) * span + t,
  and bit-identical to the paged oracle given the same slots as a page-1 table;
* mimi_attend: float64 SDPA over ring slots (p - len + 1 + t) % context
  gathered by numpy, with rings that have wrapped;
* codec_attention: the ring write (transformers' Qwen3 rotary at head_dim 64
  for k, V copied, every other frame untouched) and the output against float64
  SDPA over the ring after the write;
* lm_dep_kv_attend: the workspace write and float64 SDPA over steps 0 .. step.
"""
import warnings

import numpy as np
import pytest
import torch

import workloads as W
from refs import bf16_ulp, bits_to_f64

warnings.filterwarnings("ignore")


def sdpa(q, k, v, scale):
    """q [D], k/v [L][D] float64 -> [D]."""
    o = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q)[None, None],
                                                         torch.from_numpy(k)[None], torch.from_numpy(v)[None],
                                                         scale=scale)
    return o[0, 0].numpy()


def assert_ulp(got_bits, want, what):
    g = bits_to_f64(got_bits).reshape(want.shape)
    d = np.abs(g - want)
    assert np.all(d <= bf16_ulp(want) * 1.0001), f"{what}: worst {d.max():.3g}"


def test_qwen3_attend_dense(oracle):
    hq, hk, per, base, span = 16, 8, 5, 7, 16
    rows = 3 * per
    rng = np.random.default_rng(1)
    qkv = W.normal_bits(rng, (rows, (hq + 2 * hk) * 128))
    kv = W.normal_bits(rng, ((rows // per) * span, 2 * hk * 128))
    got = oracle.qwen3_attend_dense(qkv, kv, per, base, span, hq, hk, 128 ** -0.5)
    want = np.zeros((rows, hq, 128))
    kvf = bits_to_f64(kv).reshape(-1, 2 * hk, 128)
    for n in range(rows):
        ln = base + n % per + 1
        sl = (n // per) * span + np.arange(ln)
        for h in range(hq):
            q = bits_to_f64(qkv[n, h * 128:(h + 1) * 128])
            want[n, h] = sdpa(q, kvf[sl, h // 2], kvf[sl, hk + h // 2], 128 ** -0.5)
    assert_ulp(got, want, "dense")
    # The same rows as a page-1 table over the same slots: bit-identical.
    lens = base + np.arange(rows) % per + 1
    indptr = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pages = np.concatenate([(n // per) * span + np.arange(l) for n, l in enumerate(lens)]).astype(np.int32)
    paged = oracle.paged_attend(qkv, kv, (lens - 1).astype(np.int32), None, 0, indptr, pages, 1, hq, hk, 128 ** -0.5)
    assert np.array_equal(got, paged)


def mimi_case(seed, sessions=3, T=2, heads=4, context=40, pos_hi=60):
    rng = np.random.default_rng(seed)
    slot_bytes = 2 * heads * 64 * 2
    stride = context * slot_bytes + 64  # padded lines
    lines = rng.permutation(sessions + 2)[:sessions].astype(np.int32)
    state = rng.integers(0, 256, size=((sessions + 2) * stride,), dtype=np.uint8)
    # make every ring hold finite bf16 values
    body = W.normal_bits(rng, ((sessions + 2) * stride // 2,))
    state = body.view(np.uint8).copy()
    pos = rng.integers(0, pos_hi, size=sessions).astype(np.int32)
    qkv = W.normal_bits(rng, (sessions * T, 3 * heads * 64))
    return dict(qkv=qkv, pos=pos, lines=lines, state=state, T=T, heads=heads, context=context, stride=stride,
                rows=sessions * T)


@pytest.mark.parametrize("seed,context,pos_hi", [(1, 40, 60), (2, 250, 400), (3, 16, 5)])
def test_mimi_attend_matches_sdpa(oracle, seed, context, pos_hi):
    c = mimi_case(seed, context=context, pos_hi=pos_hi)
    scale = 64 ** -0.5
    got = oracle.mimi_attend(c["qkv"], c["pos"], c["lines"], c["state"], c["rows"], c["T"], c["heads"], scale,
                             c["context"], c["stride"])
    heads, T = c["heads"], c["T"]
    want = np.zeros((c["rows"], heads, 64))
    for n in range(c["rows"]):
        s = n // T
        p = int(c["pos"][s]) * T + n % T
        ln = min(p + 1, c["context"])
        ring = bits_to_f64(c["state"][c["lines"][s] * c["stride"]:][: c["context"] * 2 * heads * 64 * 2]
                           .view(np.uint16)).reshape(c["context"], 2 * heads, 64)
        sl = (p - ln + 1 + np.arange(ln)) % c["context"]
        for h in range(heads):
            q = bits_to_f64(c["qkv"][n, h * 64:(h + 1) * 64])
            want[n, h] = sdpa(q, ring[sl, h], ring[sl, heads + h], scale)
    assert_ulp(got, want, "mimi")


def codec_case(seed, sessions=4, heads=4, pos_hi=200):
    rng = np.random.default_rng(seed)
    width = heads * 64
    ring_bytes = 2 * 72 * width * 2
    stride = ring_bytes + 128
    lines = rng.permutation(sessions + 1)[:sessions].astype(np.int32)
    state = W.normal_bits(rng, ((sessions + 1) * stride // 2,)).view(np.uint8).copy()
    pos = rng.integers(0, pos_hi, size=sessions).astype(np.int32)
    pos[0] = 0  # a first frame: one key
    qkv = W.normal_bits(rng, (sessions, 3 * width))
    return dict(qkv=qkv, pos=pos, lines=lines, state=state, heads=heads, stride=stride, rows=sessions, width=width)


def test_codec_attention_ring_write_and_output(oracle):
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as q3

    theta = 10000.0
    c = codec_case(4)
    heads, width = c["heads"], c["width"]
    out, kv2 = oracle.codec_attention(c["qkv"], c["pos"], c["lines"], c["state"], c["rows"], c["stride"], heads, theta)
    rot = q3.Qwen3RotaryEmbedding(Qwen3Config(head_dim=64, hidden_size=256, num_attention_heads=4,
                                              num_key_value_heads=4, rope_theta=theta))
    changed = np.zeros(len(kv2), bool)
    for r in range(c["rows"]):
        p = int(c["pos"][r])
        x = bits_to_f64(c["qkv"][r]).reshape(3, heads, 64)
        xt = torch.from_numpy(x[:2]).reshape(1, 2 * heads, 1, 64)
        cos, sin = rot(xt, torch.tensor([[p]]))
        qk = q3.apply_rotary_pos_emb(xt, xt, cos, sin)[0].reshape(2, heads, 64).numpy()
        base = int(c["lines"][r]) * c["stride"]
        ring = kv2[base:base + 2 * 72 * width * 2].view(np.uint16).reshape(2, 72, heads, 64)
        f = p % 72
        kw = bits_to_f64(ring[0, f])
        pm = np.maximum(np.abs(qk[1][:, :32]), np.abs(qk[1][:, 32:]))
        assert np.all(np.abs(kw - qk[1]) <= bf16_ulp(qk[1]) + 2.0 ** -8 * np.concatenate([pm, pm], -1))
        assert np.array_equal(ring[1, f], c["qkv"][r].reshape(3, heads, 64)[2])
        for blk in (0, 1):
            off = base + (blk * 72 + f) * width * 2
            changed[off:off + width * 2] = True
        # output: float64 SDPA over frames p - n + 1 .. p of the ring after the write, q rounded to bf16 as written
        n = min(p + 1, 72)
        frames = (p - n + 1 + np.arange(n)) % 72
        qb = bits_to_f64(W.f32_to_bf16_bits(qk[0].astype(np.float32)))
        rf = bits_to_f64(ring)
        want = np.stack([sdpa(qb[h], rf[0, frames, h], rf[1, frames, h], 0.125) for h in range(heads)])
        got = bits_to_f64(out[r]).reshape(heads, 64)
        assert np.abs(got - want).max() <= 2e-2 and np.abs(got - want).mean() <= 2e-3
        assert np.mean(np.abs(got - want) <= bf16_ulp(want) * 1.0001) >= 0.98
    assert np.array_equal(kv2[~changed], c["state"][~changed])


@pytest.mark.parametrize("step", [0, 3, 7])
def test_lm_dep_kv_attend(oracle, step):
    rng = np.random.default_rng(step)
    seqs, heads = 3, 16
    width = heads * 64
    qkv = W.normal_bits(rng, (seqs, 3 * width))
    ws = W.normal_bits(rng, (seqs, 8, 2, width))
    out, ws2 = oracle.lm_dep_kv_attend(qkv, ws, step, seqs, heads, 0.125)
    x = qkv.reshape(seqs, 3, heads, 64)
    want_ws = ws.copy()
    want_ws[:, step, 0] = x[:, 1].reshape(seqs, width)
    want_ws[:, step, 1] = x[:, 2].reshape(seqs, width)
    assert np.array_equal(ws2, want_ws)
    wf = bits_to_f64(want_ws).reshape(seqs, 8, 2, heads, 64)
    want = np.zeros((seqs, heads, 64))
    for s in range(seqs):
        for h in range(heads):
            want[s, h] = sdpa(bits_to_f64(x[s, 0, h]), wf[s, : step + 1, 0, h], wf[s, : step + 1, 1, h], 0.125)
    assert_ulp(out, want, "dep")


def _helium64(x, pos):
    """[rows][heads][64] float64 turned at pos[rows] by transformers' Helium
    rotary (interleaved pairs (2i, 2i + 1), theta 10000) at head_dim 64."""
    from transformers import HeliumConfig
    from transformers.models.helium import modeling_helium as helium
    cfg = HeliumConfig(head_dim=64, hidden_size=512, num_attention_heads=8, num_key_value_heads=8, rope_theta=10000.0)
    rot = helium.HeliumRotaryEmbedding(cfg)
    xt = torch.from_numpy(x).permute(1, 0, 2)[None]
    cos, sin = rot(xt, torch.from_numpy(pos.astype(np.int64))[None])
    return helium.apply_rotary_pos_emb(xt, xt, cos, sin)[0][0].permute(1, 0, 2).numpy()


@pytest.mark.parametrize("seed,context,pos_hi", [(4, 40, 60), (5, 250, 3000)])
def test_mimi_rope_kv_matches_helium_rotary(oracle, seed, context, pos_hi):
    """mimi_rope_kv: q turned in place and k turned into ring slot p % context
    by the interleaved rotary (against transformers' Helium rotary at head_dim
    64, to 2^-7 of each pair's magnitude: the oracle rounds its output), v
    copied bit for bit; every other byte of the state and of qkv unchanged."""
    c = mimi_case(seed, context=context, pos_hi=pos_hi)
    heads, T, rows = c["heads"], c["T"], c["rows"]
    coef = float(np.float32(-np.log(10000.0) * 2.0 / 64))
    q2, st2 = oracle.mimi_rope_kv(c["qkv"], c["pos"], c["lines"], c["state"], rows, T, heads, coef, c["context"],
                                  c["stride"])
    x = bits_to_f64(c["qkv"]).reshape(rows, 3 * heads, 64)
    p = np.array([int(c["pos"][n // T]) * T + n % T for n in range(rows)])

    def bound(xn):
        m = np.maximum(np.abs(xn[..., 0::2]), np.abs(xn[..., 1::2]))
        return 2.0 ** -7 * np.repeat(m, 2, axis=-1) + 1e-30

    q_got = bits_to_f64(q2).reshape(rows, 3 * heads, 64)
    assert np.all(np.abs(q_got[:, :heads] - _helium64(x[:, :heads], p)) <= bound(x[:, :heads]))
    assert np.array_equal(q2.reshape(rows, 3, -1)[:, 1:], c["qkv"].reshape(rows, 3, -1)[:, 1:])
    k_want = _helium64(x[:, heads:2 * heads], p)
    touched = np.zeros(len(c["state"]), bool)
    slot_bytes = 2 * heads * 64 * 2
    for n in range(rows):
        s = n // T
        at = int(c["lines"][s]) * c["stride"] + (p[n] % c["context"]) * slot_bytes
        slot = st2[at:at + slot_bytes].view(np.uint16).reshape(2 * heads, 64)
        assert np.all(np.abs(bits_to_f64(slot[:heads]) - k_want[n]) <= bound(x[n, heads:2 * heads]))
        assert np.array_equal(slot[heads:], c["qkv"][n].reshape(3 * heads, 64)[2 * heads:])
        touched[at:at + slot_bytes] = True
    assert np.array_equal(st2[~touched], c["state"][~touched])


def test_lm_copy_kv_is_slot_indexing(oracle):
    """lm_copy_kv: slot dst[r] takes slot src[r]'s bytes (FP8 slots of 8448
    bytes), the rest of the cache unchanged; equal to numpy's indexing."""
    rng = np.random.default_rng(6)
    slots, sb = 300, 8448
    kv = rng.integers(0, 256, size=(slots, sb), dtype=np.uint8)
    perm = rng.permutation(slots)
    src, dst = perm[:40].astype(np.int32), perm[40:80].astype(np.int32)
    got = oracle.lm_copy_kv(kv, src, dst, sb)
    want = kv.copy()
    want[dst] = kv[src]
    assert np.array_equal(got, want)
