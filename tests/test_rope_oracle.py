"""The rotary + scatter oracle pinned by library routines (CPU):

* FP8 encode: torch's float8_e4m3fn cast (round to nearest even) on every
  finite bf16 value in range and on random f32 values;
* qwen3_rope / qwen3_rope_dense: transformers' Qwen3RMSNorm, Qwen3RotaryEmbedding
  and apply_rotary_pos_emb (half-split rotary) in float64;
* hidream_qk_rope: transformers' Qwen3-VL interleaved M-RoPE
  (Qwen3VLTextRotaryEmbedding with mrope_section [24, 20, 20] is mrope_hw 20);
* lm_rope: transformers' Helium rotary (interleaved pairs), and the FP8 bytes
  of V equal torch's cast of the scaled values exactly.

The scatter is checked by numpy: only the rows' slots change, V is copied bit
for bit. Error bounds: the oracle rounds the normalized value to bf16 before
the weight (as the reference does) and rounds its output, so a rotated pair
may differ from the float64 library result by 2^-7 of the pair's magnitude;
a wrong pairing, frequency or axis misses by O(1)."""
import warnings

import numpy as np
import pytest
import torch

import workloads as W
from refs import bits_to_f64

warnings.filterwarnings("ignore")
HEAD = 128


def _tf():
    from transformers import HeliumConfig, Qwen3Config
    from transformers.models.helium import modeling_helium as helium
    from transformers.models.qwen3 import modeling_qwen3 as qwen3
    from transformers.models.qwen3_vl import modeling_qwen3_vl as qwen3_vl
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    return dict(Qwen3Config=Qwen3Config, qwen3=qwen3, HeliumConfig=HeliumConfig, helium=helium, qwen3_vl=qwen3_vl,
                Qwen3VLTextConfig=Qwen3VLTextConfig)


def lib_norm(x, w, eps):
    """Qwen3RMSNorm in float64 over [..., 128] rows."""
    T = _tf()
    m = T["qwen3"].Qwen3RMSNorm(HEAD, eps=eps).double()
    with torch.no_grad():
        m.weight.copy_(torch.from_numpy(bits_to_f64(w)))
        return m(torch.from_numpy(x)).numpy()


def lib_half_rope(x, pos, theta):
    """[rows][heads][128] float64 rotated at pos[rows] by Qwen3's rotary."""
    T = _tf()
    cfg = T["Qwen3Config"](head_dim=HEAD, hidden_size=1024, num_attention_heads=8, num_key_value_heads=8,
                           rope_theta=theta)
    rot = T["qwen3"].Qwen3RotaryEmbedding(cfg)
    xt = torch.from_numpy(x).permute(1, 0, 2)[None]  # [1, heads, rows, 128]
    cos, sin = rot(xt, torch.from_numpy(pos.astype(np.int64))[None])
    out, _ = T["qwen3"].apply_rotary_pos_emb(xt, xt, cos, sin)
    return out[0].permute(1, 0, 2).numpy()


def pair_bound(x):
    """2^-7 of each rotary pair's magnitude, per element ([..., 128], half-split)."""
    m = np.maximum(np.abs(x[..., :64]), np.abs(x[..., 64:]))
    return 2.0 ** -7 * np.concatenate([m, m], axis=-1) + 1e-30


# ---------------------------------------------------------------- FP8 encode
def test_e4m3_encode_matches_torch_on_every_bf16_in_range(oracle):
    vals = bits_to_f64(np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)).astype(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 448)]
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.f32_to_e4m3(v) for v in vals], dtype=np.uint8)
    assert np.array_equal(got, want)


def test_e4m3_encode_random_and_saturation(oracle):
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(20000) * np.exp2(rng.integers(-12, 9, 20000))).astype(np.float32)
    vals = vals[np.abs(vals) <= 448]
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.f32_to_e4m3(v) for v in vals], dtype=np.uint8)
    assert np.array_equal(got, want)
    assert [oracle.f32_to_e4m3(v) for v in (448.5, 463.9, 1e6, -1e6, float("inf"))] == [0x7E, 0x7E, 0x7E, 0xFE, 0x7E]
    assert oracle.f32_to_e4m3(float("nan")) & 0x7F == 0x7F
    assert oracle.f32_to_e4m3(-0.0) == 0x80


# ---------------------------------------------------------------- qwen3_rope
@pytest.mark.parametrize("hq,hk,theta", [(16, 8, 1e6), (4, 4, 1e4)])
def test_qwen3_rope_matches_transformers(oracle, hq, hk, theta):
    c = W.rope_case("qwen3", 9, hq, hk, seed=hq + hk, pos_hi=40000)
    c.theta = theta
    q2, kv2 = oracle.qwen3_rope(c.qkv, c.q_norm, c.k_norm, c.pos, c.slots, c.cache["kv"], hq, hk, c.eps, c.theta)
    x = bits_to_f64(c.qkv).reshape(c.rows, hq + 2 * hk, HEAD)
    qn = lib_norm(x[:, :hq], c.q_norm, c.eps)
    kn = lib_norm(x[:, hq:hq + hk], c.k_norm, c.eps)
    q_want, k_want = lib_half_rope(qn, c.pos, theta), lib_half_rope(kn, c.pos, theta)
    q_got = bits_to_f64(q2).reshape(c.rows, hq + 2 * hk, HEAD)[:, :hq]
    assert np.all(np.abs(q_got - q_want) <= pair_bound(qn))
    kv_got = kv2.reshape(-1, 2 * hk, HEAD)
    assert np.all(np.abs(bits_to_f64(kv_got[c.slots, :hk]) - k_want) <= pair_bound(kn))
    assert np.array_equal(kv_got[c.slots, hk:], c.qkv.reshape(c.rows, -1, HEAD)[:, hq + hk:])  # V copied exactly
    untouched = np.setdiff1d(np.arange(kv2.shape[0]), c.slots)
    assert np.array_equal(kv2[untouched], c.cache["kv"][untouched])
    assert np.array_equal(q2.reshape(c.rows, -1, HEAD)[:, hq:], c.qkv.reshape(c.rows, -1, HEAD)[:, hq:])


def test_qwen3_rope_position_zero_is_the_rounded_norm(oracle):
    """At pos 0 the rotation is the identity: out = bf16(bf16(x r) w)."""
    c = W.rope_case("qwen3", 4, 2, 1, seed=3)
    c.pos[:] = 0
    q2, _ = oracle.qwen3_rope(c.qkv, c.q_norm, c.k_norm, c.pos, c.slots, c.cache["kv"], 2, 1, c.eps, c.theta)
    x = bits_to_f64(c.qkv).reshape(4, 4, HEAD)[:, :2].astype(np.float32)
    r = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True, dtype=np.float32) / HEAD + np.float32(c.eps))
    xr = W.f32_to_bf16_bits((x * r).astype(np.float32))
    want = W.f32_to_bf16_bits(bits_to_f64(xr).astype(np.float32) * bits_to_f64(c.q_norm).astype(np.float32))
    got = q2.reshape(4, 4, HEAD)[:, :2]
    assert np.mean(got == want) > 0.999  # f32 sum order may flip a rare rounding


def test_qwen3_rope_dense_slots_and_positions(oracle):
    hq, hk, per, base, span = 4, 2, 5, 3, 12
    c = W.rope_case("dense", 10, hq, hk, seed=11, per=per, base=base, span=span)
    q2, kv2 = oracle.qwen3_rope_dense(c.qkv, c.q_norm, c.k_norm, c.cache["kv"], 10, per, base, span, hq, hk, c.eps,
                                      c.theta)
    slots = (np.arange(10) // per) * span + base + np.arange(10) % per
    q3, kv3 = oracle.qwen3_rope(c.qkv, c.q_norm, c.k_norm, c.pos, slots.astype(np.int32), c.cache["kv"], hq, hk,
                                c.eps, c.theta)
    assert np.array_equal(q2, q3) and np.array_equal(kv2, kv3)


# ----------------------------------------------------------- hidream_qk_rope
def test_hidream_mrope_matches_qwen3_vl(oracle):
    T = _tf()
    hq, hk, theta = 4, 2, 5e6
    c = W.rope_case("hidream", 7, hq, hk, seed=5, pos_hi=300, ld_pad=64)
    c.theta = theta
    q2, kc, vc = oracle.hidream_qk_rope(c.qkv, c.ld, c.q_norm, c.k_norm, c.pos, c.slots, c.cache["k_cache"],
                                        c.cache["v_cache"], hq, hk, 20, c.eps, theta)
    x = bits_to_f64(c.qkv)[:, : (hq + 2 * hk) * HEAD].reshape(c.rows, -1, HEAD)
    cfg = T["Qwen3VLTextConfig"](head_dim=HEAD, hidden_size=1024, num_attention_heads=8, num_key_value_heads=8,
                                 rope_parameters={"rope_type": "default", "rope_theta": theta,
                                                  "mrope_section": [24, 20, 20]})
    rot = T["qwen3_vl"].Qwen3VLTextRotaryEmbedding(cfg)
    p3 = torch.from_numpy(c.pos.T.astype(np.int64))[:, None, :]  # [3, 1, rows]

    def vl(xn):
        xt = torch.from_numpy(xn).permute(1, 0, 2)[None]
        cos, sin = rot(xt, p3)
        return T["qwen3_vl"].apply_rotary_pos_emb(xt, xt, cos, sin)[0][0].permute(1, 0, 2).numpy()

    qn = lib_norm(x[:, :hq], c.q_norm, c.eps)
    kn = lib_norm(x[:, hq:hq + hk], c.k_norm, c.eps)
    q_got = bits_to_f64(q2[:, : (hq + 2 * hk) * HEAD]).reshape(c.rows, -1, HEAD)[:, :hq]
    assert np.all(np.abs(q_got - vl(qn)) <= pair_bound(qn))
    k_got = bits_to_f64(kc.reshape(-1, hk, HEAD)[c.slots])
    assert np.all(np.abs(k_got - vl(kn)) <= pair_bound(kn))
    assert np.array_equal(vc.reshape(-1, hk, HEAD)[c.slots], c.qkv[:, : (hq + 2 * hk) * HEAD].reshape(
        c.rows, -1, HEAD)[:, hq + hk:])
    assert np.array_equal(q2[:, (hq + 2 * hk) * HEAD:], c.qkv[:, (hq + 2 * hk) * HEAD:])  # row padding untouched


def test_hidream_mrope_hw0_is_plain_rope_at_t(oracle):
    hq, hk = 2, 1
    c = W.rope_case("hidream", 5, hq, hk, seed=6)
    a = oracle.hidream_qk_rope(c.qkv, c.ld, c.q_norm, c.k_norm, c.pos, c.slots, c.cache["k_cache"],
                               c.cache["v_cache"], hq, hk, 0, c.eps, c.theta)
    kv = np.zeros((c.cache["k_cache"].shape[0], 2 * hk * HEAD), np.uint16)
    b = oracle.qwen3_rope(c.qkv, c.q_norm, c.k_norm, np.ascontiguousarray(c.pos[:, 0]), c.slots, kv, hq, hk, c.eps,
                          c.theta)
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[1].reshape(-1, hk, HEAD)[c.slots], b[1].reshape(-1, 2 * hk, HEAD)[c.slots, :hk])


# ------------------------------------------------------------------- lm_rope
def test_lm_rope_matches_helium_and_torch_fp8(oracle):
    T = _tf()
    heads = 4
    c = W.rope_case("lm", 6, heads, heads, seed=8, pos_hi=3000)
    q2, kv2 = oracle.lm_rope(c.qkv, c.pos, c.slots, c.cache["kv"], heads, c.coef)
    x = bits_to_f64(c.qkv).reshape(c.rows, 3 * heads, HEAD)
    cfg = T["HeliumConfig"](head_dim=HEAD, hidden_size=1024, num_attention_heads=8, num_key_value_heads=8,
                            rope_theta=10000.0)
    rot = T["helium"].HeliumRotaryEmbedding(cfg)

    def hel(xn):
        xt = torch.from_numpy(xn).permute(1, 0, 2)[None]
        cos, sin = rot(xt, torch.from_numpy(c.pos.astype(np.int64))[None])
        return T["helium"].apply_rotary_pos_emb(xt, xt, cos, sin)[0][0].permute(1, 0, 2).numpy()

    def bound(xn):  # interleaved pairs (2i, 2i + 1)
        m = np.maximum(np.abs(xn[..., 0::2]), np.abs(xn[..., 1::2]))
        return 2.0 ** -7 * np.repeat(m, 2, axis=-1) + 1e-30

    q_got = bits_to_f64(q2).reshape(c.rows, 3 * heads, HEAD)[:, :heads]
    assert np.all(np.abs(q_got - hel(x[:, :heads])) <= bound(x[:, :heads]))
    body = 2 * heads * HEAD
    slot = kv2[c.slots]
    vals = torch.from_numpy(np.ascontiguousarray(slot[:, :body])).view(torch.float8_e4m3fn).double().numpy()
    sc = np.ascontiguousarray(slot[:, body:]).view(np.float32).reshape(c.rows, 2 * heads)
    deq = vals.reshape(c.rows, 2 * heads, HEAD) * sc[:, :, None]
    k_lib = hel(x[:, heads:2 * heads])
    amax = np.abs(k_lib).max(-1)
    assert np.allclose(sc[:, :heads], amax / 448.0, rtol=2e-3)
    assert np.all(np.abs(deq[:, :heads] - k_lib) <= 2.0 ** -4 * np.abs(k_lib) + sc[:, :heads, None] * 2.0 ** -9
                  + 2.0 ** -7 * amax[..., None])
    # V: the scale is exactly max(amax * f32(1/448), 1e-12) and the bytes are torch's cast of v * (1 / scale).
    v = x[:, 2 * heads:].astype(np.float32)
    vs = np.maximum(np.abs(v).max(-1) * np.float32(1.0 / 448.0), np.float32(1e-12)).astype(np.float32)
    assert np.array_equal(sc[:, heads:], vs)
    want = torch.from_numpy((v * (np.float32(1.0) / vs)[..., None]).astype(np.float32)).to(torch.float8_e4m3fn)
    assert np.array_equal(slot[:, heads * HEAD:body].reshape(c.rows, heads, HEAD), want.view(torch.uint8).numpy())
    untouched = np.setdiff1d(np.arange(kv2.shape[0]), c.slots)
    assert np.array_equal(kv2[untouched], c.cache["kv"][untouched])
