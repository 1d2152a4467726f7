"""Synthetic workloads of the attention path: the five shapes the benchmark
names, and small cases of the same construction for tests.

Index data (lengths, page tables) is drawn on the host with numpy's seeded
PCG64; values are N(0, 1) rounded to bf16, drawn on the host for small cases
(``values="host"``) or by torch's device generator for benchmark sizes.

Page tables follow the engines' ``Rows`` builders (crates/omni-qwen3-tts/src/
model.rs:266-303, crates/omni-personaplex/src/model.rs:473-506): sequence s
owns pages ``pages[indptr[s]:indptr[s+1]]``, a row at position p reads tokens
0..p (capped at ``context`` for the PersonaPlex ring), and the physical pages
are a random permutation of the pool.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

HEAD = 128


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def normal_bits(rng: np.random.Generator, shape) -> np.ndarray:
    return f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32))


@dataclass
class PagedCase:
    hq: int
    hk: int
    page: int
    pos: np.ndarray      # int32 [rows]
    seq: np.ndarray      # int32 [rows]
    ragged: int
    indptr: np.ndarray   # int32 [seqs + 1]
    pages: np.ndarray    # int32 [sum pages]
    num_pages: int
    context: int = 0     # 0: no cap (qwen3_attend); > 0: ring cap (lm_attend)
    scale: float = 1.0 / np.sqrt(128.0)
    qkv: np.ndarray | None = None  # uint16 [rows][(hq + 2 hk) * 128]
    kv: np.ndarray | None = None   # uint16 [num_pages * page][2 hk * 128]
    name: str = ""
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return int(self.pos.shape[0])

    def lens(self) -> np.ndarray:
        ln = self.pos.astype(np.int64) + 1
        if self.context > 0:
            ln = np.minimum(ln, self.context)
        return ln

    def kv_bytes(self) -> int:
        """Algorithmic bytes of one decode launch: K and V of every attended
        key once per K/V head, q and out once, page ids, indptr and pos."""
        ln = self.lens()
        kvb = int(ln.sum()) * self.hk * HEAD * 2 * 2
        qo = self.rows * self.hq * HEAD * 2 * 2
        idx = int(np.ceil(ln / self.page).sum()) * 4 + 4 * (len(self.indptr)) + 4 * self.rows
        return kvb + qo + idx


def paged_decode_case(rows, hq, hk, len_lo, len_hi, pool_pages=None, page=16, seed=0, context=0, values="host",
                      slack_pages=0, name=""):
    """Decode rows (one per sequence) with lengths uniform in [len_lo, len_hi].

    The pool holds ``pool_pages`` pages (default: exactly what the rows need
    plus ``slack_pages``); each sequence's pages are drawn from a random
    permutation of the pool."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(len_lo, len_hi + 1, size=rows).astype(np.int64)
    pos = (lens - 1).astype(np.int32)
    eff = np.minimum(lens, context) if context > 0 else lens
    need = ((eff + page - 1) // page).astype(np.int64)
    total = int(need.sum())
    if pool_pages is None:
        pool_pages = total + slack_pages
    if total > pool_pages:
        raise ValueError(f"pool of {pool_pages} pages cannot hold {total}")
    perm = rng.permutation(pool_pages).astype(np.int32)
    indptr = np.zeros(rows + 1, dtype=np.int32)
    indptr[1:] = np.cumsum(need)
    pages = perm[:total].copy()
    case = PagedCase(hq=hq, hk=hk, page=page, pos=pos, seq=np.arange(rows, dtype=np.int32), ragged=0,
                     indptr=indptr, pages=pages, num_pages=pool_pages, context=context, name=name)
    if values == "host":
        case.qkv = normal_bits(rng, (rows, (hq + 2 * hk) * HEAD))
        case.kv = normal_bits(rng, (pool_pages * page, 2 * hk * HEAD))
    return case


def ragged_prefill_case(nseq, hq, hk, new_lo, new_hi, cached_lo, cached_hi, page=16, seed=0, values="host",
                        slack_pages=0, name=""):
    """Chunked prefill: sequence r holds c_r cached tokens and L_r new rows at
    positions c_r .. c_r + L_r - 1, rows of a sequence contiguous (ragged=1)."""
    rng = np.random.default_rng(seed)
    new = rng.integers(new_lo, new_hi + 1, size=nseq).astype(np.int64)
    cached = rng.integers(cached_lo, cached_hi + 1, size=nseq).astype(np.int64)
    total_tok = new + cached
    need = (total_tok + page - 1) // page
    pool = int(need.sum()) + slack_pages
    perm = rng.permutation(pool).astype(np.int32)
    indptr = np.zeros(nseq + 1, dtype=np.int32)
    indptr[1:] = np.cumsum(need)
    pos = np.concatenate([np.arange(c, c + l) for c, l in zip(cached, new)]).astype(np.int32)
    seq = np.concatenate([np.full(l, s) for s, l in enumerate(new)]).astype(np.int32)
    case = PagedCase(hq=hq, hk=hk, page=page, pos=pos, seq=seq, ragged=1, indptr=indptr,
                     pages=perm[: int(need.sum())].copy(), num_pages=pool, name=name,
                     extra={"new": new, "cached": cached})
    if values == "host":
        case.qkv = normal_bits(rng, (len(pos), (hq + 2 * hk) * HEAD))
        case.kv = normal_bits(rng, (pool * page, 2 * hk * HEAD))
    return case


def prefill_flops(case: PagedCase) -> int:
    """4 * 128 flops per unmasked (q head, query, key) triple."""
    keys = case.pos.astype(np.int64) + 1
    return int(4 * HEAD * case.hq * keys.sum())


@dataclass
class DenseCase:
    hq: int
    hk: int
    q_len: int
    kv_len: int
    causal: int
    batch: int = 1
    q_stride: int = 0
    scale_log2: float = (128 ** -0.5) * 1.4426950408889634
    q: np.ndarray | None = None  # uint16 [batch][q_len][q_stride]
    k: np.ndarray | None = None  # uint16 [batch][kv_len][hk * 128]
    v: np.ndarray | None = None
    name: str = ""

    def flops(self) -> int:
        if self.causal:
            keys = np.minimum(np.arange(self.q_len, dtype=np.int64) + 1, self.kv_len).sum()
        else:
            keys = self.q_len * self.kv_len
        return int(4 * HEAD * self.hq * keys * self.batch)


def rms_unit(x: np.ndarray) -> np.ndarray:
    """Per-head RMSNorm to unit RMS over the last (head_dim) axis."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)


def dense_case(hq, hk, q_len, kv_len, causal, batch=1, seed=0, values="host", qkv_layout=True, rmsnorm=True, name=""):
    """DiT attention: q rows inside a qkv buffer (q_stride = (hq + 2 hk) * 128)
    when qkv_layout, k and v as separate [kv_len][hk][128] caches."""
    q_stride = (hq + 2 * hk) * HEAD if qkv_layout else hq * HEAD
    case = DenseCase(hq=hq, hk=hk, q_len=q_len, kv_len=kv_len, causal=causal, batch=batch, q_stride=q_stride,
                     name=name)
    if values == "host":
        rng = np.random.default_rng(seed)
        q = rng.standard_normal((batch, q_len, q_stride // HEAD, HEAD), dtype=np.float32)
        k = rng.standard_normal((batch, kv_len, hk, HEAD), dtype=np.float32)
        v = rng.standard_normal((batch, kv_len, hk, HEAD), dtype=np.float32)
        if rmsnorm:
            q, k = rms_unit(q), rms_unit(k)
        case.q = f32_to_bf16_bits(q).reshape(batch, q_len, q_stride)
        case.k = f32_to_bf16_bits(k).reshape(batch, kv_len, hk * HEAD)
        case.v = f32_to_bf16_bits(v).reshape(batch, kv_len, hk * HEAD)
    return case


# ------------------------------------------------------- the benchmark shapes
CONFIGS = {
    1: dict(kind="decode", rows=4, hq=16, hk=8, len_lo=64, len_hi=512, pool_pages=256, layers=1,
            desc="Qwen3-TTS talker decode, 16q/8kv, B=4, len U[64,512], pool 256 pages"),
    2: dict(kind="decode", rows=64, hq=16, hk=8, len_lo=200, len_hi=2400, pool_pages=16384, layers=28,
            desc="Qwen3-TTS talker decode, 16q/8kv, B=64, len U[200,2400], pool 16k pages, 28 layers"),
    3: dict(kind="decode", rows=128, hq=32, hk=32, len_lo=100, len_hi=3000, context=3000, layers=32,
            desc="PersonaPlex duplex tick, MHA 32/32, B=128, len U[100,3000], ring 3000, 32 layers"),
    4: dict(kind="prefill", nseq=8, hq=32, hk=8, new_lo=512, new_hi=4096, cached_lo=0, cached_hi=1024,
            desc="Higgs chunked prefill, 32q/8kv, B=8, new U[512,4096], cached U[0,1024], causal"),
    5: dict(kind="dit", hq=32, hk=8, q_len=4352, kv_len=4352, batch=2,
            desc="HiDream-O1 DiT, 32q/8kv, B=2, S=4352, full attention"),
}


def config_case(cfg: int, seed: int | None = None, values="host", layer=0):
    c = CONFIGS[cfg]
    seed = cfg * 1000 + layer if seed is None else seed
    if c["kind"] == "decode":
        return paged_decode_case(c["rows"], c["hq"], c["hk"], c["len_lo"], c["len_hi"], c.get("pool_pages"),
                                 seed=seed, context=c.get("context", 0), values=values, slack_pages=16,
                                 name=f"config{cfg}")
    if c["kind"] == "prefill":
        return ragged_prefill_case(c["nseq"], c["hq"], c["hk"], c["new_lo"], c["new_hi"], c["cached_lo"],
                                   c["cached_hi"], seed=seed, values=values, slack_pages=16, name=f"config{cfg}")
    return dense_case(c["hq"], c["hk"], c["q_len"], c["kv_len"], 0, batch=c["batch"], seed=seed, values=values,
                      name=f"config{cfg}")


# ------------------------------------------------------------- FP8 ring slots
def fp8_slot_bytes(heads: int) -> int:
    """PersonaPlex slot: [K heads x 128 B | V heads x 128 B | K scales f32 x heads
    | V scales f32 x heads] (crates/omni-personaplex/kernels/lm.cu:123-128)."""
    return 2 * heads * HEAD + 2 * heads * 4


def quantize_fp8_slots(kv: np.ndarray, heads: int) -> np.ndarray:
    """f32 K/V [slots][2 heads][128] -> FP8 E4M3 slots [slots][slot_bytes], each
    (slot, head) row scaled by max(amax / 448, 1e-12) as lm_rope does
    (lm.cu:148-176), rounded to nearest even by torch's float8_e4m3fn cast."""
    import torch

    slots = kv.shape[0]
    x = torch.from_numpy(np.ascontiguousarray(kv, dtype=np.float32)).view(slots, 2 * heads, HEAD)
    amax = x.abs().amax(dim=-1, keepdim=True)
    sc = torch.clamp(amax * (1.0 / 448.0), min=1e-12)
    q8 = (x / sc).to(torch.float8_e4m3fn).view(torch.uint8).reshape(slots, 2 * heads * HEAD)
    out = np.empty((slots, fp8_slot_bytes(heads)), dtype=np.uint8)
    out[:, : 2 * heads * HEAD] = q8.numpy()
    out[:, 2 * heads * HEAD:] = sc.reshape(slots, 2 * heads).numpy().astype(np.float32).view(np.uint8).reshape(
        slots, 8 * heads)
    return out


def fp8_ring_case(rows, heads, len_lo, len_hi, context, page=16, seed=0, slack_pages=0):
    """PersonaPlex decode rows over FP8 slots: a bf16-layout PagedCase whose
    `kv` is replaced by FP8 slot bytes (extra['kv_f32'] keeps the source)."""
    c = paged_decode_case(rows, heads, heads, len_lo, len_hi, page=page, seed=seed, context=context,
                          slack_pages=slack_pages)
    rng = np.random.default_rng(seed + 1)
    kv = rng.standard_normal((c.num_pages * page, 2 * heads, HEAD), dtype=np.float32)
    c.kv = quantize_fp8_slots(kv, heads)
    c.extra["fp8"] = True
    return c


def fp8_kv_bytes(case) -> int:
    """Algorithmic bytes of one FP8 decode launch: per attended key and head
    128 B of K, 128 B of V and the two f32 scales; q, out, page ids, indptr, pos."""
    ln = case.lens()
    kvb = int(ln.sum()) * case.hk * (2 * HEAD + 8)
    qo = case.rows * case.hq * HEAD * 2 * 2
    idx = int(np.ceil(ln / case.page).sum()) * 4 + 4 * len(case.indptr) + 4 * case.rows
    return kvb + qo + idx


# ------------------------------------------- rotary embedding + K/V scatter
@dataclass
class RopeCase:
    """Rows entering rope + scatter: qkv bf16 rows, norm weights, positions,
    the slot of each row, and the cache they scatter into (pre-filled with
    random bytes, so a test sees which slots were written)."""
    kind: str            # "qwen3", "dense", "hidream", "lm"
    rows: int
    hq: int
    hk: int
    qkv: np.ndarray      # uint16 [rows][ld]
    ld: int
    q_norm: np.ndarray | None
    k_norm: np.ndarray | None
    pos: np.ndarray      # int32 [rows] or [rows][3]
    slots: np.ndarray | None
    cache: dict          # name -> array (kv / k_cache, v_cache)
    eps: float = 1e-6
    theta: float = 1e6
    coef: float = 0.0
    mrope_hw: int = 20
    per: int = 0
    base: int = 0
    span: int = 0

    def bytes_moved(self) -> int:
        """Algorithmic HBM bytes of one launch: qkv read once, q written back,
        K and V (or their FP8 bytes and scales) written, weights and indices."""
        heads = self.hq + 2 * self.hk
        rd = self.rows * heads * HEAD * 2
        if self.kind == "lm":
            wr = self.rows * (self.hq * HEAD * 2 + 2 * self.hk * (HEAD + 4))
        else:
            wr = self.rows * heads * HEAD * 2
        idx = self.rows * 4 * (3 if self.kind == "hidream" else 2)
        return rd + wr + idx + (0 if self.kind == "lm" else 2 * HEAD * 2)


def rope_case(kind, rows, hq, hk, pool_slots=None, seed=0, pos_hi=4096, ld_pad=0, per=0, base=0, span=0):
    rng = np.random.default_rng(seed)
    if kind == "lm":
        hk = hq
    ld = (hq + 2 * hk) * HEAD + ld_pad
    qkv = normal_bits(rng, (rows, ld))
    q_norm = k_norm = None
    if kind != "lm":
        q_norm = f32_to_bf16_bits(1.0 + 0.2 * rng.standard_normal(HEAD, dtype=np.float32))
        k_norm = f32_to_bf16_bits(1.0 + 0.2 * rng.standard_normal(HEAD, dtype=np.float32))
    if kind == "hidream":
        pos = rng.integers(0, pos_hi, size=(rows, 3)).astype(np.int32)
    else:
        pos = rng.integers(0, pos_hi, size=rows).astype(np.int32)
    pool = pool_slots or max(2 * rows, 16)
    slots = rng.permutation(pool)[:rows].astype(np.int32)
    case = RopeCase(kind=kind, rows=rows, hq=hq, hk=hk, qkv=qkv, ld=ld, q_norm=q_norm, k_norm=k_norm, pos=pos,
                    slots=slots, cache={})
    if kind == "qwen3":
        case.cache["kv"] = normal_bits(rng, (pool, 2 * hk * HEAD))
    elif kind == "dense":
        nseq = (rows + per - 1) // per
        case.per, case.base, case.span = per, base, span
        case.pos = (base + np.arange(rows) % per).astype(np.int32)
        case.slots = None
        case.cache["kv"] = normal_bits(rng, (nseq * span, 2 * hk * HEAD))
    elif kind == "hidream":
        case.cache["k_cache"] = normal_bits(rng, (pool, hk * HEAD))
        case.cache["v_cache"] = normal_bits(rng, (pool, hk * HEAD))
    elif kind == "lm":
        case.cache["kv"] = rng.integers(0, 256, size=(pool, fp8_slot_bytes(hq)), dtype=np.uint8)
        case.coef = float(np.float32(-np.log(10000.0) * 2.0 / HEAD))
        case.theta = 10000.0
    else:
        raise ValueError(kind)
    return case
