"""Writes the golden fixtures of the attention path into this directory.

Each fixture is one ``<name>.npz`` (no pickles) holding:

* the index arrays of the case (pos, seq, indptr, pages, ...) verbatim;
* how to rebuild its bf16 values: the seeds of the oracle's splitmix64 +
  Box-Muller generator (``oracle_fill_normal_bf16``) and a SHA-256 digest of
  the generated bits, so a drift in the generator is caught instead of being
  silently compared; FP8 slot bytes, which are small, are stored verbatim;
* ``truth``: attention computed in float64 (stored as float32, far below any
  tolerance used) by torch's scaled_dot_product_attention over
  the same (dequantized) K/V rows, gathered by numpy fancy indexing from the
  page-table closed form (tests/refs.py) — a library routine, independent of
  the oracle;
* in ``fixtures.json``, the SHA-256 of the CPU oracle's bf16 output when the
  fixture was made, for regression.

The cases follow the reference's test shapes at sizes a fixture can hold:
config 1 of the benchmark (Qwen3-TTS talker decode, 16q/8kv, B=4, len
U[64,512], a 256-page pool), a G=1 PersonaPlex ring case, a causal chunked
prefill with cached prefixes, a 256-token HiDream DiT case (full and causal)
and a PersonaPlex FP8 ring case.

Run from the repository root: ``python tests/golden/make_fixtures.py``.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "pega-omni_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
import refs  # noqa: E402
import workloads as W  # noqa: E402

HEAD = 128

# name -> how the case is drawn. Index data: workloads' seeded numpy draws (the
# arrays are stored, so later numpy versions do not matter); values: the
# oracle's generator with the seeds below.
SPECS = {
    "decode_config1": dict(kind="paged", rows=4, hq=16, hk=8, len_lo=64, len_hi=512, pool_pages=256, context=0,
                           index_seed=1000, q_seed=1001, kv_seed=1002),
    "ring_g1": dict(kind="paged", rows=6, hq=4, hk=4, len_lo=1, len_hi=200, pool_pages=None, context=96,
                    index_seed=3000, q_seed=3001, kv_seed=3002),
    "prefill_cached": dict(kind="prefill", nseq=3, hq=4, hk=1, new_lo=5, new_hi=60, cached_lo=0, cached_hi=40,
                           index_seed=4000, q_seed=4001, kv_seed=4002),
    "dit_256_full": dict(kind="dense", hq=4, hk=1, q_len=256, kv_len=256, causal=0, q_seed=5001, k_seed=5002,
                         v_seed=5003),
    "dit_256_causal": dict(kind="dense", hq=2, hk=1, q_len=256, kv_len=256, causal=1, q_seed=5011, k_seed=5012,
                           v_seed=5013),
    "fp8_ring": dict(kind="fp8", rows=5, heads=2, len_lo=1, len_hi=90, context=60, index_seed=6000, q_seed=6001,
                     kv_seed=6002),
}


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gen(n: int, seed: int) -> np.ndarray:
    return oracle.normal_bf16(int(n), int(seed))


def build(name: str, arrays: dict | None = None):
    """The case of fixture `name`. With `arrays` (a loaded fixture) the index
    arrays come from it; otherwise they are drawn from the spec."""
    sp = SPECS[name]
    k = sp["kind"]
    if k in ("paged", "prefill"):
        if arrays is None:
            if k == "paged":
                c = W.paged_decode_case(sp["rows"], sp["hq"], sp["hk"], sp["len_lo"], sp["len_hi"], sp["pool_pages"],
                                        seed=sp["index_seed"], context=sp["context"], values=None, slack_pages=4)
            else:
                c = W.ragged_prefill_case(sp["nseq"], sp["hq"], sp["hk"], sp["new_lo"], sp["new_hi"], sp["cached_lo"],
                                          sp["cached_hi"], seed=sp["index_seed"], values=None, slack_pages=4)
        else:
            c = W.PagedCase(hq=sp["hq"], hk=sp["hk"], page=int(arrays["page"]), pos=arrays["pos"], seq=arrays["seq"],
                            ragged=int(arrays["ragged"]), indptr=arrays["indptr"], pages=arrays["pages"],
                            num_pages=int(arrays["num_pages"]), context=int(arrays["context"]), name=name)
        c.qkv = gen(c.rows * (c.hq + 2 * c.hk) * HEAD, sp["q_seed"]).reshape(c.rows, -1)
        c.kv = gen(c.num_pages * c.page * 2 * c.hk * HEAD, sp["kv_seed"]).reshape(c.num_pages * c.page, -1)
        return c
    if k == "dense":
        c = W.dense_case(sp["hq"], sp["hk"], sp["q_len"], sp["kv_len"], sp["causal"], values=None, name=name)
        c.q = gen(c.q_len * c.q_stride, sp["q_seed"]).reshape(1, c.q_len, c.q_stride)
        c.k = gen(c.kv_len * c.hk * HEAD, sp["k_seed"]).reshape(1, c.kv_len, -1)
        c.v = gen(c.kv_len * c.hk * HEAD, sp["v_seed"]).reshape(1, c.kv_len, -1)
        return c
    if k == "fp8":
        h = sp["heads"]
        if arrays is None:
            c = W.paged_decode_case(sp["rows"], h, h, sp["len_lo"], sp["len_hi"], seed=sp["index_seed"],
                                    context=sp["context"], values=None, slack_pages=2)
            kvf = refs.bits_to_f64(gen(c.num_pages * c.page * 2 * h * HEAD, sp["kv_seed"])).astype(np.float32)
            c.kv = W.quantize_fp8_slots(kvf.reshape(-1, 2 * h, HEAD), h)
        else:
            c = W.PagedCase(hq=h, hk=h, page=int(arrays["page"]), pos=arrays["pos"], seq=arrays["seq"],
                            ragged=int(arrays["ragged"]), indptr=arrays["indptr"], pages=arrays["pages"],
                            num_pages=int(arrays["num_pages"]), context=int(arrays["context"]), name=name)
            c.kv = arrays["kv_fp8"]
        c.qkv = gen(c.rows * 3 * h * HEAD, sp["q_seed"]).reshape(c.rows, -1)
        return c
    raise ValueError(k)


def fp8_truth(c) -> np.ndarray:
    """float64 SDPA over the dequantized FP8 slots (value * per-(slot, head) scale)."""
    import torch

    h = c.hq
    body = 2 * h * HEAD
    vals = torch.from_numpy(np.ascontiguousarray(c.kv[:, :body])).view(torch.float8_e4m3fn).double().numpy()
    scales = np.ascontiguousarray(c.kv[:, body:]).view(np.float32).astype(np.float64)
    deq = vals.reshape(-1, 2 * h, HEAD) * scales[:, :, None]
    out = np.zeros((c.rows, h, HEAD))
    lens = c.lens()
    for n in range(c.rows):
        sl = refs.slots_of(c, n, int(lens[n]))
        rows = deq[sl]
        kk = torch.from_numpy(rows[:, :h]).permute(1, 0, 2)
        vv = torch.from_numpy(rows[:, h:]).permute(1, 0, 2)
        q = torch.from_numpy(refs.bits_to_f64(c.qkv[n, : h * HEAD]).reshape(h, 1, HEAD))
        out[n] = torch.nn.functional.scaled_dot_product_attention(q, kk, vv, scale=float(c.scale))[:, 0].numpy()
    return out


def truth_and_oracle(name: str, c):
    k = SPECS[name]["kind"]
    if k in ("paged", "prefill"):
        t = refs.paged_truth(c)
        o = oracle.paged_attend(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale,
                                context=c.context, nthreads=8)
        return t, o
    if k == "dense":
        t = refs.dense_truth(c, 0)
        o = oracle.dense_attend(c.q[0], c.k[0], c.v[0], c.q_len, c.kv_len, c.q_stride, c.hq, c.hk, c.causal,
                                c.scale_log2, nthreads=8)
        return t, o
    t = fp8_truth(c)
    o = oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, c.hq, c.scale,
                             c.context, nthreads=8)
    return t, o


def value_digests(name: str, c) -> dict:
    k = SPECS[name]["kind"]
    if k == "dense":
        return {"q": digest(c.q), "k": digest(c.k), "v": digest(c.v)}
    if k == "fp8":
        return {"qkv": digest(c.qkv), "kv_fp8": digest(c.kv)}
    return {"qkv": digest(c.qkv), "kv": digest(c.kv)}


def main():
    index = {}
    for name, sp in SPECS.items():
        c = build(name)
        truth, ob = truth_and_oracle(name, c)
        arrays = {"truth": truth.astype(np.float32)}
        if sp["kind"] != "dense":
            arrays.update(pos=c.pos, seq=c.seq, indptr=c.indptr, pages=c.pages, page=np.int32(c.page),
                          ragged=np.int32(c.ragged), num_pages=np.int32(c.num_pages), context=np.int32(c.context))
        if sp["kind"] == "fp8":
            arrays["kv_fp8"] = c.kv
        np.savez(os.path.join(HERE, f"{name}.npz"), **arrays)
        index[name] = dict(spec=sp, digests=value_digests(name, c), oracle_digest=digest(ob),
                           tolerance={"max_abs": 2e-2, "mean_abs": 2e-3})
        print(f"{name}: truth {truth.shape}, oracle max-abs {np.abs(refs.bits_to_f64(ob).reshape(truth.shape) - truth).max():.3e}")
    with open(os.path.join(HERE, "fixtures.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
