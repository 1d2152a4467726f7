"""Independent f64 references for tests: attention by torch's
scaled_dot_product_attention in float64 (a library routine, not the oracle's
formula), with K/V rows gathered by numpy fancy indexing from the page-table
closed form slot = pages[indptr[s] + t // page] * page + t % page."""
from __future__ import annotations

import numpy as np
import torch

HEAD = 128


def bits_to_f64(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def slots_of(case, s: int, length: int) -> np.ndarray:
    t = np.arange(length)
    pg = case.pages[case.indptr[s]: case.indptr[s + 1]]
    return pg[t // case.page].astype(np.int64) * case.page + t % case.page


def paged_truth(case) -> np.ndarray:
    """f64 attention of every row of a PagedCase: [rows][hq][128]."""
    G = case.hq // case.hk
    out = np.zeros((case.rows, case.hq, HEAD))
    lens = case.lens()
    kvf = None
    for n in range(case.rows):
        s = int(case.seq[n]) if case.ragged else n
        sl = slots_of(case, s, int(lens[n]))
        rows = bits_to_f64(case.kv[sl]).reshape(len(sl), 2 * case.hk, HEAD)
        k = torch.from_numpy(rows[:, : case.hk]).permute(1, 0, 2).repeat_interleave(G, 0)  # [hq, len, D]
        v = torch.from_numpy(rows[:, case.hk:]).permute(1, 0, 2).repeat_interleave(G, 0)
        q = torch.from_numpy(bits_to_f64(case.qkv[n, : case.hq * HEAD]).reshape(case.hq, 1, HEAD))
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=float(case.scale))
        out[n] = o[:, 0].numpy()
    del kvf
    return out


def dense_truth(case, b: int = 0) -> np.ndarray:
    """f64 attention of a DenseCase batch entry: [q_len][hq][128]."""
    G = case.hq // case.hk
    q = bits_to_f64(case.q[b]).reshape(case.q_len, -1, HEAD)[:, : case.hq]
    k = bits_to_f64(case.k[b]).reshape(case.kv_len, case.hk, HEAD)
    v = bits_to_f64(case.v[b]).reshape(case.kv_len, case.hk, HEAD)
    qt = torch.from_numpy(np.ascontiguousarray(q.transpose(1, 0, 2)))
    kt = torch.from_numpy(np.ascontiguousarray(k.transpose(1, 0, 2))).repeat_interleave(G, 0)
    vt = torch.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2))).repeat_interleave(G, 0)
    mask = None
    if case.causal:
        i = torch.arange(case.q_len)[:, None]
        j = torch.arange(case.kv_len)[None, :]
        mask = j <= i
    scale = case.scale_log2 / 1.4426950408889634
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return o.permute(1, 0, 2).numpy()


def dense_weight_abs(case, b: int = 0) -> np.ndarray:
    """sum_j p_j |v_j| / sum_j p_j per output element, in f64: the scale of
    the error that rounding each p_j to bf16 (relative 2^-9) can cause."""
    G = case.hq // case.hk
    q = bits_to_f64(case.q[b]).reshape(case.q_len, -1, HEAD)[:, : case.hq]
    k = bits_to_f64(case.k[b]).reshape(case.kv_len, case.hk, HEAD)
    v = np.abs(bits_to_f64(case.v[b]).reshape(case.kv_len, case.hk, HEAD))
    qt = torch.from_numpy(np.ascontiguousarray(q.transpose(1, 0, 2)))
    kt = torch.from_numpy(np.ascontiguousarray(k.transpose(1, 0, 2))).repeat_interleave(G, 0)
    vt = torch.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2))).repeat_interleave(G, 0)
    mask = None
    if case.causal:
        mask = torch.arange(case.kv_len)[None, :] <= torch.arange(case.q_len)[:, None]
    scale = case.scale_log2 / 1.4426950408889634
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return o.permute(1, 0, 2).numpy()


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (8 significant bits)."""
    ax = np.maximum(np.abs(x), 2.0 ** -120)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def err_stats(got_bits: np.ndarray, want: np.ndarray):
    got = bits_to_f64(got_bits).reshape(want.shape)
    d = np.abs(got - want)
    return float(d.max()), float(d.mean())
