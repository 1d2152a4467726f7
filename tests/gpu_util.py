"""Helpers for the GPU tests: upload numpy cases to device tensors, run the
HIP path through the C ABI, compare with the oracle to the stated tolerance."""
from __future__ import annotations

import numpy as np
import torch

import omni_attn as oa

# Tolerance the attention path is held to against the reference math
# (bf16 in, f32 accumulate): max-abs 2e-2 and mean-abs 2e-3.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def dev_bits(a: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bits -> contiguous bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def dev_i32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def host_bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def bits_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def compare(got_bits: np.ndarray, want_bits: np.ndarray):
    g, w = bits_f32(got_bits).astype(np.float64), bits_f32(want_bits).astype(np.float64)
    assert np.all(np.isfinite(g)), "non-finite output"
    d = np.abs(g - w)
    return float(d.max()), float(d.mean())


def assert_close(got_bits, want_bits, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    mx, mn = compare(got_bits, want_bits)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3g} mean-abs {mn:.3g}"
    return mx, mn


class DevPaged:
    """A PagedCase on the device."""

    def __init__(self, case):
        self.c = case
        self.qkv = dev_bits(case.qkv)
        self.kv = dev_bits(case.kv)
        self.pos = dev_i32(case.pos)
        self.seq = dev_i32(case.seq)
        self.indptr = dev_i32(case.indptr)
        self.pages = dev_i32(case.pages)
        self.out = torch.zeros(case.rows, case.hq * 128, dtype=torch.bfloat16, device="cuda")

    def decode(self, chunk=0, max_len=None, lm=False, group_heads=0):
        c = self.c
        if max_len is None:
            max_len = int(c.lens().max())
        plan = oa.decode_plan(c.rows, c.hq, c.hk, c.page, max_len, chunk)
        plan.group_heads = group_heads
        ws = oa.workspace_for(plan)
        self.out.zero_()
        if lm:
            oa.lm_attend(self.qkv, self.kv, self.pos, self.seq, c.ragged, self.indptr, self.pages, c.page, self.out,
                         c.hq, c.scale, c.context, plan, ws)
        else:
            oa.qwen3_attend(self.qkv, self.kv, self.pos, self.seq, c.ragged, self.indptr, self.pages, c.page,
                            self.out, c.hq, c.hk, c.scale, plan, ws)
        torch.cuda.synchronize()
        return host_bits(self.out)


def seen_slots(c):
    """Mask of the cache slots some row of a paged case reads (keys 0..len-1 of
    its sequence through the page table)."""
    seen = np.zeros(c.kv.shape[0], bool)
    lens = c.lens()
    for n in range(c.rows):
        s = int(c.seq[n]) if c.ragged else n
        keys = np.arange(int(lens[n]))
        pg = c.pages[c.indptr[s]:c.indptr[s + 1]]
        seen[pg[keys // c.page] * c.page + keys % c.page] = True
    return seen
