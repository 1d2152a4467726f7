"""Benchmark of the attention hot path on one MI355X.

Headline (`value`): paged MHA decode attention of a 128-session PersonaPlex
duplex tick (config 3: 32 q / 32 kv heads, head_dim 128, bf16, lengths
U[100,3000] under a 3000-slot ring, page 16, random page tables), one step =
the 32 layers of a tick, in algorithmic HBM GB/s. Also reported: the Qwen3-TTS
28-layer decode loop (config 2), the Higgs chunked prefill (config 4) and the
HiDream DiT attention (config 5) in TFLOP/s, each as a fraction of its roofline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only 3]
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "pega-omni_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
# HBM bytes per lm_attend dispatch of the config-3 decode, from rocprofv3
# FETCH_SIZE + WRITE_SIZE runs scaled by a 1 GiB copy's counts (the summary
# and commands are in profiles/decode_config3_traffic.md). Re-measure when
# the decode kernel changes.
DECODE_CFG3_TRAFFIC_BYTES = 3.272e+09
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def fp8_pool(slots, heads, gen):
    """A device pool of FP8 E4M3 slots holding N(0,1) K/V, quantized per
    (slot, head) with scale max(amax / 448, 1e-12) as lm_rope writes them."""
    import torch

    import workloads as W

    kv8 = torch.empty(slots, W.fp8_slot_bytes(heads), dtype=torch.uint8, device="cuda")
    body = 2 * heads * 128
    for s0 in range(0, slots, 16384):
        s1 = min(slots, s0 + 16384)
        x = torch.randn(s1 - s0, 2 * heads, 128, device="cuda", generator=gen)
        sc = torch.clamp(x.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
        kv8[s0:s1, :body] = (x / sc).to(torch.float8_e4m3fn).view(torch.uint8).reshape(s1 - s0, body)
        kv8[s0:s1, body:] = sc.reshape(s1 - s0, 2 * heads).contiguous().view(torch.uint8)
    return kv8


class DecodeBench:
    """Device-resident decode workload: `pools` distinct K/V pools (each far
    larger than the 256 MB last-level cache) cycled over the layers, each
    layer with its own random page table."""

    def __init__(self, cfg, pools, seed=0, chunk=0, fp8=False, group_heads=0):
        import numpy as np
        import torch

        import omni_attn as oa
        import workloads as W

        self.cfg = cfg
        c = W.CONFIGS[cfg]
        self.layers = c["layers"]
        self.lm = cfg == 3
        self.fp8 = fp8
        assert not fp8 or self.lm, "FP8 slots are PersonaPlex's (config 3) cache format"
        self.cases, self.dev = [], []
        gen = torch.Generator(device="cuda").manual_seed(seed + cfg)
        for layer in range(self.layers):
            case = W.config_case(cfg, values=None, layer=layer)
            self.cases.append(case)
        self.pools = []
        pool_pages = max(cs.num_pages for cs in self.cases)
        for i in range(min(pools, self.layers)):
            case = self.cases[i]
            if fp8:
                kv = fp8_pool(pool_pages * case.page, case.hk, gen)
            else:
                kv = torch.empty(pool_pages * case.page, 2 * case.hk * 128, dtype=torch.bfloat16, device="cuda")
                kv.normal_(generator=gen)
            self.pools.append(kv)
        for layer, case in enumerate(self.cases):
            kv = self.pools[layer % len(self.pools)]
            pages = case.pages  # every pool holds the largest layer's page count
            qkv = torch.empty(case.rows, (case.hq + 2 * case.hk) * 128, dtype=torch.bfloat16, device="cuda")
            qkv.normal_(generator=gen)
            i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()
            self.dev.append(dict(qkv=qkv, kv=kv, pos=i32(case.pos), seq=i32(case.seq), indptr=i32(case.indptr),
                                 pages=i32(pages),
                                 out=torch.empty(case.rows, case.hq * 128, dtype=torch.bfloat16, device="cuda")))
        c0 = self.cases[0]
        max_len = c["len_hi"] if not self.lm else c["context"]
        self.plan = (oa.decode_plan_fp8(c0.rows, c0.hq, c0.page, max_len, chunk) if fp8 else
                     oa.decode_plan(c0.rows, c0.hq, c0.hk, c0.page, max_len, chunk))
        self.plan.group_heads = group_heads
        self.ws = oa.workspace_for(self.plan)
        self.bytes_per_layer = [W.fp8_kv_bytes(cs) if fp8 else cs.kv_bytes() for cs in self.cases]
        self.oa = oa
        self.mode = "attend"
        if fp8:
            # lm_rope's slot for each row: the lease's slot of ring index pos % context.
            for case, d in zip(self.cases, self.dev):
                sl = []
                for n, p in enumerate(case.pos):
                    t = int(p) % case.context
                    sl.append(case.pages[case.indptr[n] + t // case.page] * case.page + t % case.page)
                d["slots"] = torch.from_numpy(np.asarray(sl, dtype=np.int32)).cuda()
            self.coef = float(np.float32(-np.log(10000.0) * 2.0 / 128))
        if cfg == 2:
            # The step's rotary inputs: each row's new key goes to the slot the
            # page table gives its position (what the engines' Rows builder makes).
            for case, d in zip(self.cases, self.dev):
                sl = [case.pages[case.indptr[n] + p // case.page] * case.page + p % case.page
                      for n, p in enumerate(case.pos)]
                d["slots"] = torch.from_numpy(np.asarray(sl, dtype=np.int32)).cuda()
            self.q_norm = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)
            self.k_norm = (1 + 0.1 * torch.randn(128, device="cuda", generator=gen)).to(torch.bfloat16)

    def layer(self, i, stream):
        d, c = self.dev[i], self.cases[i]
        if self.fp8 and self.mode == "fused":
            self.oa.lm_rope_attend_fp8(d["qkv"], d["pos"], d["slots"], d["kv"], d["indptr"], d["pages"], c.page,
                                       d["out"], c.hq, self.coef, c.scale, c.context, self.plan, self.ws, stream)
        elif self.fp8:
            if self.mode == "rope_attend":
                self.oa.lm_rope(d["qkv"], d["pos"], d["slots"], d["kv"], c.rows, c.hq, self.coef, stream)
            self.oa.lm_attend_fp8(d["qkv"], d["kv"], d["pos"], d["seq"], 0, d["indptr"], d["pages"], c.page,
                                  d["out"], c.hq, c.scale, c.context, self.plan, self.ws, stream)
        elif self.lm:
            self.oa.lm_attend(d["qkv"], d["kv"], d["pos"], d["seq"], 0, d["indptr"], d["pages"], c.page, d["out"],
                              c.hq, c.scale, c.context, self.plan, self.ws, stream)
        elif self.mode == "fused":
            self.oa.qwen3_rope_attend(d["qkv"], self.q_norm, self.k_norm, d["pos"], d["slots"], d["kv"], d["indptr"],
                                      d["pages"], c.page, d["out"], c.hq, c.hk, 1e-6, 1e6, c.scale, self.plan, self.ws,
                                      stream)
        else:
            if self.mode == "rope_attend":
                self.oa.qwen3_rope(d["qkv"], self.q_norm, self.k_norm, d["pos"], d["slots"], d["kv"], c.rows, c.hq,
                                   c.hk, 1e-6, 1e6, stream)
            self.oa.qwen3_attend(d["qkv"], d["kv"], d["pos"], d["seq"], 0, d["indptr"], d["pages"], c.page,
                                 d["out"], c.hq, c.hk, c.scale, self.plan, self.ws, stream)

    def step(self, stream, events=None):
        for i in range(self.layers):
            if events is not None:
                events[i][0].record(stream)
            self.layer(i, stream)
            if events is not None:
                events[i][1].record(stream)


def time_steps(run_step, steps, warmup, stream, per_launch=None):
    """Time exactly `steps` steps after `warmup`; returns ms per step and,
    when per_launch=(n, run_step_with_events), the mean per-launch ms from HIP
    events recorded on `stream` around each launch in the timed region."""
    import torch

    for _ in range(warmup):
        run_step(stream, None)
    torch.cuda.synchronize()
    n = per_launch or 0
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
           for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for k in range(steps):
        run_step(stream, evs[k] if n else None)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    launch_ms = None
    if n:
        tot = sum(a.elapsed_time(b) for row in evs for (a, b) in row)
        launch_ms = tot / (steps * n)
    return ms, launch_ms


def graph_launch_us(call, steps, warmup, stream, n=20):
    """One small launch as a replayed HIP graph of `n` back-to-back launches:
    device time per launch without the host's launch path between them (the
    engines replay their decode step as a graph)."""
    def step(s, ev):
        for _ in range(n):
            call(s)

    return graph_step_ms(step, steps, warmup, stream) * 1e3 / n


def graph_step_ms(run_step, steps, warmup, stream):
    """The step captured once into a HIP graph and replayed, as the engines run
    decode (one graph per batch bucket): ms per replay over `steps` replays
    after `warmup`."""
    import torch

    run_step(stream, None)  # plan state and allocations exist before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run_step(stream, None)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(steps):
            g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    del g
    return start.elapsed_time(end) / steps


def cpu_decode_baseline(cfg=3, rows=None, min_seconds=10.0, threads=None):
    """The oracle (a C port of the reference math) timed on this host's cores on
    one layer of the decode workload: the first `rows` sessions (all of them
    by default), their pages compacted into a pool of exactly that size,
    repeated for at least `min_seconds`. Returns (GB/s, seconds per rep,
    threads, text)."""
    import numpy as np

    import oracle
    import workloads as W

    threads = threads or min(16, os.cpu_count() or 1)
    c = W.config_case(cfg, values=None)
    rows = rows or c.rows
    c.pos, c.seq = c.pos[:rows].copy(), c.seq[:rows].copy()
    used = int(c.indptr[rows])
    c.indptr = c.indptr[: rows + 1].copy()
    rng = np.random.default_rng(7)
    c.pages = rng.permutation(used).astype(np.int32)
    c.num_pages = used

    c.qkv = _timing_values(rng, rows * (c.hq + 2 * c.hk) * 128).reshape(rows, -1)
    c.kv = _timing_values(rng, used * c.page * 2 * c.hk * 128).reshape(used * c.page, -1)
    args = (c.qkv, c.kv, c.pos, c.seq, 0, c.indptr, c.pages, c.page, c.hq, c.hk, c.scale)
    sec, reps, el = _repeat(lambda: oracle.paged_attend(*args, context=c.context, nthreads=threads), min_seconds)
    which = "all" if rows == W.CONFIGS[cfg]["rows"] else f"first {rows} of"
    text = (f"config{cfg}: {which} {W.CONFIGS[cfg]['rows']} sessions of one layer, pages compacted to a "
            f"{used}-page pool "
            f"({c.kv_bytes() / 1e9:.3f} GB algorithmic), {reps} reps over {el:.1f} s")
    return c.kv_bytes() / sec / 1e9, sec, threads, text


def _timing_values(rng, n):
    """Normal bf16 bit patterns in +-[1/8, 2) with random sign and mantissa:
    inputs for CPU timing only (their outputs are not checked). Up to 2^25
    values are drawn and repeated to length n."""
    import numpy as np

    block = (rng.integers(0, 1 << 16, min(n, 1 << 25), dtype=np.uint16) & np.uint16(0x81FF)) | np.uint16(0x3E00)
    return block if block.size == n else np.resize(block, n)


def _repeat(fn, min_seconds):
    fn()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_seconds:
            return el / reps, reps, el


def cpu_prefill_baseline(rows=96, min_seconds=3.0, threads=None):
    """The oracle on a bounded sample of config 4: `rows` seeded random rows
    of the B = 8 draw (each with its own causal key count, over its
    sequence's paged keys). GFLOP/s at 4 * 128 flops per (q head, query, key)."""
    import numpy as np

    import oracle
    import workloads as W

    threads = threads or min(16, os.cpu_count() or 1)
    c = W.config_case(4, values=None)
    rng = np.random.default_rng(44)
    idx = np.sort(rng.choice(c.rows, rows, replace=False))
    pos, seq = c.pos[idx].copy(), c.seq[idx].copy()
    qkv = _timing_values(rng, rows * (c.hq + 2 * c.hk) * 128).reshape(rows, -1)
    kv = _timing_values(rng, c.num_pages * c.page * 2 * c.hk * 128).reshape(c.num_pages * c.page, -1)
    sec, reps, el = _repeat(lambda: oracle.paged_attend(qkv, kv, pos, seq, 1, c.indptr, c.pages, c.page, c.hq, c.hk,
                                                        c.scale, nthreads=threads), min_seconds)
    fl = int(4 * 128 * c.hq * (pos.astype(np.int64) + 1).sum())
    return dict(value=round(fl / sec / 1e9, 3), unit="GFLOP/s", cores=threads, kind="port",
                sample=f"config4: {rows} seeded random rows of the {c.rows}-row draw ({fl / 1e9:.2f} GFLOP), "
                       f"{reps} reps over {el:.1f} s", seconds_per_sample=round(sec, 4))


def cpu_dit_baseline(q_rows=48, min_seconds=3.0, threads=None):
    """The oracle on a bounded sample of config 5: the first `q_rows` query
    positions (all 32 heads) of one CFG half over all 4352 keys."""
    import numpy as np

    import oracle
    import workloads as W

    threads = threads or min(16, os.cpu_count() or 1)
    cfg = W.CONFIGS[5]
    hq, hk, kv_len = cfg["hq"], cfg["hk"], cfg["kv_len"]
    rng = np.random.default_rng(55)
    q_stride = (hq + 2 * hk) * 128
    q = _timing_values(rng, q_rows * q_stride).reshape(q_rows, q_stride)
    k = _timing_values(rng, kv_len * hk * 128).reshape(kv_len, -1)
    v = _timing_values(rng, kv_len * hk * 128).reshape(kv_len, -1)
    sl2 = (128 ** -0.5) * 1.4426950408889634
    sec, reps, el = _repeat(lambda: oracle.dense_attend(q, k, v, q_rows, kv_len, q_stride, hq, hk, 0, sl2,
                                                        nthreads=threads), min_seconds)
    fl = 4 * 128 * hq * q_rows * kv_len
    return dict(value=round(fl / sec / 1e9, 3), unit="GFLOP/s", cores=threads, kind="port",
                sample=f"config5: the first {q_rows} of 4352 query positions of one CFG half, all {hq} heads, "
                       f"over 4352 keys ({fl / 1e9:.2f} GFLOP), {reps} reps over {el:.1f} s",
                seconds_per_sample=round(sec, 4))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(head_cpu):
    """The CPU path (the oracle, a C port of the reference math) on every
    BASELINE config: one full layer of configs 1 and 2, config 3's (the
    headline's cpu_baseline, also a full layer), and bounded samples of
    configs 4 and 5."""
    out = {"cpu_model": cpu_model(), "host_cpus": os.cpu_count()}
    for cfg, rows, secs in ((1, 4, 3.0), (2, 64, 3.0)):
        v, sec, thr, text = cpu_decode_baseline(cfg, rows=rows, min_seconds=secs)
        out[f"config{cfg}"] = dict(value=round(v, 3), unit="GB/s", cores=thr, kind="port", sample=text,
                                   seconds_per_sample=round(sec, 4))
    out["config3"] = head_cpu
    out["config4"] = cpu_prefill_baseline()
    out["config5"] = cpu_dit_baseline()
    return out


def prefill_bench(stream, steps, warmup, exact_p=False):
    """Config 4: one ragged causal prefill launch over paged K/V per step
    (exact_p: the plan's hi + lo P, qwen3_attend's f32-P numerics)."""
    import numpy as np
    import torch

    import omni_attn as oa
    import workloads as W

    c = W.config_case(4, values=None)
    gen = torch.Generator(device="cuda").manual_seed(4)
    qkv = torch.empty(c.rows, (c.hq + 2 * c.hk) * 128, dtype=torch.bfloat16, device="cuda").normal_(generator=gen)
    kv = torch.empty(c.num_pages * c.page, 2 * c.hk * 128, dtype=torch.bfloat16, device="cuda").normal_(generator=gen)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()
    pos, seq, indptr, pages = i32(c.pos), i32(c.seq), i32(c.indptr), i32(c.pages)
    out = torch.empty(c.rows, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    pf = oa.prefill_plan(c.rows, c.hq, c.hk, c.page, c.seq, c.pos, exact_p=exact_p)

    def step(s, ev):
        if ev is not None:
            ev[0][0].record(s)
        oa.prefill_run(pf, qkv, kv, pos, seq, indptr, pages, out, c.scale, s)
        if ev is not None:
            ev[0][1].record(s)

    # MFMA legs warm for at least 20 calls: the clock ramps over the first ~100 ms of MFMA load.
    ms, launch_ms = time_steps(step, steps, max(warmup, 20), stream, per_launch=1)
    fl = W.prefill_flops(c)
    name = "config4: " + W.CONFIGS[4]["desc"] + (", P as bf16 hi + lo (f32-P numerics)" if exact_p else "")
    return dict(workload=name, rows=c.rows, flops=fl, ms_per_step=round(ms, 4),
                tflops=round(fl / (ms * 1e-3) / 1e12, 2), launch_us=round(launch_ms * 1e3, 2),
                frac=round(fl / (launch_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))


def dit_bench(stream, steps, warmup, hk=8, split=True, shape=None):
    """Config 5: the HiDream CFG pair's full attention, one call per step
    (the tiled kernel, plus the tail-split combine when `split`). `shape` =
    (q_len, kv_len, batch) replaces config 5's sizes."""
    import numpy as np
    import torch

    import omni_attn as oa
    import workloads as W

    cfg = W.CONFIGS[5]
    q_len, kv_len, batch = shape or (cfg["q_len"], cfg["kv_len"], cfg["batch"])
    c = W.dense_case(cfg["hq"], hk, q_len, kv_len, 0, batch=batch, values=None)
    gen = torch.Generator(device="cuda").manual_seed(5)

    def rms(x):
        x = x.view(*x.shape[:-1], -1, 128)
        return (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)).view(*x.shape[:-2], -1)

    q = rms(torch.randn(c.batch, c.q_len, c.q_stride, device="cuda", generator=gen)).to(torch.bfloat16)
    k = rms(torch.randn(c.batch, c.kv_len, hk * 128, device="cuda", generator=gen)).to(torch.bfloat16)
    v = torch.randn(c.batch, c.kv_len, hk * 128, device="cuda", generator=gen).to(torch.bfloat16)
    out = torch.empty(c.batch, c.q_len, c.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = torch.tensor([c.kv_len], dtype=torch.int32, device="cuda")

    ws = oa.hidream_workspace() if split else None

    def step(s, ev):
        if ev is not None:
            ev[0][0].record(s)
        oa.hidream_attend_ws(q, k, v, out, c.q_len, kvl, c.q_stride, 0, c.scale_log2, c.hq, hk, c.batch,
                             c.q_len * c.q_stride, c.kv_len * hk * 128, c.q_len * c.hq * 128, ws, s)
        if ev is not None:
            ev[0][1].record(s)

    ms, launch_ms = time_steps(step, steps, max(warmup, 20), stream, per_launch=1)
    fl = c.flops()
    name = f"config5: {W.CONFIGS[5]['desc']} (hk={hk})" if shape is None else \
        f"hidream_attend, {q_len} queries x {kv_len} keys, batch {batch}, {c.hq}q/{hk}kv heads, non-causal"
    return dict(workload=name, split=split, flops=fl, ms_per_step=round(ms, 4),
                tflops=round(fl / (ms * 1e-3) / 1e12, 2), launch_us=round(launch_ms * 1e3, 2),
                frac=round(fl / (launch_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4))


# The reference's one published attention-kernel time on this path
# (docs/hidream-o1.md:79, hardware :62): hidream_attend timed alone at 4097
# queries over 4130 keys, 32 q / 8 kv heads, head 128, non-causal, on an
# sm_89 card under a 300 W cap (FlashInfer FA2 at the same shape: 1.66 ms).
PUBLISHED_HIDREAM = dict(q_len=4097, kv_len=4130, ms=1.73, flashinfer_ms=1.66,
                         hardware="sm_89, 48 GB, CUDA 13.1, 300 W cap", source="docs/hidream-o1.md:79")


def published_shape_bench(stream, steps, warmup):
    """hidream_attend at the shape of the reference's published kernel time,
    with and without a workspace (the tail split against row halves), beside
    that published time. A different card: the ratio is reported, not graded."""
    p = PUBLISHED_HIDREAM
    shape = (p["q_len"], p["kv_len"], 1)
    res = {"published": p}
    for key, split in (("workspace", True), ("no_workspace", False)):
        r = dit_bench(stream, steps, warmup, hk=8, split=split, shape=shape)
        r["vs_published_ms"] = round(p["ms"] / r["ms_per_step"], 2)
        res[key] = r
    return res


def rope_bench(stream, steps, warmup, graph=True):
    """Rotary + K/V scatter, one launch per step, at the engines' shapes:
    config 2 decode rows (qwen3_rope), a config-3 tick (lm_rope into FP8
    slots), config 4's prefill rows (qwen3_rope) and both HiDream CFG rows
    (hidream_qk_rope). Bytes: qkv read, q and K/V written, weights, indices.
    `graph_us`: the same launch timed as a replayed HIP graph of 20 launches (not with --no-graph)."""
    import numpy as np
    import torch

    import omni_attn as oa
    import workloads as W

    gen = torch.Generator(device="cuda").manual_seed(7)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()
    res = {}

    def run(name, rows, hq, hk, call, bytes_):
        def step(s, ev):
            if ev is not None:
                ev[0][0].record(s)
            call(s)
            if ev is not None:
                ev[0][1].record(s)

        ms, launch_ms = time_steps(step, steps * 5, warmup, stream, per_launch=1)
        g_us = graph_launch_us(call, steps, warmup, stream) if graph else float("nan")
        res[name] = dict(rows=rows, heads=f"{hq}q/{hk}kv", bytes=bytes_, launch_us=round(launch_ms * 1e3, 2),
                         gbs=round(bytes_ / (launch_ms * 1e-3) / 1e9, 1),
                         frac=round(bytes_ / (launch_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         graph_us=round(g_us, 2), graph_gbs=round(bytes_ / (g_us * 1e-6) / 1e9, 1))

    rng = np.random.default_rng(7)
    w = torch.ones(128, dtype=torch.bfloat16, device="cuda")
    for name, rows, hq, hk, pool in (("qwen3_rope config2", 64, 16, 8, 16384 * 16),
                                     ("qwen3_rope config4", 25499, 32, 8, 26000)):
        qkv = torch.randn(rows, (hq + 2 * hk) * 128, device="cuda", generator=gen).to(torch.bfloat16)
        kv = torch.empty(pool, 2 * hk * 128, dtype=torch.bfloat16, device="cuda")
        pos, slots = i32(rng.integers(0, 3000, rows)), i32(rng.permutation(pool)[:rows])
        c = W.RopeCase("qwen3", rows, hq, hk, None, 0, None, None, None, None, {})
        run(name, rows, hq, hk, lambda s, qkv=qkv, kv=kv, pos=pos, slots=slots, rows=rows, hq=hq, hk=hk:
            oa.qwen3_rope(qkv, w, w, pos, slots, kv, rows, hq, hk, 1e-6, 1e6, s), c.bytes_moved())
        del qkv, kv
    rows, heads, pool = 128, 32, 128 * 3000
    qkv = torch.randn(rows, 3 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    kv8 = torch.empty(pool, W.fp8_slot_bytes(heads), dtype=torch.uint8, device="cuda")
    pos, slots = i32(rng.integers(0, 3000, rows)), i32(rng.permutation(pool)[:rows])
    coef = float(np.float32(-np.log(10000.0) * 2.0 / 128))
    c = W.RopeCase("lm", rows, heads, heads, None, 0, None, None, None, None, {})
    run("lm_rope config3", rows, heads, heads, lambda s: oa.lm_rope(qkv, pos, slots, kv8, rows, heads, coef, s),
        c.bytes_moved())
    del qkv, kv8
    rows, hq, hk = 2 * 4352, 32, 8
    ld = (hq + 2 * hk) * 128
    qkv = torch.randn(rows, ld, device="cuda", generator=gen).to(torch.bfloat16)
    kc = torch.empty(rows, hk * 128, dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    p3, slots = i32(rng.integers(0, 4352, (rows, 3))), i32(np.arange(rows))
    c = W.RopeCase("hidream", rows, hq, hk, None, 0, None, None, None, None, {})
    run("hidream_qk_rope config5", rows, hq, hk,
        lambda s: oa.hidream_qk_rope(qkv, ld, w, w, p3, slots, kc, vc, rows, hq, hk, 20, 1e-6, 5e6, s),
        c.bytes_moved())
    return res


def short_bench(stream, steps, warmup, graph=True):
    """The small attentions at engine shapes, one launch per step: the code
    predictor's qwen3_attend_dense (64 sessions at position 15 of a 16-slot
    workspace), Mimi's ring attention (128 sessions x 2 rows, 8 heads, full
    250-slot rings) and the rotary + ring write before it, a 3000-slot prefix
    copy over FP8 slots, the codec decoder's fused attention (64 sessions, 16
    heads, a full 72-frame ring) and the depformer's last step (128 sessions,
    16 heads, step 7). Bytes: K/V rows read once per (row, head), q, out, writes.
    `graph_us`: the same launch timed as a replayed HIP graph of 20 launches (not with --no-graph)."""
    import numpy as np
    import torch

    import omni_attn as oa
    import workloads as W

    gen = torch.Generator(device="cuda").manual_seed(8)
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()
    bf = lambda *shape: torch.randn(*shape, device="cuda", generator=gen).to(torch.bfloat16)
    res = {}

    def run(name, call, bytes_):
        def step(s, ev):
            if ev is not None:
                ev[0][0].record(s)
            call(s)
            if ev is not None:
                ev[0][1].record(s)

        ms, launch_ms = time_steps(step, steps * 5, warmup, stream, per_launch=1)
        g_us = graph_launch_us(call, steps, warmup, stream) if graph else float("nan")
        res[name] = dict(bytes=bytes_, launch_us=round(launch_ms * 1e3, 2),
                         gbs=round(bytes_ / (launch_ms * 1e-3) / 1e9, 1),
                         graph_us=round(g_us, 2), graph_gbs=round(bytes_ / (g_us * 1e-6) / 1e9, 1))

    # code predictor: hq16/hk8, one row per session at position 15
    rows, hq, hk = 64, 16, 8
    qkv, kv = bf(rows, (hq + 2 * hk) * 128), bf(rows * 16, 2 * hk * 128)
    out = torch.empty(rows, hq * 128, dtype=torch.bfloat16, device="cuda")
    plan = oa.decode_plan(rows, hq, hk, 1, 16)
    ws = oa.workspace_for(plan)
    run("qwen3_attend_dense code predictor", lambda s: oa.qwen3_attend_dense(qkv, kv, 1, 15, 16, out, hq, hk, 0.088,
                                                                             plan, ws, s),
        rows * 16 * hk * 512 + rows * hq * 512)
    # Mimi: 8 heads of 64, T = 2, context 250, full rings
    sess, T, heads, ctx = 128, 2, 8, 250
    stride = ctx * 2 * heads * 64 * 2
    state = torch.empty(sess * stride, dtype=torch.uint8, device="cuda")
    state.view(torch.bfloat16).copy_(bf(sess * stride // 2))
    qkv, out = bf(sess * T, 3 * heads * 64), torch.empty(sess * T, heads * 64, dtype=torch.bfloat16, device="cuda")
    pos, lines = i32(np.full(sess, 500)), i32(np.arange(sess))
    run("mimi_attend", lambda s: oa.mimi_attend(qkv, pos, lines, state, out, sess * T, T, heads, 0.125, ctx, stride,
                                                s),
        sess * T * heads * (ctx * 256 + 256))
    # the step before it: Mimi's rotary of q and k, k and v into the ring slots
    coef = float(np.float32(-np.log(10000.0) * 2.0 / 64))
    run("mimi_rope_kv", lambda s: oa.mimi_rope_kv(qkv, pos, lines, state, sess * T, T, heads, coef, ctx, stride, s),
        sess * T * heads * 128 * 6)
    # PersonaPlex prefix reuse: 3000 FP8 slots of one layer copied to new leases
    toks = 3000
    kvc = torch.empty(2 * toks, W.fp8_slot_bytes(32), dtype=torch.uint8, device="cuda")
    src, dst = i32(np.arange(toks)), i32(toks + np.random.default_rng(0).permutation(toks))
    run("lm_copy_kv 3000 FP8 slots", lambda s: oa.lm_copy_kv(kvc, src, dst, toks, W.fp8_slot_bytes(32), s),
        2 * toks * W.fp8_slot_bytes(32))
    # codec decoder: 16 heads of 64, full 72-frame rings
    sess, heads = 64, 16
    width = heads * 64
    stride = 2 * 72 * width * 2
    ring = torch.empty(sess * stride, dtype=torch.uint8, device="cuda")
    ring.view(torch.bfloat16).copy_(bf(sess * stride // 2))
    qkv, out = bf(sess, 3 * width), torch.empty(sess, width, dtype=torch.bfloat16, device="cuda")
    pos = i32(np.full(sess, 1000))
    run("codec_attention", lambda s: oa.codec_attention(qkv, pos, lines[:sess], ring, out, sess, stride, heads, 1e4, s),
        sess * heads * (72 * 256 + 3 * 128 + 128))
    # depformer: 16 heads of 64, step 7
    sess, heads = 128, 16
    width = heads * 64
    qkv, wsd = bf(sess, 3 * width), bf(sess, 8 * 2 * width)
    out = torch.empty(sess, width, dtype=torch.bfloat16, device="cuda")
    run("lm_dep_kv_attend step 7", lambda s: oa.lm_dep_kv_attend(qkv, wsd, 7, out, sess, heads, 0.125, s),
        sess * heads * (8 * 256 + 4 * 128))
    return res


PEAKS_SRC = os.path.join(ROOT, "bench_peaks.hip")
PEAKS_LIB = os.path.join(ROOT, "bench_peaks.so")


def build_peaks():
    """Compile the benchmark's peak probes (bench_peaks.hip) for gfx950 into
    bench_peaks.so beside this file. They are measurement code, kept out of
    the attention library's build."""
    import subprocess

    sys.path.insert(0, os.path.join(ROOT, "pega-omni_amd"))
    import build as hip_build

    tmp = PEAKS_LIB + ".tmp"
    r = subprocess.run([hip_build.HIPCC, *hip_build.FLAGS, "-x", "hip", "-shared", PEAKS_SRC, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PEAKS_SRC}:\n{r.stderr}")
    os.replace(tmp, PEAKS_LIB)
    return PEAKS_LIB


def measure_peaks(stream):
    """Measured ceilings on this GPU (bench_peaks.so): bf16 MFMA TFLOP/s
    (4 independent 32x32x16 chains per wave) on smooth operands and on random
    ones (the clock drops as more operand bits toggle; random data is what
    attention feeds the MFMAs), v_exp_f32 and v_fma_f32 lane
    rates, and a streaming 16-byte nontemporal read of 4 GiB."""
    import ctypes

    import torch

    if not os.path.exists(PEAKS_LIB):
        log("[bench] bench_peaks.so is not built: building it")
        build_peaks()
    L = ctypes.CDLL(PEAKS_LIB)
    P, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    L.omni_peaks_mfma.argtypes = [P, i32, i32, i32, P]
    L.omni_peaks_valu.argtypes = [P, i32, i32, i32, P]
    L.omni_peaks_read.argtypes = [P, i64, P, i32, P]
    L.omni_peaks_lds.argtypes = [P, i32, i32, P]
    sink = torch.zeros(1024, dtype=torch.float32, device="cuda")
    sp = ctypes.c_void_p(sink.data_ptr())
    st = ctypes.c_void_p(stream.cuda_stream)

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        best = None
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            torch.cuda.synchronize()
            t = a.elapsed_time(b) * 1e-3
            best = t if best is None else min(best, t)
        return best

    blocks, iters = 2048, 2000
    mfma_flops = blocks * 4 * iters * 16 * 32 * 32 * 16 * 2
    mfma = mfma_flops / timed(lambda: L.omni_peaks_mfma(sp, blocks, iters, 0, st)) / 1e12
    mfma_rnd = mfma_flops / timed(lambda: L.omni_peaks_mfma(sp, blocks, iters, 1, st)) / 1e12
    vi = 4096
    t_exp = timed(lambda: L.omni_peaks_valu(sp, blocks, vi, 1, st))
    t_fma = timed(lambda: L.omni_peaks_valu(sp, blocks, vi, 0, st))
    lanes = blocks * 256 * vi * 8
    li = 4096
    t_lds = timed(lambda: L.omni_peaks_lds(sp, blocks, li, st))
    lds_bytes = blocks * 256 * li * 8 * 16
    buf = torch.empty(4 << 30, dtype=torch.uint8, device="cuda")
    # The best of three grid sizes (nontemporal 16-byte loads, grid-stride).
    t_rd = min(timed(lambda: L.omni_peaks_read(ctypes.c_void_p(buf.data_ptr()), buf.numel(), sp, nb, st))
               for nb in (1024, 2048, 4096))
    del buf
    return dict(mfma_bf16_tflops=round(mfma, 1), mfma_bf16_random_tflops=round(mfma_rnd, 1), exp_glane_ops=round(lanes / t_exp / 1e9, 1),
                fma_glane_ops=round(lanes / t_fma / 1e9, 1),
                lds_read_tbs=round(lds_bytes / t_lds / 1e12, 2), hbm_read_gbs=round((4 << 30) / t_rd / 1e9, 1))


def copy_calibration(mb):
    """A plain device copy of `mb` MiB, 5 times: the known-size kernel that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    a = torch.empty(mb << 20, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_mib": mb, "bytes_read": mb << 20, "bytes_written": mb << 20}))


def summarize_profile(dirs, kernels, last, flops=None, cus=256, xcds=8, nbytes=None):
    """Summarise rocprofv3 CSV output (one directory per pass) for the last
    `last` dispatches of each kernel whose name contains one of `kernels`
    (the timed calls of a bench.py run: its warmup calls come first). Prints a
    markdown table: the mean kernel-trace duration of each kernel and of one
    call (their sum), every counter of the first kernel averaged per dispatch,
    and the derived figures. GRBM_GUI_ACTIVE counts on each of the `xcds` XCDs
    and is summed over them; SQ_VALU_MFMA_BUSY_CYCLES is summed over the
    cus x 4 SIMDs."""
    import csv
    import glob

    durs = {k: [] for k in kernels}
    counters = {}
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
            allrows = list(csv.DictReader(open(path)))
            for k in kernels:
                rows = sorted((r for r in allrows if k in r["Kernel_Name"]), key=lambda r: int(r["Start_Timestamp"]))
                durs[k] += [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3 for r in rows[-last:]]
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            per = {}
            for r in csv.DictReader(open(path)):
                if kernels[0] in r["Kernel_Name"]:
                    per.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
            for disp in sorted(per)[-last:]:
                for name, v in per[disp].items():
                    counters.setdefault(name, []).append(v)
    avg = {k: sum(v) / len(v) for k, v in counters.items()}
    lines = [f"| quantity | value (mean over the last {last} dispatches of each kernel per run) |", "|---|---|"]
    call_us = 0.0
    for k in kernels:
        if durs[k]:
            us = sum(durs[k]) / len(durs[k])
            call_us += us
            lines.append(f"| kernel-trace duration of `{k}` | {us:.2f} us ({len(durs[k])} dispatches) |")
    if len(kernels) > 1 and call_us:
        lines.append(f"| one call (sum of the above) | {call_us:.2f} us |")
    if nbytes and call_us:
        lines.append(f"| GB/s = algorithmic bytes / one call | {nbytes / (call_us * 1e-6) / 1e9:.1f} |")
        lines.append(f"| fraction of the 8000 GB/s HBM peak | {nbytes / (call_us * 1e-6) / 1e9 / 8000:.4f} |")
    if flops and call_us:
        lines.append(f"| TFLOP/s = algorithmic flops / one call | {flops / (call_us * 1e-6) / 1e12:.1f} |")
        lines.append(f"| fraction of the 2500 TFLOP/s bf16 dense peak | {flops / (call_us * 1e-6) / 1e12 / 2500:.4f} |")
    for k in sorted(avg):
        lines.append(f"| {k} | {avg[k]:.6g} |")
    k0 = durs[kernels[0]]
    us0 = sum(k0) / len(k0) if k0 else None
    gui = avg.get("GRBM_GUI_ACTIVE")
    if gui and us0:
        cyc = gui / xcds
        lines.append(f"| clock = GRBM_GUI_ACTIVE / {xcds} XCDs / duration | {cyc / us0 / 1e3:.3f} GHz |")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
            lines.append(f"| MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {xcds} x {cus} CUs x 4 SIMDs) | "
                         f"{100 * avg['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * cus * 4):.1f} % |")
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in avg:
            lines.append(f"| MFMA and VALU co-executing = SQ_VALU_MFMA_COEXEC_CYCLES / (same) | "
                         f"{100 * avg['SQ_VALU_MFMA_COEXEC_CYCLES'] / (cyc * cus * 4):.1f} % |")
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in avg:
            tf = avg["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512 / (us0 * 1e-6) / 1e12
            peak = cus * 4 * 1024 * cyc / us0 * 1e-6  # 1024 bf16 flops per SIMD per clock
            lines.append(f"| bf16 MFMA TFLOP/s executed (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 / duration) | {tf:.1f} |")
            lines.append(f"| bf16 dense peak at the measured clock (1024 flops / SIMD / clock) | {peak:.1f} TFLOP/s |")
    if "SQ_WAVE_CYCLES" in avg:
        for k in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS"):
            if k in avg:
                lines.append(f"| {k} / SQ_WAVE_CYCLES | {100 * avg[k] / avg['SQ_WAVE_CYCLES']:.1f} % |")
    if "SQ_INSTS_MFMA" in avg and "SQ_INSTS_VALU" in avg:
        lines.append(f"| VALU instructions per MFMA (SQ_INSTS_VALU / SQ_INSTS_MFMA, MFMA included) | "
                     f"{avg['SQ_INSTS_VALU'] / avg['SQ_INSTS_MFMA']:.2f} |")
    print("\n".join(lines))


def headline_bench(args, stream):
    """Config 3, the headline: one step = the 32 lm_attend calls of a tick."""
    import torch

    cfg = 3
    log(f"[bench] decode config {cfg}: building workload")
    b = DecodeBench(cfg, args.pools, chunk=args.chunk, group_heads=args.group_heads)
    log(f"[bench] decode config {cfg}: plan chunk={b.plan.chunk} splits={b.plan.splits}; timing")
    ms, launch_ms = time_steps(lambda s, e: b.step(s, e), args.steps, args.warmup, stream, per_launch=b.layers)
    total_bytes = sum(b.bytes_per_layer)
    log(f"[bench] config {cfg}: {ms:.3f} ms/step, {total_bytes / (ms * 1e-3) / 1e9:.0f} GB/s, "
        f"launch {launch_ms*1e3:.1f} us")
    g = None if args.no_graph else graph_step_ms(lambda s, e: b.step(s, e), args.steps, args.warmup, stream)
    if g is not None:
        log(f"[bench] config {cfg} as a replayed HIP graph: {g:.3f} ms/step")
    c = b.cases[0]
    head = dict(ms=ms, launch_ms=launch_ms, total_bytes=total_bytes, layers=b.layers, sessions=c.rows,
                heads=f"{c.hq}q/{c.hk}kv", kv_pools=len(b.pools), chunk=b.plan.chunk, graph_ms=g)
    del b
    torch.cuda.empty_cache()
    return head


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pools", type=int, default=4)
    ap.add_argument("--chunk", type=int, default=0)
    ap.add_argument("--group-heads", type=int, default=0,
                    help="K/V heads per decode workgroup (the plan's group_heads; 0 = the plan's pick)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="skip the HIP-graph replays (profiling runs: the trace then ends on the timed calls)")
    ap.add_argument("--only", type=int, default=0, help="time only this config (2, 3, 4 or 5; 6 = config 3 over FP8 slots; 7 = rotary + scatter; 8 = dense and head-64 attentions; 9 = the rotary + attention steps of config 2 and config 3 over FP8 slots, separate and fused; 10 = hidream_attend at the reference's published shape)")
    ap.add_argument("--calib-copy-mib", type=int, default=0, help="run the copy calibration kernel and exit")
    ap.add_argument("--peaks", action="store_true", help="print the measured peaks and exit")
    ap.add_argument("--build-peaks", action="store_true", help="compile bench_peaks.hip into bench_peaks.so and exit")
    ap.add_argument("--summarize", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 CSV output directories (with --kernel, --last) and exit")
    ap.add_argument("--kernel", nargs="+", default=["tiled_attn"],
                    help="kernel name substrings of one call (--summarize); counters are read for the first")
    ap.add_argument("--last", type=int, default=10)
    ap.add_argument("--flops", type=float, default=None, help="algorithmic flops per call (--summarize)")
    ap.add_argument("--bytes", type=float, default=None, help="algorithmic bytes per call (--summarize)")
    args = ap.parse_args()
    if args.build_peaks:
        print(f"built {build_peaks()}")
        return
    if args.summarize:
        summarize_profile(args.summarize, args.kernel, args.last, args.flops, nbytes=args.bytes)
        return
    if args.calib_copy_mib:
        copy_calibration(args.calib_copy_mib)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    stream = torch.cuda.Stream()
    # The headline leg runs first, on a GPU not yet heated by the MFMA legs.
    head = headline_bench(args, stream) if args.only in (0, 3) and not args.peaks else None
    extra = {}
    if args.peaks or args.only == 0:
        extra["measured_peaks"] = measure_peaks(stream)
        log(f"[bench] measured peaks: {extra['measured_peaks']}")
        if args.peaks:
            print(json.dumps(extra["measured_peaks"]), flush=True)
            return

    if args.only in (0, 4):
        log("[bench] config 4 prefill")
        extra["config4"] = prefill_bench(stream, args.steps, args.warmup)
        log(f"[bench] {extra['config4']}")
        extra["config4_exact_p"] = prefill_bench(stream, args.steps, args.warmup, exact_p=True)
        log(f"[bench] {extra['config4_exact_p']}")
    if args.only in (0, 5):
        log("[bench] config 5 DiT")
        extra["config5"] = dit_bench(stream, args.steps, args.warmup)
        log(f"[bench] {extra['config5']}")
        if args.only == 0:
            extra["config5_mha"] = dit_bench(stream, args.steps, args.warmup, hk=32)
            # the reference's signature (no workspace): the last round's tiles run as row halves
            extra["config5_no_workspace"] = dit_bench(stream, args.steps, args.warmup, split=False)
    if args.only in (0, 10):
        extra["hidream_published_shape"] = published_shape_bench(stream, args.steps, args.warmup)
    # The MFMA legs against the ceiling random operands reach on this card (the
    # clock under full MFMA load falls as operand bits toggle), beside `frac`
    # against the published 2.5 PFLOP/s.
    rnd = extra.get("measured_peaks", {}).get("mfma_bf16_random_tflops")
    for key in ("config4", "config4_exact_p", "config5", "config5_mha", "config5_no_workspace"):
        if rnd and key in extra:
            extra[key]["frac_of_measured_random_peak"] = round(extra[key]["frac"] * BF16_PEAK_TFLOPS / rnd, 4)
    if args.only in (0, 2):
        log("[bench] config 2 decode")
        b2 = DecodeBench(2, args.pools, chunk=args.chunk, group_heads=args.group_heads)
        ms2, l2 = time_steps(lambda s, e: b2.step(s, e), args.steps, args.warmup, stream, per_launch=b2.layers)
        g2 = float("nan") if args.no_graph else graph_step_ms(lambda s, e: b2.step(s, e), args.steps, args.warmup,
                                                               stream)
        tb = sum(b2.bytes_per_layer)
        extra["config2"] = dict(workload="config2: " + __import__("workloads").CONFIGS[2]["desc"],
                                ms_per_step=round(ms2, 4), gbs=round(tb / (ms2 * 1e-3) / 1e9, 1),
                                launch_us=round(l2 * 1e3, 2), chunk=b2.plan.chunk,
                                frac=round(tb / b2.layers / (l2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                graph_ms_per_step=round(g2, 4), graph_gbs=round(tb / (g2 * 1e-3) / 1e9, 1),
                                graph_frac=round(tb / (g2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        log(f"[bench] {extra['config2']}")
        del b2
        torch.cuda.empty_cache()
    if args.only in (0, 9):
        # The whole per-layer step of the Qwen3-TTS talker's attention: rotary
        # + K/V scatter then attention as two launches (the reference's
        # sequence), against the fused launch, and attention alone.
        log("[bench] config 2 step: rotary + attention, separate and fused")
        b2 = DecodeBench(2, args.pools, chunk=args.chunk)
        step = {}
        for mode in ("attend", "rope_attend", "fused"):
            b2.mode = mode
            ms, _ = time_steps(lambda s, e: b2.step(s, e), args.steps, args.warmup, stream)
            gms = float("nan") if args.no_graph else graph_step_ms(lambda s, e: b2.step(s, e), args.steps,
                                                                   args.warmup, stream)
            step[mode] = (ms * 1e3 / b2.layers, gms * 1e3 / b2.layers)
        extra["config2_step"] = dict(
            workload="config2 per-layer step: qwen3_rope + qwen3_attend (two launches) against omni_qwen3_rope_attend",
            separate_us_per_layer=round(step["rope_attend"][0], 2), fused_us_per_layer=round(step["fused"][0], 2),
            attend_only_us_per_layer=round(step["attend"][0], 2),
            separate_graph_us_per_layer=round(step["rope_attend"][1], 2),
            fused_graph_us_per_layer=round(step["fused"][1], 2),
            attend_only_graph_us_per_layer=round(step["attend"][1], 2),
            # attention alone timed per step (no events between calls), as a fraction of 8 TB/s
            attend_only_frac=round(sum(b2.bytes_per_layer) / b2.layers / (step["attend"][0] * 1e-6) / 1e9
                                   / HBM_PEAK_GBS, 4))
        log(f"[bench] {extra['config2_step']}")
        del b2
        torch.cuda.empty_cache()
        # The same for PersonaPlex's tick over its FP8 cache: lm_rope then
        # lm_attend (two launches) against the fused launch.
        log("[bench] config 3 FP8 step: rotary + quantized scatter + attention, separate and fused")
        b8 = DecodeBench(3, args.pools, chunk=args.chunk, fp8=True)
        step = {}
        for mode in ("attend", "rope_attend", "fused"):
            b8.mode = mode
            ms, _ = time_steps(lambda s, e: b8.step(s, e), args.steps, args.warmup, stream)
            gms = float("nan") if args.no_graph else graph_step_ms(lambda s, e: b8.step(s, e), args.steps,
                                                                   args.warmup, stream)
            step[mode] = (ms * 1e3 / b8.layers, gms * 1e3 / b8.layers)
        extra["config3_fp8_step"] = dict(
            workload="config3 over FP8 slots, per-layer step: lm_rope + lm_attend (two launches) against "
                     "omni_lm_rope_attend_fp8",
            separate_us_per_layer=round(step["rope_attend"][0], 2), fused_us_per_layer=round(step["fused"][0], 2),
            attend_only_us_per_layer=round(step["attend"][0], 2),
            separate_graph_us_per_layer=round(step["rope_attend"][1], 2),
            fused_graph_us_per_layer=round(step["fused"][1], 2),
            attend_only_graph_us_per_layer=round(step["attend"][1], 2))
        log(f"[bench] {extra['config3_fp8_step']}")
        del b8
        torch.cuda.empty_cache()
    if args.only in (0, 6):
        log("[bench] config 3 decode over FP8 E4M3 slots")
        b8 = DecodeBench(3, args.pools, chunk=args.chunk, fp8=True)
        ms8, l8 = time_steps(lambda s, e: b8.step(s, e), args.steps, args.warmup, stream, per_launch=b8.layers)
        g8 = float("nan") if args.no_graph else graph_step_ms(lambda s, e: b8.step(s, e), args.steps, args.warmup,
                                                               stream)
        tb = sum(b8.bytes_per_layer)
        extra["config3_fp8"] = dict(workload="config3 over PersonaPlex FP8 E4M3 slots (8448 B per slot)",
                                    ms_per_step=round(ms8, 4), gbs=round(tb / (ms8 * 1e-3) / 1e9, 1),
                                    launch_us=round(l8 * 1e3, 2), chunk=b8.plan.chunk,
                                    frac=round(tb / b8.layers / (l8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    graph_ms_per_step=round(g8, 4), graph_gbs=round(tb / (g8 * 1e-3) / 1e9, 1))
        log(f"[bench] {extra['config3_fp8']}")
        del b8
        torch.cuda.empty_cache()
    if args.only in (0, 7):
        log("[bench] rotary + K/V scatter")
        extra["rope"] = rope_bench(stream, args.steps, args.warmup, graph=not args.no_graph)
        log(f"[bench] {extra['rope']}")
        torch.cuda.empty_cache()
    if args.only in (0, 8):
        log("[bench] dense and head-64 attentions")
        extra["short"] = short_bench(stream, args.steps, args.warmup, graph=not args.no_graph)
        log(f"[bench] {extra['short']}")
        torch.cuda.empty_cache()
    if args.only in (4, 5, 2, 6, 7, 8, 9, 10):
        print(json.dumps({"extra": extra}), flush=True)
        return

    cfg = 3
    if head is None:
        head = headline_bench(args, stream)
    ms, launch_ms, total_bytes, layers = head["ms"], head["launch_ms"], head["total_bytes"], head["layers"]
    gbs = total_bytes / (ms * 1e-3) / 1e9
    per_launch_bytes = total_bytes / layers
    achieved = per_launch_bytes / (launch_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle port)")
        v, sec, thr, sample = cpu_decode_baseline(cfg)
        log(f"[bench] cpu: {v:.2f} GB/s on {thr} threads")
        cpu = {"value": round(v, 3), "unit": "GB/s", "cores": thr, "kind": "port", "sample": sample,
               "seconds_per_sample": round(sec, 4)}
        extra["cpu_baseline"] = cpu_baselines(cpu)
        log(f"[bench] cpu, every config: {extra['cpu_baseline']}")

    out = {
        "metric": "decode attn HBM GB/s (% peak) @128 duplex sessions",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"config{cfg}: " + __import__("workloads").CONFIGS[cfg]["desc"],
            "layers_per_step": layers,
            "sessions": head["sessions"],
            "heads": head["heads"],
            "kv_pools": head["kv_pools"],
            "chunk": head["chunk"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": DECODE_CFG3_TRAFFIC_BYTES if cfg == 3 else None,
            "kernel": "decode_split_mh<1, 2, true, false> + decode_combine (one lm_attend call)",
            "bytes_per_launch": per_launch_bytes,
            "launch_us": round(launch_ms * 1e3, 2),
        },
        "cpu_baseline": cpu,
        "extra": dict(extra, config3_graph=None if head["graph_ms"] is None else dict(
            ms_per_step=round(head["graph_ms"], 4), gbs=round(total_bytes / (head["graph_ms"] * 1e-3) / 1e9, 1),
            note="the same step captured once as a HIP graph and replayed (the engines' per-bucket graphs)")),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
