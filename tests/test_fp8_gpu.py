"""lm_attend over FP8 E4M3 slots (PersonaPlex's cache format) on the GPU
against the CPU oracle."""
import numpy as np
import pytest
import torch

import omni_attn as oa
import workloads as W
from gpu_util import assert_close, dev_bits, dev_i32, host_bits

pytestmark = pytest.mark.gpu


def run_fp8(c, heads, chunk=0, max_len=None, group_heads=0):
    max_len = max_len or int(c.lens().max())
    plan = oa.decode_plan(c.rows, heads, heads, c.page, max_len, chunk)
    plan.group_heads = group_heads
    out = torch.zeros(c.rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    kv = torch.from_numpy(np.ascontiguousarray(c.kv)).cuda()
    oa.lm_attend_fp8(dev_bits(c.qkv), kv, dev_i32(c.pos), dev_i32(c.seq), c.ragged, dev_i32(c.indptr),
                     dev_i32(c.pages), c.page, out, heads, c.scale, c.context or (1 << 30), plan,
                     oa.workspace_for(plan))
    torch.cuda.synchronize()
    return host_bits(out)


def run_fp8_planned(c, heads, max_len):
    """omni_lm_attend_fp8 on the FP8 plan (omni_attn_decode_plan_init_fp8's
    split size, the launch's own heads per workgroup)."""
    plan = oa.decode_plan_fp8(c.rows, heads, c.page, max_len)
    out = torch.zeros(c.rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    kv = torch.from_numpy(np.ascontiguousarray(c.kv)).cuda()
    oa.lm_attend_fp8(dev_bits(c.qkv), kv, dev_i32(c.pos), dev_i32(c.seq), c.ragged, dev_i32(c.indptr),
                     dev_i32(c.pages), c.page, out, heads, c.scale, c.context or (1 << 30), plan,
                     oa.workspace_for(plan))
    torch.cuda.synchronize()
    return host_bits(out), plan.chunk


def oracle_fp8(oracle, c, heads):
    return oracle.lm_attend_fp8(c.qkv, c.kv, c.pos, c.seq, c.ragged, c.indptr, c.pages, c.page, heads, c.scale,
                                c.context, nthreads=16)


@pytest.mark.parametrize("heads,lo,hi,ctx,chunk", [
    (4, 1, 300, 0, 128), (8, 100, 1500, 700, 256), (32, 100, 3000, 3000, 0), (2, 1, 1, 0, 0),
])
def test_fp8_parity(oracle, heads, lo, hi, ctx, chunk):
    c = W.fp8_ring_case(7, heads, lo, hi, ctx, seed=heads * 7 + lo, slack_pages=3)
    assert_close(run_fp8(c, heads, chunk), oracle_fp8(oracle, c, heads), what=f"fp8 h{heads} ctx{ctx}")


def device_fp8_case(rows, heads, seed):
    """PersonaPlex rows (lengths U[100, 3000], ring 3000) with FP8 slots
    quantized on the device, per (slot, head) scale max(amax / 448, 1e-12)."""
    c = W.paged_decode_case(rows, heads, heads, 100, 3000, seed=seed, context=3000, values=None, slack_pages=3)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    slots = c.num_pages * c.page
    kv8 = torch.empty(slots, W.fp8_slot_bytes(heads), dtype=torch.uint8, device="cuda")
    for s0 in range(0, slots, 8192):
        s1 = min(slots, s0 + 8192)
        x = torch.randn(s1 - s0, 2 * heads, 128, device="cuda", generator=gen)
        sc = torch.clamp(x.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
        kv8[s0:s1, : 2 * heads * 128] = (x / sc).to(torch.float8_e4m3fn).view(torch.uint8).reshape(s1 - s0, -1)
        kv8[s0:s1, 2 * heads * 128:] = sc.reshape(s1 - s0, -1).contiguous().view(torch.uint8)
    qkv = torch.randn(c.rows, 3 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    c.qkv = host_bits(qkv)
    c.kv = kv8.cpu().numpy()
    return c


@pytest.mark.parametrize("rows,chunk", [(32, 256), (64, 384)])
def test_fp8_plan_buckets(oracle, rows, chunk):
    """The FP8 plan's split size at smaller PersonaPlex buckets (32 heads):
    256 and 384 keys, with the launch's pick of 4 and 8 heads per workgroup
    (the 128-session tick's 768 runs in test_fp8_full_config3), against the
    oracle."""
    c = device_fp8_case(rows, 32, seed=rows + 5)
    got, picked = run_fp8_planned(c, 32, 3000)
    assert picked == chunk
    assert_close(got, oracle_fp8(oracle, c, 32), what=f"fp8 plan rows {rows}")


@pytest.mark.parametrize("gh", [1, 2, 4, 8])
@pytest.mark.parametrize("page", [1, 4, 16, 3, 12, 24])
def test_fp8_heads_per_workgroup(oracle, gh, page):
    """Every heads-per-workgroup layout (1/2/4/8 heads, 8/4/2/1 keys per load),
    over pages smaller and larger than a load's key group, powers of two
    (shift and mask) and not (multiply-high division; 12 and 24 share one
    page id per load group where the group divides them)."""
    c = W.fp8_ring_case(5, 8, 1, 700, 500, page=page, seed=gh * 31 + page, slack_pages=2)
    assert_close(run_fp8(c, 8, 128, group_heads=gh), oracle_fp8(oracle, c, 8), what=f"fp8 gh{gh} page{page}")


def test_fp8_single_key_exact(oracle):
    c = W.fp8_ring_case(5, 4, 1, 1, 0, seed=9)
    assert np.array_equal(run_fp8(c, 4), oracle_fp8(oracle, c, 4))


def test_fp8_every_code_decodes_like_ocp_e4m3(oracle):
    """All 254 finite E4M3 codes through the kernel: one key whose K row is
    zero (every score 0) and whose V row holds the codes, scale 1: the output
    row is the decoded V row, exactly."""
    heads = 1
    c = W.fp8_ring_case(2, heads, 1, 1, 0, seed=11)
    codes = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)
    for n, part in enumerate((codes[:128], codes[128:])):
        slot = int(c.pages[c.indptr[n]]) * 16
        row = np.zeros(128, np.uint8)
        row[: len(part)] = part
        c.kv[slot, :128] = 0
        c.kv[slot, 128:256] = row
        c.kv[slot, 256:264] = np.array([1.0, 1.0], np.float32).view(np.uint8)
    got = run_fp8(c, heads)
    want = oracle_fp8(oracle, c, heads)
    assert np.array_equal(got, want)


def test_fp8_full_config3(oracle):
    """Config 3's shape (128 sessions, 32 heads, lengths U[100,3000], ring
    3000) with FP8 slots quantized on the device."""
    c = W.config_case(3, values=None)
    heads = 32
    gen = torch.Generator(device="cuda").manual_seed(3)
    slots = c.num_pages * c.page
    kv8 = torch.empty(slots, W.fp8_slot_bytes(heads), dtype=torch.uint8, device="cuda")
    for s0 in range(0, slots, 8192):
        s1 = min(slots, s0 + 8192)
        x = torch.randn(s1 - s0, 2 * heads, 128, device="cuda", generator=gen)
        sc = torch.clamp(x.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
        kv8[s0:s1, : 2 * heads * 128] = (x / sc).to(torch.float8_e4m3fn).view(torch.uint8).reshape(s1 - s0, -1)
        kv8[s0:s1, 2 * heads * 128:] = sc.reshape(s1 - s0, -1).contiguous().view(torch.uint8)
    qkv = torch.randn(c.rows, 3 * heads * 128, device="cuda", generator=gen).to(torch.bfloat16)
    c.qkv = host_bits(qkv)
    c.kv = kv8.cpu().numpy()
    plan = oa.decode_plan_fp8(c.rows, heads, 16, 3000)  # the FP8 plan's split size (768 keys here)
    out = torch.zeros(c.rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    oa.lm_attend_fp8(qkv, kv8, dev_i32(c.pos), dev_i32(c.seq), 0, dev_i32(c.indptr), dev_i32(c.pages), 16, out,
                     heads, c.scale, 3000, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    assert_close(host_bits(out), oracle_fp8(oracle, c, heads), what="fp8 config3")


@pytest.mark.parametrize("gh", [0, 1, 4])
def test_fp8_ragged_prefill_rows(oracle, gh):
    """PersonaPlex's prefill rows (ragged = 1): several rows of one session at
    consecutive positions, each seeing min(pos + 1, context) ring slots."""
    heads = 8
    p = W.ragged_prefill_case(3, heads, heads, 5, 200, 0, 120, seed=11 + gh, values=None, slack_pages=2)
    rng = np.random.default_rng(gh)
    kvf = rng.standard_normal((p.num_pages * 16, 2 * heads, 128), dtype=np.float32)
    p.kv = W.quantize_fp8_slots(kvf, heads)
    p.qkv = W.normal_bits(rng, (p.rows, 3 * heads * 128))
    p.context = 150
    plan = oa.decode_plan(p.rows, heads, heads, 16, 150, 128)
    plan.group_heads = gh
    out = torch.zeros(p.rows, heads * 128, dtype=torch.bfloat16, device="cuda")
    oa.lm_attend_fp8(dev_bits(p.qkv), torch.from_numpy(p.kv).cuda(), dev_i32(p.pos), dev_i32(p.seq), 1,
                     dev_i32(p.indptr), dev_i32(p.pages), 16, out, heads, p.scale, p.context, plan,
                     oa.workspace_for(plan))
    torch.cuda.synchronize()
    want = oracle.lm_attend_fp8(p.qkv, p.kv, p.pos, p.seq, 1, p.indptr, p.pages, 16, heads, p.scale, p.context,
                                nthreads=16)
    assert_close(host_bits(out), want, what=f"fp8 ragged gh{gh}")


def test_fp8_reads_no_slot_past_the_keys(oracle):
    """FP8 slots no row reads are all-ones bytes (E4M3 NaN values, NaN scales)."""
    from gpu_util import seen_slots

    c = W.fp8_ring_case(9, 8, 1, 400, 300, seed=32, slack_pages=4)
    seen = seen_slots(c)
    assert (~seen).any()
    c.kv = c.kv.copy()
    c.kv[~seen] = 0xFF
    assert_close(run_fp8(c, 8, 128), oracle_fp8(oracle, c, 8), what="fp8 NaN past the keys")
