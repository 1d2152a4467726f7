"""The HIP path against the committed golden fixtures' float64 truth, through
the C ABI: decode (qwen3_attend, lm_attend ring), ragged prefill (MFMA prefill
and the decode kernels' ragged rows), HiDream DiT (full and causal) and the
FP8 ring. Tolerance: max-abs 2e-2, mean-abs 2e-3 (stored with each fixture)."""
import numpy as np
import pytest
import torch

import golden_cases as GC
import omni_attn as oa
import refs
from gpu_util import DevPaged, dev_bits, dev_i32, host_bits

pytestmark = pytest.mark.gpu


def check(name, got_bits, truth, meta):
    got = refs.bits_to_f64(got_bits).reshape(truth.shape)
    assert np.all(np.isfinite(got)), f"{name}: non-finite output"
    err = np.abs(got - truth)
    tol = meta["tolerance"]
    assert err.max() <= tol["max_abs"] and err.mean() <= tol["mean_abs"], \
        f"{name}: max-abs {err.max():.3g} mean-abs {err.mean():.3g}"


@pytest.mark.parametrize("name,chunk", [("decode_config1", 0), ("decode_config1", 128), ("ring_g1", 0),
                                        ("ring_g1", 128)])
def test_decode_fixture(name, chunk):
    case, truth, meta = GC.load(name)
    d = DevPaged(case)
    got = d.decode(chunk=chunk, lm=case.context > 0)
    check(name, got, truth, meta)


def test_prefill_fixture_mfma_and_decode():
    case, truth, meta = GC.load("prefill_cached")
    d = DevPaged(case)
    pf = oa.prefill_plan(case.rows, case.hq, case.hk, case.page, case.seq, case.pos)
    out = torch.zeros(case.rows, case.hq * 128, dtype=torch.bfloat16, device="cuda")
    oa.prefill_run(pf, d.qkv, d.kv, d.pos, d.seq, d.indptr, d.pages, out, case.scale)
    torch.cuda.synchronize()
    check("prefill_cached (MFMA)", host_bits(out), truth, meta)
    check("prefill_cached (decode kernels)", d.decode(), truth, meta)


@pytest.mark.parametrize("name", ["dit_256_full", "dit_256_causal"])
def test_dit_fixture(name):
    case, truth, meta = GC.load(name)
    q, k, v = dev_bits(case.q[0]), dev_bits(case.k[0]), dev_bits(case.v[0])
    out = torch.zeros(case.q_len, case.hq * 128, dtype=torch.bfloat16, device="cuda")
    kvl = dev_i32(np.array([case.kv_len]))
    oa.hidream_attend(q, k, v, out, case.q_len, kvl, case.q_stride, case.causal, case.scale_log2, case.hq, case.hk)
    torch.cuda.synchronize()
    check(name, host_bits(out), truth, meta)


@pytest.mark.parametrize("group_heads", [0, 1, 2])
def test_fp8_fixture(group_heads):
    case, truth, meta = GC.load("fp8_ring")
    h = case.hq
    plan = oa.decode_plan(case.rows, h, h, case.page, int(case.lens().max()), 0)
    plan.group_heads = group_heads
    out = torch.zeros(case.rows, h * 128, dtype=torch.bfloat16, device="cuda")
    kv = torch.from_numpy(np.ascontiguousarray(case.kv)).cuda()
    oa.lm_attend_fp8(dev_bits(case.qkv), kv, dev_i32(case.pos), dev_i32(case.seq), 0, dev_i32(case.indptr),
                     dev_i32(case.pages), case.page, out, h, case.scale, case.context, plan, oa.workspace_for(plan))
    torch.cuda.synchronize()
    check("fp8_ring", host_bits(out), truth, meta)
