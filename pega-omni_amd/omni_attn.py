"""Host-side mirror of the engines' attention ops over the C ABI.

The reference engines launch ``qwen3_attend`` (crates/omni-qwen3/src/stack.rs:
207-241), ``lm_attend`` (crates/omni-personaplex/src/helium.rs:256-275) and
``hidream_attend`` (crates/omni-hidream-o1/src/model.rs:362-380) with raw
device pointers. This module exposes the same calls, argument for argument,
over ``libomni_attn.so`` via ctypes, taking torch tensors only as holders of
device memory and streams. There is no fallback: if the HIP library is absent
or a launch fails, the call raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libomni_attn.so")
HEAD_DIM = 128

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
ELAUNCH = -3
EWORKSPACE = -4
ETABLE = -5

EXPORTS = (
    "omni_attn_decode_plan_init",
    "omni_attn_decode_plan_init_fp8",
    "omni_qwen3_attend",
    "omni_qwen3_attend_noalloc",
    "omni_lm_attend",
    "omni_lm_attend_fp8",
    "omni_attn_decode_run_lastlen",
    "omni_attn_check_table",
    "omni_attn_gather_kv",
    "omni_attn_prefill_plan_init",
    "omni_hidream_rows",
    "omni_attn_prefill_run",
    "omni_hidream_attend",
    "omni_hidream_attend_batched",
    "omni_hidream_attend_ws",
    "omni_hidream_workspace_bytes",
    "omni_qwen3_attend_dense",
    "omni_mimi_attend",
    "omni_mimi_rope_kv",
    "omni_lm_copy_kv",
    "omni_codec_attention",
    "omni_lm_dep_kv_attend",
    "omni_qwen3_rope",
    "omni_qwen3_rope_dense",
    "omni_qwen3_rope_attend",
    "omni_lm_rope_attend_fp8",
    "omni_lm_rope",
    "omni_hidream_qk_rope",
    "omni_attn_rows_new",
    "omni_attn_rows_free",
    "omni_attn_rows_clear",
    "omni_attn_rows_push",
    "omni_attn_rows_count",
    "omni_attn_rows_get",
    "omni_attn_version",
    "omni_attn_last_error",
)


class OmniAttnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"omni_attn error {code}: {msg}")
        self.code = code


class DecodePlan(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int32),
        ("hq", ctypes.c_int32),
        ("hk", ctypes.c_int32),
        ("page", ctypes.c_int32),
        ("max_len", ctypes.c_int32),
        ("chunk", ctypes.c_int32),
        ("splits", ctypes.c_int32),
        ("group_heads", ctypes.c_int32),  # FP8 kernel: heads per workgroup, 0 = auto
        ("workspace_bytes", ctypes.c_int64),
    ]


class PrefillPlan(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int32),
        ("hq", ctypes.c_int32),
        ("hk", ctypes.c_int32),
        ("page", ctypes.c_int32),
        ("tiles", ctypes.c_int32),
        ("tile_rows", ctypes.c_int32),
        ("work_bytes", ctypes.c_int64),
        ("workgroups", ctypes.c_int32),
        ("exact_p", ctypes.c_int32),
    ]


_lib = None


def load(path: str | None = None):
    """Load the HIP library (raises if it was not built). OMNI_ATTN_LIB names
    another build of the same library (A/B measurements)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or os.environ.get("OMNI_ATTN_LIB") or LIB_PATH
    if not os.path.exists(path):
        raise OmniAttnError(ELAUNCH, f"{path} is missing: build it with pega-omni_amd/build.py")
    # torch brings its own HIP runtime; load it first so the library binds to
    # the same one instead of pulling in a second copy from /opt/rocm.
    import torch  # noqa: F401

    L = ctypes.CDLL(path)
    P, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    dplan = ctypes.POINTER(DecodePlan)
    pplan = ctypes.POINTER(PrefillPlan)
    sig = {
        "omni_attn_decode_plan_init": [i32, i32, i32, i32, i32, i32, dplan],
        "omni_attn_decode_plan_init_fp8": [i32, i32, i32, i32, i32, dplan],
        "omni_qwen3_attend": [P, P, P, P, i32, P, P, i32, P, i32, i32, f32, dplan, P, P],
        "omni_qwen3_attend_noalloc": [P, P, P, P, i32, P, P, i32, P, i32, i32, f32, dplan, P],
        "omni_lm_attend": [P, P, P, P, i32, P, P, i32, P, i32, f32, i32, dplan, P, P],
        "omni_lm_attend_fp8": [P, P, P, P, i32, P, P, i32, P, i32, f32, i32, dplan, P, P],
        "omni_attn_decode_run_lastlen": [P, P, P, P, i32, P, P, i32, P, i32, i32, f32, dplan, P, P],
        "omni_attn_check_table": [P, i32, P, i32, P, P, i32, i32, i32, i32],
        "omni_attn_gather_kv": [P, i32, P, P, i32, P, P, P, i32, P, P],
        "omni_attn_prefill_plan_init": [i32, i32, i32, i32, P, P, P, i64, pplan],
        "omni_hidream_rows": [i32, i32, i32, i32, P, P, P, P, P],
        "omni_attn_prefill_run": [pplan, P, P, P, P, P, P, P, f32, P, P],
        "omni_hidream_attend": [P, P, P, P, i32, P, i32, i32, f32, i32, i32, P],
        "omni_hidream_attend_batched": [P, P, P, P, i32, P, i32, i32, f32, i32, i32, i32, i64, i64, i64, P],
        "omni_hidream_attend_ws": [P, P, P, P, i32, P, i32, i32, f32, i32, i32, i32, i64, i64, i64, P, i64, P],
        "omni_hidream_workspace_bytes": [],
        "omni_qwen3_attend_dense": [P, P, i32, i32, i32, P, i32, i32, f32, dplan, P, P],
        "omni_mimi_attend": [P, P, P, P, P, i32, i32, i32, f32, i32, i64, P],
        "omni_mimi_rope_kv": [P, P, P, P, i32, i32, i32, f32, i32, i64, P],
        "omni_lm_copy_kv": [P, P, P, i32, i32, P],
        "omni_codec_attention": [P, P, P, P, P, i32, i64, i32, f32, P],
        "omni_lm_dep_kv_attend": [P, P, i32, P, i32, i32, f32, P],
        "omni_qwen3_rope": [P, P, P, P, P, P, i32, i32, i32, f32, f32, P],
        "omni_qwen3_rope_dense": [P, P, P, P, i32, i32, i32, i32, i32, i32, f32, f32, P],
        "omni_qwen3_rope_attend": [P, P, P, P, P, P, P, P, i32, P, i32, i32, f32, f32, f32, dplan, P, P],
        "omni_lm_rope_attend_fp8": [P, P, P, P, P, P, i32, P, i32, f32, f32, i32, dplan, P, P],
        "omni_lm_rope": [P, P, P, P, i32, i32, f32, P],
        "omni_hidream_qk_rope": [P, i32, P, P, P, P, P, P, i32, i32, i32, i32, f32, f32, P],
        "omni_attn_version": [],
        "omni_attn_last_error": [],
    }
    sig.update({
        "omni_attn_rows_new": [i32, i32],
        "omni_attn_rows_free": [P],
        "omni_attn_rows_clear": [P],
        "omni_attn_rows_push": [P, P, i32, i32, i32, i32],
        "omni_attn_rows_count": [P, P, P, P],
        "omni_attn_rows_get": [P, i32],
    })
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = (ctypes.c_char_p if name == "omni_attn_last_error"
                      else ctypes.c_int64 if name == "omni_hidream_workspace_bytes"
                      else ctypes.c_void_p if name == "omni_attn_rows_new"
                      else ctypes.POINTER(ctypes.c_int32) if name == "omni_attn_rows_get"
                      else None if name in ("omni_attn_rows_free", "omni_attn_rows_clear") else ctypes.c_int)
    _lib = L
    return L


def _check(rc: int):
    if rc != OK:
        raise OmniAttnError(rc, load().omni_attn_last_error().decode())


def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _bf16_dev(t, name):
    import torch

    if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
        raise OmniAttnError(EINVAL, f"{name} must be a contiguous bf16 device tensor")


def _i32_dev(t, name):
    import torch

    if t is None:
        return
    if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous():
        raise OmniAttnError(EINVAL, f"{name} must be a contiguous int32 device tensor")


def _ws(plan, workspace):
    """The workspace pointer for a decode run, after checking that it holds the
    plan's split partials (the C call takes no size: a smaller buffer would be
    written past its end)."""
    need = int(plan.workspace_bytes)
    if workspace is None:
        return None
    if workspace.numel() * workspace.element_size() < need:
        raise OmniAttnError(EWORKSPACE, f"workspace holds {workspace.numel() * workspace.element_size()} bytes, "
                                        f"the plan needs {need}")
    if not workspace.is_cuda or not workspace.is_contiguous():
        raise OmniAttnError(EINVAL, "workspace must be a contiguous device tensor")
    return _ptr(workspace)


# --------------------------------------------------------------------- decode
def decode_plan(rows: int, hq: int, hk: int, page: int, max_len: int, chunk: int = 0) -> DecodePlan:
    plan = DecodePlan()
    _check(load().omni_attn_decode_plan_init(rows, hq, hk, page, max_len, chunk, ctypes.byref(plan)))
    return plan


def decode_plan_fp8(rows: int, heads: int, page: int, max_len: int, chunk: int = 0) -> DecodePlan:
    """The plan for lm_attend over FP8 slots (split size picked for the FP8 kernel)."""
    plan = DecodePlan()
    _check(load().omni_attn_decode_plan_init_fp8(rows, heads, page, max_len, chunk, ctypes.byref(plan)))
    return plan


def workspace_for(plan, device="cuda"):
    """Device workspace for a plan (None when the plan needs none)."""
    import torch

    n = int(plan.workspace_bytes)
    return torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None


def check_table(indptr_h, pages_h, num_pages, pos_h=None, seq_h=None, ragged=False, page=16, context=0):
    """Host validation of a page table (numpy int32 arrays)."""
    import numpy as np

    indptr_h = np.ascontiguousarray(indptr_h, dtype=np.int32)
    pages_h = np.ascontiguousarray(pages_h, dtype=np.int32)
    rows = 0 if pos_h is None else len(pos_h)
    pos_a = None if pos_h is None else np.ascontiguousarray(pos_h, dtype=np.int32)
    seq_a = None if seq_h is None else np.ascontiguousarray(seq_h, dtype=np.int32)
    rc = load().omni_attn_check_table(
        indptr_h.ctypes.data_as(ctypes.c_void_p), len(indptr_h) - 1, pages_h.ctypes.data_as(ctypes.c_void_p),
        num_pages, None if pos_a is None else pos_a.ctypes.data_as(ctypes.c_void_p),
        None if seq_a is None else seq_a.ctypes.data_as(ctypes.c_void_p), int(ragged), rows, page, context)
    _check(rc)


def qwen3_attend(qkv, kv, pos, seq, ragged, indptr, pages, page, out, hq, hk, scale, plan, workspace=None,
                 stream=None):
    """``qwen3_attend`` (crates/omni-qwen3/kernels/qwen3.cu:234-240) on the GPU."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    for t, n in ((pos, "pos"), (seq, "seq"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_qwen3_attend(_ptr(qkv), _ptr(kv), _ptr(pos), _ptr(seq), int(ragged), _ptr(indptr),
                                    _ptr(pages), page, _ptr(out), hq, hk, float(scale), ctypes.byref(plan),
                                    _ws(plan, workspace), _stream(stream)))
    return out


def qwen3_attend_noalloc(qkv, kv, pos, seq, ragged, indptr, pages, page, out, hq, hk, scale, plan, stream=None):
    """``qwen3_attend`` without a workspace argument: the split partials go to
    the library's static per-GPU scratch (no allocation; calls that overlap on
    one GPU race). No counterpart in the reference."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    for t, n in ((pos, "pos"), (seq, "seq"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_qwen3_attend_noalloc(_ptr(qkv), _ptr(kv), _ptr(pos), _ptr(seq), int(ragged), _ptr(indptr),
                                            _ptr(pages), page, _ptr(out), hq, hk, float(scale), ctypes.byref(plan),
                                            _stream(stream)))
    return out


def lm_attend(qkv, kv, pos, seq, ragged, indptr, pages, page, out, heads, scale, context, plan, workspace=None,
              stream=None):
    """``lm_attend`` (crates/omni-personaplex/kernels/lm.cu:275-290) over bf16 slots."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    for t, n in ((pos, "pos"), (seq, "seq"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_lm_attend(_ptr(qkv), _ptr(kv), _ptr(pos), _ptr(seq), int(ragged), _ptr(indptr), _ptr(pages),
                                 page, _ptr(out), heads, float(scale), context, ctypes.byref(plan),
                                 _ws(plan, workspace), _stream(stream)))
    return out


def lm_attend_fp8(qkv, kv, pos, seq, ragged, indptr, pages, page, out, heads, scale, context, plan, workspace=None,
                  stream=None):
    """``lm_attend`` over FP8 E4M3 slots (crates/omni-personaplex/kernels/lm.cu:196-290).
    kv is a uint8 device tensor of slots of 2*heads*128 + 2*heads*4 bytes."""
    import torch

    _bf16_dev(qkv, "qkv"), _bf16_dev(out, "out")
    if kv.dtype != torch.uint8 or not kv.is_cuda or not kv.is_contiguous():
        raise OmniAttnError(EINVAL, "kv must be a contiguous uint8 device tensor of FP8 slots")
    for t, n in ((pos, "pos"), (seq, "seq"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_lm_attend_fp8(_ptr(qkv), _ptr(kv), _ptr(pos), _ptr(seq), int(ragged), _ptr(indptr),
                                     _ptr(pages), page, _ptr(out), heads, float(scale), context, ctypes.byref(plan),
                                     _ws(plan, workspace), _stream(stream)))
    return out


def decode_lastlen(qkv, kv, last_page_len, seq, ragged, indptr, pages, page, out, hq, hk, scale, plan,
                   workspace=None, stream=None):
    """Decode with per-sequence last-page lengths instead of positions."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    _check(load().omni_attn_decode_run_lastlen(_ptr(qkv), _ptr(kv), _ptr(last_page_len), _ptr(seq), int(ragged),
                                               _ptr(indptr), _ptr(pages), page, _ptr(out), hq, hk, float(scale),
                                               ctypes.byref(plan), _ws(plan, workspace), _stream(stream)))
    return out


def gather_kv(kv, hk, indptr, pages, page, seq_ids, lens, out_indptr, out, stream=None):
    """Bit-exact paged -> dense copy of K/V slots (the page-table rule)."""
    nseq = int(seq_ids.numel())
    _check(load().omni_attn_gather_kv(_ptr(kv), hk, _ptr(indptr), _ptr(pages), page, _ptr(seq_ids), _ptr(lens),
                                      _ptr(out_indptr), nseq, _ptr(out), _stream(stream)))
    return out


# -------------------------------------------------------------------- prefill
@dataclass
class Prefill:
    plan: PrefillPlan
    work: object  # device int32 tensor


def prefill_plan(rows, hq, hk, page, seq_h, pos_h, device="cuda", exact_p=False) -> Prefill:
    """Host plan of a ragged causal prefill; uploads the work list. exact_p:
    P carried as two bf16 terms through P.V (qwen3_attend's f32 P, ~1.4x the time)."""
    import numpy as np
    import torch

    seq_a = np.ascontiguousarray(seq_h, dtype=np.int32)
    pos_a = np.ascontiguousarray(pos_h, dtype=np.int32)
    plan = PrefillPlan()
    L = load()
    rc = L.omni_attn_prefill_plan_init(rows, hq, hk, page, seq_a.ctypes.data_as(ctypes.c_void_p),
                                       pos_a.ctypes.data_as(ctypes.c_void_p), None, 0, ctypes.byref(plan))
    if rc not in (OK, EWORKSPACE):
        _check(rc)
    cap = max(1, int(plan.work_bytes) // 4)
    work_h = np.zeros(cap, dtype=np.int32)
    _check(L.omni_attn_prefill_plan_init(rows, hq, hk, page, seq_a.ctypes.data_as(ctypes.c_void_p),
                                         pos_a.ctypes.data_as(ctypes.c_void_p),
                                         work_h.ctypes.data_as(ctypes.c_void_p), cap, ctypes.byref(plan)))
    plan.exact_p = 1 if exact_p else 0
    return Prefill(plan, torch.from_numpy(work_h).to(device))


def prefill_run(pf: Prefill, qkv, kv, pos, seq, indptr, pages, out, scale, stream=None):
    """Ragged causal prefill with qwen3_attend(ragged = 1) semantics (MFMA)."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    _check(load().omni_attn_prefill_run(ctypes.byref(pf.plan), _ptr(qkv), _ptr(kv), _ptr(pos), _ptr(seq),
                                        _ptr(indptr), _ptr(pages), _ptr(out), float(scale), _ptr(pf.work),
                                        _stream(stream)))
    return out


# ------------------------------------------------------------------------ DiT
def hidream_attend(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, stream=None):
    """``hidream_attend`` (crates/omni-hidream-o1/kernels/hidream.cu:209-347)."""
    _check(load().omni_hidream_attend(_ptr(q), _ptr(k), _ptr(v), _ptr(out), q_len, _ptr(kv_len_at), q_stride,
                                      int(causal), float(scale_log2), hq, hk, _stream(stream)))
    return out


def hidream_attend_batched(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, batch, q_bstride,
                           kv_bstride, out_bstride, stream=None):
    _check(load().omni_hidream_attend_batched(_ptr(q), _ptr(k), _ptr(v), _ptr(out), q_len, _ptr(kv_len_at), q_stride,
                                              int(causal), float(scale_log2), hq, hk, batch, q_bstride, kv_bstride,
                                              out_bstride, _stream(stream)))
    return out


# ------------------------------------------------ rotary embedding + K/V scatter
def qwen3_rope(qkv, q_norm, k_norm, pos, slots, kv, rows, hq, hk, eps, theta, stream=None):
    """``qwen3_rope`` (crates/omni-qwen3/kernels/qwen3.cu:64-103): q rotated in
    place, K and V written to slot ``slots[n]`` of the bf16 paged cache."""
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (kv, "kv")):
        _bf16_dev(t, n)
    _i32_dev(pos, "pos"), _i32_dev(slots, "slots")
    _check(load().omni_qwen3_rope(_ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(pos), _ptr(slots), _ptr(kv), rows, hq,
                                  hk, float(eps), float(theta), _stream(stream)))


def qwen3_rope_attend(qkv, q_norm, k_norm, pos, slots, kv, indptr, pages, page, out, hq, hk, eps, theta, scale, plan,
                      workspace=None, stream=None):
    """``qwen3_rope`` then ``qwen3_attend`` (ragged = 0) in one launch: K and V
    of row n written to ``slots[n]`` (which must be the slot of key pos[n]),
    q rotated in registers only (qkv is not written)."""
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (kv, "kv"), (out, "out")):
        _bf16_dev(t, n)
    for t, n in ((pos, "pos"), (slots, "slots"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_qwen3_rope_attend(_ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(pos), _ptr(slots), _ptr(kv),
                                         _ptr(indptr), _ptr(pages), page, _ptr(out), hq, hk, float(eps), float(theta),
                                         float(scale), ctypes.byref(plan), _ws(plan, workspace), _stream(stream)))
    return out


def lm_rope_attend_fp8(qkv, pos, slots, kv, indptr, pages, page, out, heads, coef, scale, context, plan,
                       workspace=None, stream=None):
    """``lm_rope`` then ``lm_attend`` over FP8 slots (ragged = 0) in one launch:
    K and V of row n quantized into ``slots[n]`` (which must be the slot of ring
    index pos[n] % context), q rotated in registers only (qkv is not written)."""
    import torch
    for t, n in ((qkv, "qkv"), (out, "out")):
        _bf16_dev(t, n)
    if kv.dtype != torch.uint8 or not kv.is_cuda or not kv.is_contiguous():
        raise OmniAttnError(EINVAL, "kv must be a contiguous uint8 device tensor of FP8 slots")
    for t, n in ((pos, "pos"), (slots, "slots"), (indptr, "indptr"), (pages, "pages")):
        _i32_dev(t, n)
    _check(load().omni_lm_rope_attend_fp8(_ptr(qkv), _ptr(pos), _ptr(slots), _ptr(kv), _ptr(indptr), _ptr(pages), page,
                                          _ptr(out), heads, float(coef), float(scale), context, ctypes.byref(plan),
                                          _ws(plan, workspace), _stream(stream)))
    return out


def qwen3_rope_dense(qkv, q_norm, k_norm, kv, rows, per, base, span, hq, hk, eps, theta, stream=None):
    """``qwen3_rope_dense`` (qwen3.cu:105-111)."""
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (kv, "kv")):
        _bf16_dev(t, n)
    _check(load().omni_qwen3_rope_dense(_ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(kv), rows, per, base, span, hq,
                                        hk, float(eps), float(theta), _stream(stream)))


def lm_rope(qkv, pos, slots, kv, rows, heads, coef, stream=None):
    """``lm_rope`` (crates/omni-personaplex/kernels/lm.cu:125-182): kv is a
    uint8 device tensor of FP8 slots."""
    import torch

    _bf16_dev(qkv, "qkv"), _i32_dev(pos, "pos"), _i32_dev(slots, "slots")
    if kv.dtype != torch.uint8 or not kv.is_cuda or not kv.is_contiguous():
        raise OmniAttnError(EINVAL, "kv must be a contiguous uint8 device tensor of FP8 slots")
    _check(load().omni_lm_rope(_ptr(qkv), _ptr(pos), _ptr(slots), _ptr(kv), rows, heads, float(coef),
                               _stream(stream)))


def hidream_qk_rope(qkv, ld, q_norm, k_norm, positions, slots, k_cache, v_cache, rows, hq, hk, mrope_hw, eps, theta,
                    stream=None):
    """``hidream_qk_rope`` (crates/omni-hidream-o1/kernels/hidream.cu:55-106)."""
    for t, n in ((qkv, "qkv"), (q_norm, "q_norm"), (k_norm, "k_norm"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16_dev(t, n)
    _i32_dev(positions, "positions"), _i32_dev(slots, "slots")
    _check(load().omni_hidream_qk_rope(_ptr(qkv), ld, _ptr(q_norm), _ptr(k_norm), _ptr(positions), _ptr(slots),
                                       _ptr(k_cache), _ptr(v_cache), rows, hq, hk, mrope_hw, float(eps),
                                       float(theta), _stream(stream)))


# ------------------------------------------------- dense and head-64 attentions
def qwen3_attend_dense(qkv, kv, per, base, span, out, hq, hk, scale, plan, workspace=None, stream=None):
    """``qwen3_attend_dense`` (crates/omni-qwen3/kernels/qwen3.cu:243-248); the
    plan is made with page = 1 and max_len >= base + per."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(kv, "kv"), _bf16_dev(out, "out")
    _check(load().omni_qwen3_attend_dense(_ptr(qkv), _ptr(kv), per, base, span, _ptr(out), hq, hk, float(scale),
                                          ctypes.byref(plan), _ws(plan, workspace), _stream(stream)))
    return out


def mimi_rope_kv(qkv, pos, lines, state, rows, T, heads, coef, context, stride, stream=None):
    """``mimi_rope_kv`` (crates/omni-personaplex/kernels/mimi.cu:226-246): q turned
    in place, k turned and v copied into each row's ring slot of ``state``."""
    _bf16_dev(qkv, "qkv"), _i32_dev(pos, "pos"), _i32_dev(lines, "lines")
    _check(load().omni_mimi_rope_kv(_ptr(qkv), _ptr(pos), _ptr(lines), _ptr(state), rows, T, heads, float(coef),
                                    context, int(stride), _stream(stream)))
    return qkv


def lm_copy_kv(kv, src_slot, dst_slot, tokens, slot_bytes, stream=None):
    """``lm_copy_kv`` (crates/omni-personaplex/kernels/lm.cu:583-593): slot
    dst_slot[r] takes the bytes of slot src_slot[r] (prefix K/V reuse)."""
    _i32_dev(src_slot, "src_slot"), _i32_dev(dst_slot, "dst_slot")
    _check(load().omni_lm_copy_kv(_ptr(kv), _ptr(src_slot), _ptr(dst_slot), tokens, slot_bytes, _stream(stream)))
    return kv


def mimi_attend(qkv, pos, lines, state, out, rows, T, heads, scale, context, stride, stream=None):
    """``mimi_attend`` (crates/omni-personaplex/kernels/mimi.cu:248-263); state is
    any contiguous device tensor holding the per-session rings."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(out, "out"), _i32_dev(pos, "pos"), _i32_dev(lines, "lines")
    _check(load().omni_mimi_attend(_ptr(qkv), _ptr(pos), _ptr(lines), _ptr(state), _ptr(out), rows, T, heads,
                                   float(scale), context, int(stride), _stream(stream)))
    return out


def codec_attention(qkv, pos, lines, kv, out, rows, stride, heads, theta, stream=None):
    """``codec_attention`` (crates/omni-qwen3-tts/kernels/codec.cu:168-277)."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(out, "out"), _i32_dev(pos, "pos"), _i32_dev(lines, "lines")
    _check(load().omni_codec_attention(_ptr(qkv), _ptr(pos), _ptr(lines), _ptr(kv), _ptr(out), rows, int(stride),
                                       heads, float(theta), _stream(stream)))
    return out


def lm_dep_kv_attend(qkv, ws, step, out, rows, heads, scale, stream=None):
    """``lm_dep_kv_attend`` (crates/omni-personaplex/kernels/lm.cu:314-366)."""
    _bf16_dev(qkv, "qkv"), _bf16_dev(ws, "ws"), _bf16_dev(out, "out")
    _check(load().omni_lm_dep_kv_attend(_ptr(qkv), _ptr(ws), step, _ptr(out), rows, heads, float(scale),
                                        _stream(stream)))
    return out


def hidream_workspace(device="cuda"):
    """A workspace for hidream_attend_ws on the current device."""
    import torch

    return torch.empty(int(load().omni_hidream_workspace_bytes()), dtype=torch.uint8, device=device)


def hidream_attend_ws(q, k, v, out, q_len, kv_len_at, q_stride, causal, scale_log2, hq, hk, batch, q_bstride,
                      kv_bstride, out_bstride, workspace, stream=None):
    """The batched DiT call with the tail split (a workspace from hidream_workspace)."""
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(load().omni_hidream_attend_ws(_ptr(q), _ptr(k), _ptr(v), _ptr(out), q_len, _ptr(kv_len_at), q_stride,
                                         int(causal), float(scale_log2), hq, hk, batch, int(q_bstride),
                                         int(kv_bstride), int(out_bstride), _ptr(workspace), nbytes,
                                         _stream(stream)))
    return out


# ------------------------------------------------------------ host row builder
class Rows:
    """The engines' ``Rows`` (crates/omni-qwen3-tts/src/model.rs:266-303,
    crates/omni-personaplex/src/model.rs:472-499) on the native builder:
    ``push(page_ids, first, count, seq)`` per sequence, then the int32 arrays
    ``pos``, ``slot``, ``seq``, ``indptr``, ``pages`` (numpy copies)."""

    _WHICH = {"pos": 0, "slot": 1, "seq": 2, "indptr": 3, "pages": 4}

    def __init__(self, page: int = 16, ring: int = 0):
        h = load().omni_attn_rows_new(page, ring)
        if not h:
            raise OmniAttnError(EINVAL, load().omni_attn_last_error().decode())
        self._h = ctypes.c_void_p(h)

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.omni_attn_rows_free(self._h)
            self._h = None

    def push(self, page_ids, first: int, count: int, seq: int):
        import numpy as np

        ids = np.ascontiguousarray(page_ids, dtype=np.int32)
        _check(load().omni_attn_rows_push(self._h, ids.ctypes.data_as(ctypes.c_void_p), len(ids), first, count, seq))

    def clear(self):
        load().omni_attn_rows_clear(self._h)

    def counts(self):
        r, s, p = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(load().omni_attn_rows_count(self._h, ctypes.byref(r), ctypes.byref(s), ctypes.byref(p)))
        return r.value, s.value, p.value

    def __getattr__(self, name):
        if name not in Rows._WHICH:
            raise AttributeError(name)
        import numpy as np

        rows, seqs, pages = self.counts()
        n = {"pos": rows, "slot": rows, "seq": rows, "indptr": seqs + 1 if seqs else 0, "pages": pages}[name]
        if n == 0:
            return np.zeros(0, np.int32)
        ptr = load().omni_attn_rows_get(self._h, Rows._WHICH[name])
        return np.ctypeslib.as_array(ptr, shape=(n,)).copy()


def hidream_rows(causal, grid, image_position=4096):
    """HiDream-O1's host row arrays (``model.rs:123-160``): (text_pos [causal][3],
    text_slots, gen_pos [rows][3], gen_slots, step_kv) as numpy int32."""
    import numpy as np

    rows = 1 + grid[0] * grid[1]
    tp = np.zeros((causal, 3), np.int32)
    ts = np.zeros(causal, np.int32)
    gp = np.zeros((rows, 3), np.int32)
    gs = np.zeros(rows, np.int32)
    kv = np.zeros(1, np.int32)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    _check(load().omni_hidream_rows(causal, grid[0], grid[1], image_position, ptr(tp), ptr(ts), ptr(gp), ptr(gs),
                                    ptr(kv)))
    return tp, ts, gp, gs, int(kv[0])
