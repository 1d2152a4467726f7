"""CPU oracle bindings — test infrastructure only.

ctypes wrappers around ``liboracle.so`` (built from ``omni_attn_oracle.c`` by
``oracle/Makefile``), plus numpy helpers for bf16. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module; the product library never does.

Every function is a restatement of the reference kernel it names (file:line in
the pega-omni tree):

* :func:`paged_attend`  — ``crates/omni-qwen3/kernels/qwen3.cu:123-240``
  (``qwen3_attend``) and, with ``context``, ``crates/omni-personaplex/kernels/
  lm.cu:273-290`` (``lm_attend``) over bf16 slots (``attend.cuh:41-106``).
* :func:`dense_attend`  — ``crates/omni-hidream-o1/kernels/hidream.cu:209-347``.
* :func:`lm_attend_fp8` — ``crates/omni-personaplex/kernels/lm.cu:196-290`` (FP8 E4M3 slots).
* :func:`gather_kv` / :func:`slot` — ``qwen3.cu:210-214`` (``PagedSlots``).
* :func:`qwen3_rope` / :func:`qwen3_rope_dense` — ``qwen3.cu:64-111``.
* :func:`qwen3_attend_dense` — ``qwen3.cu:243-248``.
* :func:`mimi_attend` — ``crates/omni-personaplex/kernels/mimi.cu:248-263``.
* :func:`mimi_rope_kv` — ``crates/omni-personaplex/kernels/mimi.cu:226-246``.
* :func:`lm_copy_kv` — ``crates/omni-personaplex/kernels/lm.cu:583-593``.
* :func:`codec_attention` — ``crates/omni-qwen3-tts/kernels/codec.cu:168-277``.
* :func:`lm_dep_kv_attend` — ``crates/omni-personaplex/kernels/lm.cu:314-366``.
* :func:`hidream_qk_rope` — ``crates/omni-hidream-o1/kernels/hidream.cu:55-106``.
* :func:`lm_rope` / :func:`f32_to_e4m3` — ``crates/omni-personaplex/kernels/lm.cu:125-182``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so with gcc (the oracle Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        # OMNI_ORACLE_LIB names another build of the same source (the
        # sanitizer build of tests/c/Makefile).
        path = os.environ.get("OMNI_ORACLE_LIB") or _LIB
        if path == _LIB and not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        i32, f32, i64, u64 = ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_uint64
        L.oracle_paged_attend.argtypes = [P, P, P, P, i32, P, P, i32, P, i32, i32, i32, f32, i32, i32]
        L.oracle_paged_attend.restype = i32
        L.oracle_dense_attend.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i32, f32, i32]
        L.oracle_dense_attend.restype = i32
        L.oracle_gather_kv.argtypes = [P, i32, P, P, i32, i32, i32, P]
        L.oracle_gather_kv.restype = None
        L.oracle_slot.argtypes = [P, P, i32, i32, i32]
        L.oracle_slot.restype = i64
        L.oracle_fill_normal_bf16.argtypes = [P, i64, u64]
        L.oracle_fill_normal_bf16.restype = None
        L.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.oracle_e4m3_to_f32.restype = ctypes.c_float
        L.oracle_lm_attend_fp8.argtypes = [P, P, P, P, i32, P, P, i32, P, i32, i32, f32, i32, i32]
        L.oracle_lm_attend_fp8.restype = i32
        L.oracle_qwen3_attend_dense.argtypes = [P, P, i32, i32, i32, P, i32, i32, i32, f32, i32]
        L.oracle_qwen3_attend_dense.restype = i32
        L.oracle_mimi_attend.argtypes = [P, P, P, P, P, i32, i32, i32, f32, i32, i64]
        L.oracle_mimi_attend.restype = None
        L.oracle_mimi_rope_kv.argtypes = [P, P, P, P, i32, i32, i32, f32, i32, i64]
        L.oracle_mimi_rope_kv.restype = None
        L.oracle_lm_copy_kv.argtypes = [P, P, P, i32, i32]
        L.oracle_lm_copy_kv.restype = None
        L.oracle_codec_attention.argtypes = [P, P, P, P, P, i32, i64, i32, f32]
        L.oracle_codec_attention.restype = None
        L.oracle_lm_dep_kv_attend.argtypes = [P, P, i32, P, i32, i32, f32]
        L.oracle_lm_dep_kv_attend.restype = None
        L.oracle_f32_to_e4m3.argtypes = [f32]
        L.oracle_f32_to_e4m3.restype = ctypes.c_uint8
        L.oracle_qwen3_rope.argtypes = [P, P, P, P, P, P, i32, i32, i32, f32, f32]
        L.oracle_qwen3_rope.restype = None
        L.oracle_qwen3_rope_dense.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, i32, f32, f32]
        L.oracle_qwen3_rope_dense.restype = None
        L.oracle_hidream_qk_rope.argtypes = [P, i32, P, P, P, P, P, P, i32, i32, i32, i32, f32, f32]
        L.oracle_hidream_qk_rope.restype = None
        L.oracle_lm_rope.argtypes = [P, P, P, P, i32, i32, f32]
        L.oracle_lm_rope.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------- bf16 helpers
def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round-to-nearest-even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def normal_bf16(n: int, seed: int) -> np.ndarray:
    """n draws of N(0,1) (splitmix64 + Box-Muller in double), as bf16 bits."""
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_fill_normal_bf16(_p(out), n, seed)
    return out


# ------------------------------------------------------------------ oracle calls
def paged_attend(qkv, kv, pos, seq, ragged, indptr, pages, page, hq, hk, scale, context=0, nthreads=1):
    """qwen3_attend / lm_attend over bf16 slots. Arrays are numpy: qkv uint16
    [rows][(hq+2hk)*128], kv uint16 [slots][2hk*128], int32 index arrays.
    Returns out uint16 [rows][hq*128]."""
    rows = int(pos.shape[0])
    out = np.zeros((rows, hq * 128), dtype=np.uint16)
    seq = np.ascontiguousarray(seq if seq is not None else np.zeros(rows, np.int32), dtype=np.int32)
    rc = lib().oracle_paged_attend(_p(qkv), _p(kv), _p(pos), _p(seq), int(ragged), _p(indptr), _p(pages), page,
                                   _p(out), rows, hq, hk, float(scale), int(context), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_paged_attend: unsupported shape")
    return out


def dense_attend(q, k, v, q_len, kv_len, q_stride, hq, hk, causal, scale_log2, nthreads=1):
    """hidream_attend: q uint16 rows of q_stride elements, k/v uint16
    [kv_len][hk*128]. Returns out uint16 [q_len][hq*128]."""
    out = np.zeros((q_len, hq * 128), dtype=np.uint16)
    rc = lib().oracle_dense_attend(_p(q), _p(k), _p(v), _p(out), q_len, kv_len, q_stride, hq, hk, int(causal),
                                   float(scale_log2), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_dense_attend: unsupported shape")
    return out


def e4m3_to_f32(b: int) -> float:
    return float(lib().oracle_e4m3_to_f32(b))


def lm_attend_fp8(qkv, kv, pos, seq, ragged, indptr, pages, page, heads, scale, context, nthreads=1):
    """lm_attend over FP8 E4M3 slots (lm.cu:196-290). kv is uint8
    [slots][2*heads*128 + 2*heads*4]. Returns out uint16 [rows][heads*128]."""
    rows = int(pos.shape[0])
    out = np.zeros((rows, heads * 128), dtype=np.uint16)
    seq = np.ascontiguousarray(seq if seq is not None else np.zeros(rows, np.int32), dtype=np.int32)
    rc = lib().oracle_lm_attend_fp8(_p(qkv), _p(kv), _p(pos), _p(seq), int(ragged), _p(indptr), _p(pages), page,
                                    _p(out), rows, heads, float(scale), int(context), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_lm_attend_fp8: unsupported shape")
    return out


def gather_kv(kv, hk, indptr, pages, page, s, length):
    out = np.zeros((length, 2 * hk * 128), dtype=np.uint16)
    lib().oracle_gather_kv(_p(kv), hk, _p(indptr), _p(pages), page, s, length, _p(out))
    return out


def slot(indptr, pages, s, t, page) -> int:
    return int(lib().oracle_slot(_p(indptr), _p(pages), s, t, page))


def f32_to_e4m3(x: float) -> int:
    return int(lib().oracle_f32_to_e4m3(float(x)))


def qwen3_rope(qkv, q_norm, k_norm, pos, slots, kv, hq, hk, eps, theta):
    """In place on copies: returns (qkv', kv') after qwen3_rope."""
    qkv, kv = qkv.copy(), kv.copy()
    lib().oracle_qwen3_rope(_p(qkv), _p(q_norm), _p(k_norm), _p(pos), _p(slots), _p(kv), int(pos.shape[0]), hq, hk,
                            float(eps), float(theta))
    return qkv, kv


def qwen3_rope_dense(qkv, q_norm, k_norm, kv, rows, per, base, span, hq, hk, eps, theta):
    qkv, kv = qkv.copy(), kv.copy()
    lib().oracle_qwen3_rope_dense(_p(qkv), _p(q_norm), _p(k_norm), _p(kv), rows, per, base, span, hq, hk, float(eps),
                                  float(theta))
    return qkv, kv


def hidream_qk_rope(qkv, ld, q_norm, k_norm, positions, slots, k_cache, v_cache, hq, hk, mrope_hw, eps, theta):
    qkv, k_cache, v_cache = qkv.copy(), k_cache.copy(), v_cache.copy()
    lib().oracle_hidream_qk_rope(_p(qkv), ld, _p(q_norm), _p(k_norm), _p(positions), _p(slots), _p(k_cache),
                                 _p(v_cache), int(slots.shape[0]), hq, hk, mrope_hw, float(eps), float(theta))
    return qkv, k_cache, v_cache


def lm_rope(qkv, pos, slots, kv, heads, coef):
    """kv: uint8 [slots][slot_bytes]. Returns (qkv', kv')."""
    qkv, kv = qkv.copy(), kv.copy()
    lib().oracle_lm_rope(_p(qkv), _p(pos), _p(slots), _p(kv), int(pos.shape[0]), heads, float(coef))
    return qkv, kv


def qwen3_attend_dense(qkv, kv, per, base, span, hq, hk, scale, nthreads=1):
    rows = int(qkv.shape[0])
    out = np.zeros((rows, hq * 128), dtype=np.uint16)
    if lib().oracle_qwen3_attend_dense(_p(qkv), _p(kv), per, base, span, _p(out), rows, hq, hk, float(scale),
                                       int(nthreads)) != 0:
        raise ValueError("oracle_qwen3_attend_dense: unsupported shape")
    return out


def mimi_attend(qkv, pos, lines, state, rows, T, heads, scale, context, stride):
    """state: uint8 bytes of every session's ring. Returns out uint16 [rows][heads*64]."""
    out = np.zeros((rows, heads * 64), dtype=np.uint16)
    lib().oracle_mimi_attend(_p(qkv), _p(pos), _p(lines), _p(state), _p(out), rows, T, heads, float(scale), context,
                             int(stride))
    return out


def mimi_rope_kv(qkv, pos, lines, state, rows, T, heads, coef, context, stride):
    """Returns (qkv', state'): q rotated in place, k rotated and v copied into
    each row's ring slot."""
    qkv, state = qkv.copy(), state.copy()
    lib().oracle_mimi_rope_kv(_p(qkv), _p(pos), _p(lines), _p(state), rows, T, heads, float(coef), context,
                              int(stride))
    return qkv, state


def lm_copy_kv(kv, src_slot, dst_slot, slot_bytes):
    """kv: uint8 [slots][slot_bytes]. Returns the cache after the copies."""
    kv = np.ascontiguousarray(kv).copy()
    src = np.ascontiguousarray(src_slot, dtype=np.int32)
    dst = np.ascontiguousarray(dst_slot, dtype=np.int32)
    lib().oracle_lm_copy_kv(_p(kv), _p(src), _p(dst), len(src), int(slot_bytes))
    return kv


def codec_attention(qkv, pos, lines, kv, rows, stride, heads, theta):
    """Returns (out, kv') with kv' the ring bytes after the frame writes."""
    kv = kv.copy()
    out = np.zeros((rows, heads * 64), dtype=np.uint16)
    lib().oracle_codec_attention(_p(qkv), _p(pos), _p(lines), _p(kv), _p(out), rows, int(stride), heads, float(theta))
    return out, kv


def lm_dep_kv_attend(qkv, ws, step, seqs, heads, scale):
    """Returns (out, ws')."""
    ws = ws.copy()
    out = np.zeros((seqs, heads * 64), dtype=np.uint16)
    lib().oracle_lm_dep_kv_attend(_p(qkv), _p(ws), step, _p(out), seqs, heads, float(scale))
    return out, ws
