"""The boundary checked from compiled code, without a GPU:

* tests/c/abi_check.c, a C consumer of include/omni_attn.h built with gcc
  -Werror and linked to libomni_attn.so, asserts the documented return codes
  of the host-only entry points and of the validation every run call does
  before it launches;
* the same program and tests/c/host_fuzz.c (seeded malformed inputs) against
  a build of capi.cpp's host pass under AddressSanitizer + UBSan;
* the kernels' index arithmetic (csrc/indexing.h) on the host (tests/c/indexing_check.cpp);
* the ctypes signatures the Python mirror binds agree, parameter by
  parameter, with the prototypes the header declares.
"""
import ctypes
import os
import re
import subprocess

import pytest

import omni_attn as oa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CDIR = os.path.join(ROOT, "tests", "c")


def _make(*targets):
    r = subprocess.run(["make", "-s", "-C", CDIR, *targets], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return r.stdout


def test_abi_check_c_consumer():
    if not os.path.exists(oa.LIB_PATH):
        pytest.skip("libomni_attn.so is not built")
    out = _make("abi")
    assert "checks passed" in out


def test_kernel_index_arithmetic_on_the_host():
    """A host build of csrc/indexing.h: the kernels' multiply-high division by
    any page size against / and %, and the decode split rotation (every split
    index of a unit exactly once, for 1..64 splits and many units)."""
    out = _make("indexing")
    assert "page division" in out and "split rotation" in out


@pytest.mark.skipif(os.environ.get("OMNI_SANITIZED") == "1", reason="already running under the sanitizer build")
def test_host_code_under_asan_ubsan():
    if not os.path.exists(os.path.join(ROOT, "pega-omni_amd", "_build", "decode.hip.o")):
        pytest.skip("kernel objects are not built")
    _make(*(os.path.join(CDIR, "_build", t) for t in ("abi_check_san", "host_fuzz_san")))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1")
    for exe, want in (("abi_check_san", "checks passed"), ("host_fuzz_san", "cases")):
        r = subprocess.run([os.path.join(CDIR, "_build", exe)], capture_output=True, text=True, env=env)
        assert r.returncode == 0 and want in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


def _header_prototypes():
    text = open(os.path.join(ROOT, "include", "omni_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(omni_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        protos[m.group(1)] = params
    return protos


def _kind_of_c(param: str) -> str:
    if "*" in param:
        return "ptr"
    if param.startswith("int64_t"):
        return "i64"
    if param.startswith("float"):
        return "f32"
    if param.startswith(("int ", "int32_t")):
        return "i32"
    raise AssertionError(f"unclassified parameter {param!r}")


def _kind_of_ctypes(t) -> str:
    if t is ctypes.c_void_p or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return "ptr"
    return {ctypes.c_int64: "i64", ctypes.c_float: "f32", ctypes.c_int: "i32", ctypes.c_int32: "i32"}[t]


def test_ctypes_signatures_match_header():
    if not os.path.exists(oa.LIB_PATH):
        pytest.skip("libomni_attn.so is not built")
    L = oa.load()
    protos = _header_prototypes()
    assert set(protos) == set(oa.EXPORTS)
    for name, params in protos.items():
        want = [_kind_of_c(p) for p in params]
        got = [_kind_of_ctypes(t) for t in getattr(L, name).argtypes]
        assert got == want, f"{name}: header {want}, ctypes {got}"
