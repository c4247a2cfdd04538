"""The C-ABI library loads and exports every entry point include/splatx_hip.h declares (no GPU use)."""
import ctypes
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "splatx_hip.h")
LIB = os.path.join(REPO, "splatx-metal_amd", "build", "libsplatx_hip.so")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(sxh_[a-z0-9_]+)\s*\(", txt)))


def test_header_is_pure_c():
    txt = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for bad in ("class ", "template", "namespace", "std::", "#include <hip", "torch"):
        assert bad not in txt.replace('extern "C"', "")


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail("library not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_library_exports_nothing_else():
    """The dynamic symbol table holds the header's entry points and nothing more: no C++ internals and no
    undeclared extern "C" function (the library is linked with a version script)."""
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", LIB], check=True, capture_output=True, text=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if ln.strip()})
    assert exported == declared(), (sorted(set(exported) - set(declared())), sorted(set(declared()) - set(exported)))


def test_abi_version_without_gpu():
    lib = ctypes.CDLL(LIB)
    lib.sxh_abi_version.restype = ctypes.c_int32
    assert lib.sxh_abi_version() == 1


def test_executor_switches_reject_a_null_executor_without_gpu():
    lib = ctypes.CDLL(LIB)
    lib.sxh_last_error.restype = ctypes.c_char_p
    for name in ("sxh_exec_set_graph", "sxh_exec_set_profiling", "sxh_exec_set_isect_order"):
        f = getattr(lib, name)
        f.restype = ctypes.c_int32
        f.argtypes = [ctypes.c_void_p, ctypes.c_int32]
        assert f(None, 1) != 0, name
        assert b"null executor" in lib.sxh_last_error(), name


def test_executor_sync_rejects_a_null_executor_without_gpu():
    lib = ctypes.CDLL(LIB)
    lib.sxh_last_error.restype = ctypes.c_char_p
    lib.sxh_exec_sync.restype = ctypes.c_int32
    lib.sxh_exec_sync.argtypes = [ctypes.c_void_p]
    assert lib.sxh_exec_sync(None) != 0
    assert b"null executor" in lib.sxh_last_error()
