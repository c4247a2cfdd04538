"""The C++ KernelBackend adapter compiles against the reference's own interface header.

splatx-metal_amd/host/hip_kernel_backend.cpp implements splatx::KernelBackend
(Sources/SplatXCore/include/splatx/KernelBackend.h:396-509) over the C ABI; this checks, with the
reference tree's headers on the include path, that every override matches the reference's
signatures (a pure virtual left unimplemented or a mismatched override fails to compile).
"""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/Sources"


@pytest.mark.skipif(not os.path.isdir(REF) or shutil.which("g++") is None,
                    reason="reference tree or g++ not present (only the build container has them)")
def test_adapter_compiles_against_reference_header():
    src = os.path.join(REPO, "splatx-metal_amd", "host", "hip_kernel_backend.cpp")
    cmd = ["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
           "-I", os.path.join(REF, "SplatXCore", "include"), "-I", os.path.join(REF, "SplatXKernelSrc"),
           "-I", os.path.join(REPO, "include"), src]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
