"""The reference-side shim (forge_amd/shim/matmul_hip.cpp) compiles against
the reference's own headers (include/forge/operator_matmul.h, tensor.h) and
this repository's C ABI header.  Skipped where the reference tree is absent
(it is read as headers only; nothing of it is built or run)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/include"
SHIM = os.path.join(ROOT, "forge_amd", "shim", "matmul_hip.cpp")


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF_INCLUDE, "forge")),
                    reason="reference headers not present")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_shim_compiles_against_reference_headers():
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                        "-I", REF_INCLUDE, "-I", os.path.join(ROOT, "include"), SHIM],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
