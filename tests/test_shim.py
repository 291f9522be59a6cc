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
HIP_INCLUDE = "/opt/rocm/include"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF_INCLUDE, "forge")),
                    reason="reference headers not present")
@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_shim_compiles_against_reference_headers():
    # the shim includes the HIP runtime API header for its strided device copies
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                        "-D__HIP_PLATFORM_AMD__", "-isystem", HIP_INCLUDE,
                        "-I", REF_INCLUDE, "-I", os.path.join(ROOT, "include"), SHIM],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF_INCLUDE, "forge")),
                    reason="reference headers not present")
def test_shim_covers_every_device_operator():
    """Every operator of operator_matmul.h that the engines call on a device
    tensor has a device branch in the shim."""
    src = open(SHIM).read()
    for op in ("matmul_transB", "dequantize_weight", "ffn_up_fused", "matmul_transB_dual",
               "matmul_transB_fused_qkv_q4_0", "matmul_transB_fused_qkv_q4_k",
               "matmul_transB_fused_ffn_up_q4_0", "matmul_transB_fused_ffn_up_q4_k",
               "matmul_transB_fused_ffn_down_residual_q4_0",
               "matmul_transB_fused_ffn_down_residual_q6_k"):
        assert f"TensorPtr {op}_device(" in src or f"void {op}_device(" in src, op
        assert op in open(os.path.join(REF_INCLUDE, "forge", "operator_matmul.h")).read(), op
