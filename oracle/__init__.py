"""Checkers for the HIP path (test infrastructure only).

``load_oracle()`` loads this directory's C restatement (libfq_oracle.so);
``load_ref()`` loads oracle/_ref/libforge_ref.so, the reference's own CPU
operator path compiled from its sources.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use these.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libfq_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libforge_ref.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32


def build(ref: bool = False) -> None:
    import subprocess
    targets = ["all"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def load_oracle() -> ctypes.CDLL:
    if not os.path.exists(ORACLE_SO):
        build()
    L = ctypes.CDLL(ORACLE_SO)
    L.fqo_fp16_to_fp32.restype = ctypes.c_float
    L.fqo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
    L.fqo_dequant_rows.argtypes = [_U, _P, _P, _I, _I]
    L.fqo_matmul_transB_f64.argtypes = [_U, _P, _P, _P, _I, _I, _I]
    L.fqo_matmul_transB_f32.argtypes = [_U, _P, _P, _P, _I, _I, _I]
    L.fqo_block_info.argtypes = [_U, ctypes.POINTER(_I), ctypes.POINTER(_I)]
    return L


def have_ref() -> bool:
    return os.path.exists(REF_SO)


def load_ref() -> ctypes.CDLL:
    L = ctypes.CDLL(REF_SO)
    L.fqr_dequant_rows.argtypes = [_U, _P, _P, _I, _I]
    L.fqr_matmul_transB.argtypes = [_U, _P, _P, _P, _I, _I, _I, _I]
    L.fqr_ffn_up_fused.argtypes = [_U, _P, _P, _P, _P, _I, _I, _I, _I]
    return L


def _p(a: np.ndarray):
    return a.ctypes.data_as(_P)


def dequant(dtype: int, w: np.ndarray, N: int, K: int) -> np.ndarray:
    out = np.empty((N, K), np.float32)
    w = np.ascontiguousarray(w)
    if load_oracle().fqo_dequant_rows(dtype, _p(w), _p(out), N, K) != 0:
        raise ValueError("oracle dequant rejected the input")
    return out


def matmul_f64(dtype: int, x: np.ndarray, w: np.ndarray, N: int, K: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.empty((M, N), np.float64)
    w = np.ascontiguousarray(w)
    if load_oracle().fqo_matmul_transB_f64(dtype, _p(x), _p(w), _p(y), M, K, N) != 0:
        raise ValueError("oracle matmul rejected the input")
    return y


def matmul_f32(dtype: int, x: np.ndarray, w: np.ndarray, N: int, K: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    w = np.ascontiguousarray(w)
    if load_oracle().fqo_matmul_transB_f32(dtype, _p(x), _p(w), _p(y), M, K, N) != 0:
        raise ValueError("oracle matmul rejected the input")
    return y


def ref_matmul(dtype: int, x: np.ndarray, w: np.ndarray, N: int, K: int,
               threads: int = 0) -> np.ndarray:
    """The reference's own ops::matmul_transB on the CPU (AVX2 + OpenMP)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    w = np.ascontiguousarray(w)
    rc = load_ref().fqr_matmul_transB(dtype, _p(x), _p(w), _p(y), M, K, N, threads)
    if rc != 0:
        raise RuntimeError(f"reference matmul_transB failed ({rc})")
    return y
