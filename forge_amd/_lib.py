"""ctypes binding of the C ABI in include/forge_q.h (libforge_q.so).

The library is loaded from this package directory only.  There is no
fallback: if the shared library is missing the import of ``lib()`` raises,
so no caller can silently run anything but the HIP path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libforge_q.so")

FQ_OK = 0
FQ_ERR_DTYPE = 1
FQ_ERR_SHAPE = 2
FQ_ERR_NULL = 3
FQ_ERR_HIP = 4
FQ_ERR_NO_DEVICE = 5
FQ_ERR_ALIGN = 6
FQ_ERR_WORKSPACE = 7

# Every symbol include/forge_q.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32
_L = ctypes.c_int64
SIGNATURES = {
    "fq_block_info": (_I, [_U, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "fq_status_str": (ctypes.c_char_p, [_I]),
    "fq_last_hip_error": (_I, []),
    "fq_gemv": (_I, [_U, _P, _P, _P, _I, _I, _P]),
    "fq_gemv_batch": (_I, [_U, _P, _P, _P, _I, _I, _I, _P]),
    "fq_matmul_prefill": (_I, [_U, _P, _P, _P, _I, _I, _I, _P]),
    "fq_matmul_transB": (_I, [_U, _P, _P, _P, _I, _L, _P, _I, _I, _I, _P]),
    "fq_dequant_rows": (_I, [_U, _P, _P, _I, _I, _P]),
    "fq_packed_row_bytes": (_L, [_U, _I]),
    "fq_pack_weights": (_I, [_U, _P, _P, _I, _I, _P]),
    "fq_unpack_weights": (_I, [_U, _P, _P, _I, _I, _P]),
    "fq_gemv_packed": (_I, [_U, _P, _P, _P, _L, _P, _I, _I, _P]),
    "fq_ffn_up_fused": (_I, [_U, _P, _P, _P, _P, _I, _I, _I, _P]),
    "fq_ffn_up_fused_packed": (_I, [_U, _P, _P, _P, _P, _I, _I, _P]),
    "fq_fused_qkv": (_I, [_U, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fq_fused_qkv_packed": (_I, [_U, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fq_ffn_down_residual": (_I, [_U, _P, _P, _P, _P, _I, _I, _I, _P]),
    "fq_ffn_down_residual_packed": (_I, [_U, _P, _P, _P, _P, _I, _I, _P]),
    "fq_matmul_transB_noalloc": (_I, [_U, _P, _P, _P, _I, _L, _P, _I, _I, _I, _P]),
    "fq_reserve_workspace": (_I, [_I, _I, _I, _P]),
    "fq_release_workspace": (_I, [_P]),
}

_lib = None


class FqError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = lib().fq_status_str(status).decode()
        if status == FQ_ERR_HIP:
            msg += f" (hipError {lib().fq_last_hip_error()})"
        super().__init__(f"{what}: {msg}")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m forge_amd.build` "
                "(there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, what: str) -> None:
    if status != FQ_OK:
        raise FqError(status, what)
