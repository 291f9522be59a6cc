"""CPU tests of the C ABI library: it loads, exports every declared symbol,
and validates arguments before touching a device (no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from forge_amd import _lib
from forge_amd import formats as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    syms = set()
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            syms |= set(re.findall(r"^\w[\w\s\*]*?\b(fq_\w+)\s*\(", text, re.M))
    return sorted(syms)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 8
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_block_info_matches_reference_traits():
    L = _lib.lib()
    for dt, f in F.FORMATS.items():
        e, b = ctypes.c_int(), ctypes.c_int()
        assert L.fq_block_info(dt, ctypes.byref(e), ctypes.byref(b)) == 0
        assert (e.value, b.value) == (f.block_elems, f.block_bytes)
    assert L.fq_block_info(0, None, None) == _lib.FQ_ERR_DTYPE  # FP32 is not a block format
    assert L.fq_block_info(10, None, None) == _lib.FQ_ERR_DTYPE  # Q2_K not implemented
    assert L.fq_block_info(16, None, None) == _lib.FQ_ERR_DTYPE  # IQ2_XXS not implemented


def test_status_strings():
    L = _lib.lib()
    for code in range(6):
        assert L.fq_status_str(code)
    assert L.fq_status_str(_lib.FQ_ERR_DTYPE) == b"unsupported quantized type"


@pytest.mark.parametrize("fn", ["fq_gemv", "fq_gemv_batch", "fq_matmul_prefill"])
def test_validation_needs_no_device(fn):
    L = _lib.lib()
    f = getattr(L, fn)
    one = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    if fn == "fq_gemv":
        assert f(99, one, one, one, 64, 4, None) == _lib.FQ_ERR_DTYPE
        assert f(F.Q4_0, one, one, one, 48, 4, None) == _lib.FQ_ERR_SHAPE  # K % 32
        assert f(F.Q4_K, one, one, one, 128, 4, None) == _lib.FQ_ERR_SHAPE  # K % 256
        assert f(F.Q4_0, None, one, one, 64, 4, None) == _lib.FQ_ERR_NULL
        assert f(F.Q4_0, one, one, one, 64, 0, None) == _lib.FQ_OK  # empty: no-op
    else:
        assert f(99, one, one, one, 2, 64, 4, None) == _lib.FQ_ERR_DTYPE
        assert f(F.Q8_0, one, one, one, 2, 40, 4, None) == _lib.FQ_ERR_SHAPE
        assert f(F.Q8_0, one, one, one, 0, 64, 4, None) == _lib.FQ_ERR_SHAPE
    if fn == "fq_gemv_batch":
        assert f(F.Q4_0, one, one, one, 33, 64, 4, None) == _lib.FQ_ERR_SHAPE  # M > 32


def test_matmul_transB_bias_validation():
    L = _lib.lib()
    one = ctypes.c_void_p(16)
    # 2-D bias shorter than M*N is rejected (apply_bias adds M*N elements)
    assert L.fq_matmul_transB(F.Q4_0, one, one, one, 2, 7, one, 2, 64, 4, None) == _lib.FQ_ERR_SHAPE
    assert L.fq_matmul_transB(F.Q4_0, one, one, one, 3, 8, one, 2, 64, 4, None) == _lib.FQ_ERR_SHAPE
    assert L.fq_dequant_rows(5, one, one, 1, 32, None) == _lib.FQ_ERR_DTYPE
    assert L.fq_dequant_rows(F.Q4_0, None, one, 1, 32, None) == _lib.FQ_ERR_NULL


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(ImportError):
        _lib.lib()


def test_packed_row_bytes():
    L = _lib.lib()
    # same bytes as the GGUF row (plus at most 15 bytes of row padding)
    for dt, f in F.FORMATS.items():
        if dt not in F.PACKED:  # GGUF layout only
            assert L.fq_packed_row_bytes(dt, 256) == 0
            one = ctypes.c_void_p(16)
            assert L.fq_pack_weights(dt, one, one, 1, 256, None) == _lib.FQ_ERR_DTYPE
            assert L.fq_gemv_packed(dt, one, one, None, 0, one, 256, 1, None) == _lib.FQ_ERR_DTYPE
            continue
        for K in (256, 2048, 3584, 18944):
            pb = L.fq_packed_row_bytes(dt, K)
            assert pb % 16 == 0
            assert f.row_bytes(K) <= pb <= f.row_bytes(K) + 15
    assert L.fq_packed_row_bytes(F.Q4_0, 96) == 0  # K must be a multiple of 256
    assert L.fq_packed_row_bytes(5, 256) == 0
