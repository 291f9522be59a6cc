"""Operator-level mirror of Forge's quantized matmul API on the HIP device.

``matmul_transB(a, b, bias)`` follows ``forge::ops::matmul_transB``
(include/forge/operator_matmul.h:9, src/operators/cpu/matmul.cpp:1134-1286):
same argument meaning (a: fp32 [M, K]; b: block-quantized weight of logical
shape [N, K]; optional bias [N] or [M, N]), same dispatch on M, a new fp32
[M, N] output, and the reference's error messages for the conditions it
rejects.  torch only provides device memory and the current stream here; all
arithmetic runs in libforge_q.so through the C ABI.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .formats import fmt


@dataclass
class QWeight:
    """A block-quantized weight: raw GGUF block bytes on the device.

    Mirrors a forge::Tensor whose dtype is a block format and whose shape is
    [N, K] in elements (include/forge/tensor.h:11-68); ``data`` holds
    N * row_bytes(K) bytes, rows contiguous.
    """
    data: torch.Tensor  # uint8, contiguous, on the device
    dtype: int
    N: int
    K: int

    @property
    def shape(self):
        return (self.N, self.K)

    def ndim(self) -> int:
        return 2

    @classmethod
    def from_numpy(cls, blocks, dtype: int, N: int, K: int, device="cuda"):
        t = torch.from_numpy(blocks.reshape(-1)).to(device)
        return cls(t, int(dtype), int(N), int(K))


def _stream_ptr(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def matmul_transB(a: torch.Tensor, b: QWeight, bias: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = a[M, K] @ dequant(b)[N, K]^T (+ bias), on the device."""
    if a.dim() != 2 or b.ndim() != 2:
        raise RuntimeError("matmul_transB expects 2D tensors")
    M, K = a.shape
    if K != b.K:
        raise RuntimeError(f"matmul_transB dimension mismatch: K={K} K2={b.K} "
                           f"b_shape=[{b.N},{b.K}]")
    if a.dtype != torch.float32 or not a.is_cuda or not a.is_contiguous():
        raise RuntimeError("matmul_transB: input must be a contiguous fp32 device tensor")
    out = torch.empty((M, b.N), dtype=torch.float32, device=a.device)
    bias_ptr, bias_ndim, bias_len = None, 0, 0
    if bias is not None:
        bias = bias.to(device=a.device, dtype=torch.float32).contiguous()
        bias_ptr, bias_ndim, bias_len = bias.data_ptr(), bias.dim(), bias.numel()
    st = _lib.lib().fq_matmul_transB(b.dtype, a.data_ptr(), b.data.data_ptr(), bias_ptr,
                                     bias_ndim, bias_len, out.data_ptr(), M, K, b.N,
                                     _stream_ptr(a))
    if st == _lib.FQ_ERR_DTYPE:
        raise RuntimeError("Unsupported quantized type in matmul_transB CUDA")
    _lib.check(st, "matmul_transB")
    return out


def gemv(x: torch.Tensor, b: QWeight) -> torch.Tensor:
    """Batch-1 GEMV through fq_gemv (x: [K] or [1, K])."""
    xv = x.reshape(-1)
    y = torch.empty((b.N,), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_gemv(b.dtype, xv.data_ptr(), b.data.data_ptr(), y.data_ptr(),
                                  b.K, b.N, _stream_ptr(x)), "fq_gemv")
    return y


def gemv_batch(x: torch.Tensor, b: QWeight) -> torch.Tensor:
    M = x.shape[0]
    y = torch.empty((M, b.N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_gemv_batch(b.dtype, x.data_ptr(), b.data.data_ptr(), y.data_ptr(),
                                        M, b.K, b.N, _stream_ptr(x)), "fq_gemv_batch")
    return y


def matmul_prefill(x: torch.Tensor, b: QWeight) -> torch.Tensor:
    M = x.shape[0]
    y = torch.empty((M, b.N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_matmul_prefill(b.dtype, x.data_ptr(), b.data.data_ptr(),
                                            y.data_ptr(), M, b.K, b.N, _stream_ptr(x)),
               "fq_matmul_prefill")
    return y


def dequantize_weight(b: QWeight) -> torch.Tensor:
    """fp32 [N, K] dequantized copy, bit-identical to the reference's rows."""
    out = torch.empty((b.N, b.K), dtype=torch.float32, device=b.data.device)
    _lib.check(_lib.lib().fq_dequant_rows(b.dtype, b.data.data_ptr(), out.data_ptr(), b.N, b.K,
                                          _stream_ptr(b.data)), "fq_dequant_rows")
    return out


def row_bytes(dtype: int, K: int) -> int:
    return fmt(dtype).row_bytes(K)


@dataclass
class PackedWeight:
    """A block-quantized weight in the aligned device layout (fq_pack_weights).

    Same logical [N, K] matrix and identical dequantized values as the GGUF
    bytes it was made from; rows are packed_row_bytes(K) apart.
    """
    data: torch.Tensor  # uint8, 16-byte aligned, on the device
    dtype: int
    N: int
    K: int


def packed_row_bytes(dtype: int, K: int) -> int:
    return int(_lib.lib().fq_packed_row_bytes(int(dtype), int(K)))


def pack_weights(b: QWeight) -> PackedWeight:
    rb = packed_row_bytes(b.dtype, b.K)
    if rb == 0:
        raise RuntimeError(f"no packed layout for dtype {b.dtype} with K={b.K}")
    out = torch.empty(b.N * rb, dtype=torch.uint8, device=b.data.device)
    _lib.check(_lib.lib().fq_pack_weights(b.dtype, b.data.data_ptr(), out.data_ptr(), b.N, b.K,
                                          _stream_ptr(b.data)), "fq_pack_weights")
    return PackedWeight(out, b.dtype, b.N, b.K)


def unpack_weights(p: PackedWeight) -> QWeight:
    out = torch.empty(fmt(p.dtype).matrix_bytes(p.N, p.K), dtype=torch.uint8,
                      device=p.data.device)
    _lib.check(_lib.lib().fq_unpack_weights(p.dtype, p.data.data_ptr(), out.data_ptr(), p.N, p.K,
                                            _stream_ptr(p.data)), "fq_unpack_weights")
    return QWeight(out, p.dtype, p.N, p.K)


def gemv_packed(x: torch.Tensor, p: PackedWeight, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Batch-1 GEMV over packed weights (x: [K] or [1, K]); returns [N]."""
    xv = x.reshape(-1)
    if xv.numel() != p.K:
        raise RuntimeError(f"gemv_packed dimension mismatch: K={xv.numel()} K2={p.K}")
    y = torch.empty((p.N,), dtype=torch.float32, device=x.device)
    bptr, blen = None, 0
    if bias is not None:
        bias = bias.to(device=x.device, dtype=torch.float32).contiguous()
        bptr, blen = bias.data_ptr(), bias.numel()
    _lib.check(_lib.lib().fq_gemv_packed(p.dtype, xv.data_ptr(), p.data.data_ptr(), bptr, blen,
                                         y.data_ptr(), p.K, p.N, _stream_ptr(x)), "fq_gemv_packed")
    return y


def ffn_up_fused(x: torch.Tensor, w_gate: QWeight, w_up: QWeight) -> torch.Tensor:
    """silu(x @ w_gate^T) * (x @ w_up^T) for GGUF weights, any M; mirrors
    ops::ffn_up_fused (src/operators/cpu/matmul.cpp:1472-1533)."""
    if x.dim() != 2:
        raise RuntimeError("ffn_up_fused expects a 2D input")
    M, K = x.shape
    if (w_gate.dtype, w_gate.N, w_gate.K) != (w_up.dtype, w_up.N, w_up.K):
        raise RuntimeError("ffn_up_fused: gate and up weights differ in dtype or shape")
    if K != w_gate.K:
        raise RuntimeError(f"ffn_up_fused dimension mismatch: K={K} K2={w_gate.K}")
    x = x.contiguous()
    y = torch.empty((M, w_gate.N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_ffn_up_fused(w_gate.dtype, x.data_ptr(), w_gate.data.data_ptr(),
                                          w_up.data.data_ptr(), y.data_ptr(), M, K, w_gate.N,
                                          _stream_ptr(x)), "fq_ffn_up_fused")
    return y


def ffn_up_fused_packed(x: torch.Tensor, w_gate: PackedWeight, w_up: PackedWeight) -> torch.Tensor:
    """Batch-1 fused gate/up over packed weights (x: [K] or [1, K]); returns [N]."""
    xv = x.reshape(-1)
    if (w_gate.dtype, w_gate.N, w_gate.K) != (w_up.dtype, w_up.N, w_up.K):
        raise RuntimeError("ffn_up_fused: gate and up weights differ in dtype or shape")
    if xv.numel() != w_gate.K:
        raise RuntimeError(f"ffn_up_fused dimension mismatch: K={xv.numel()} K2={w_gate.K}")
    y = torch.empty((w_gate.N,), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_ffn_up_fused_packed(w_gate.dtype, xv.data_ptr(),
                                                 w_gate.data.data_ptr(), w_up.data.data_ptr(),
                                                 y.data_ptr(), w_gate.K, w_gate.N,
                                                 _stream_ptr(x)), "fq_ffn_up_fused_packed")
    return y


def _same_k(name, K, *ws):
    for w in ws:
        if w.K != K:
            raise RuntimeError(f"{name} dimension mismatch: K={K} K2={w.K}")
    if len({w.dtype for w in ws}) != 1:
        raise RuntimeError(f"{name}: weights differ in dtype")


def fused_qkv(x: torch.Tensor, wq: QWeight, wk: QWeight, wv: QWeight) -> torch.Tensor:
    """[x Wq^T | x Wk^T | x Wv^T] for GGUF weights, any M; mirrors
    matmul_transB_fused_qkv_q4_0 / _q4_k (src/operators/cpu/matmul.cpp:1535-1600)."""
    if x.dim() != 2:
        raise RuntimeError("fused_qkv expects a 2D input")
    M, K = x.shape
    _same_k("fused_qkv", K, wq, wk, wv)
    x = x.contiguous()
    y = torch.empty((M, wq.N + wk.N + wv.N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_fused_qkv(wq.dtype, x.data_ptr(), wq.data.data_ptr(),
                                       wk.data.data_ptr(), wv.data.data_ptr(), y.data_ptr(), M, K,
                                       wq.N, wk.N, wv.N, _stream_ptr(x)), "fq_fused_qkv")
    return y


def fused_qkv_packed(x: torch.Tensor, wq: PackedWeight, wk: PackedWeight,
                     wv: PackedWeight) -> torch.Tensor:
    """Batch-1 fused QKV over packed weights (x: [K] or [1, K]); returns [Nq + Nk + Nv]."""
    xv = x.reshape(-1)
    _same_k("fused_qkv", xv.numel(), wq, wk, wv)
    y = torch.empty((wq.N + wk.N + wv.N,), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_fused_qkv_packed(wq.dtype, xv.data_ptr(), wq.data.data_ptr(),
                                              wk.data.data_ptr(), wv.data.data_ptr(),
                                              y.data_ptr(), wq.K, wq.N, wk.N, wv.N,
                                              _stream_ptr(x)), "fq_fused_qkv_packed")
    return y


def ffn_down_residual(x: torch.Tensor, w: QWeight, residual: torch.Tensor) -> torch.Tensor:
    """x W^T + residual for GGUF weights, any M; mirrors
    matmul_transB_fused_ffn_down_residual_q4_0 / _q6_k (matmul.cpp:1601-1637)."""
    if x.dim() != 2 or residual.dim() != 2:
        raise RuntimeError("ffn_down_residual expects 2D tensors")
    M, K = x.shape
    _same_k("ffn_down_residual", K, w)
    if tuple(residual.shape) != (M, w.N):
        raise RuntimeError("ffn_down_residual: residual shape mismatch")
    x = x.contiguous()
    r = residual.to(device=x.device, dtype=torch.float32).contiguous()
    y = torch.empty((M, w.N), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_ffn_down_residual(w.dtype, x.data_ptr(), w.data.data_ptr(),
                                               r.data_ptr(), y.data_ptr(), M, K, w.N,
                                               _stream_ptr(x)), "fq_ffn_down_residual")
    return y


def ffn_down_residual_packed(x: torch.Tensor, w: PackedWeight,
                             residual: torch.Tensor) -> torch.Tensor:
    """Batch-1 x W^T + residual over packed weights; returns [N]."""
    xv = x.reshape(-1)
    _same_k("ffn_down_residual", xv.numel(), w)
    r = residual.reshape(-1).to(device=x.device, dtype=torch.float32).contiguous()
    if r.numel() != w.N:
        raise RuntimeError("ffn_down_residual: residual shape mismatch")
    y = torch.empty((w.N,), dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().fq_ffn_down_residual_packed(w.dtype, xv.data_ptr(), w.data.data_ptr(),
                                                      r.data_ptr(), y.data_ptr(), w.K, w.N,
                                                      _stream_ptr(x)),
               "fq_ffn_down_residual_packed")
    return y
