"""Seeded synthetic block matrices and activations.

Distributions follow the benchmark definition of the hot path: fp16 scales
drawn |N(0, 0.02)| and rounded to nearest-even fp16; Q4_0/Q4_K nibbles and
Q6_K ql/qh bytes uniform; Q8_0 values uniform in -127..127; Q6_K sub-scales
uniform int8; activations N(0, 1) fp32.  numpy's PCG64 generator makes the
bytes identical on every host for the same seed.

Block layouts (byte offsets inside one block) are the on-disk GGUF ones the
reference reads (src/operators/cpu/matmul.cpp:73-377):
  Q4_0  18 B: d f16 @0, qs[16] @2
  Q4_1  20 B: d f16 @0, m f16 @2, qs[16] @4
  Q8_0  34 B: d f16 @0, qs int8[32] @2
  Q4_K 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
  Q6_K 210 B: ql[128] @0, qh[64] @128, sc int8[16] @192, d f16 @208
  Q5_0  22 B: d f16 @0, qh u32 @2, qs[16] @6
  Q5_1  24 B: d f16 @0, m f16 @2, qh u32 @4, qs[16] @8
  Q3_K 110 B: hmask[32] @0, qs[64] @32, scales[12] @96, d f16 @108
  Q5_K 176 B: d f16 @0, dmin f16 @2, scales[12] @4, qh[32] @16, qs[128] @48
  IQ4_NL 18 B: d f16 @0, qs[16] @2
The quant payload bytes of the formats outside the benchmark configs are
uniform, like Q4_K's.
"""
from __future__ import annotations

import numpy as np

from .formats import IQ4_NL, Q3_K, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1, Q5_K, Q6_K, Q8_0, fmt

SCALE_SIGMA = 0.02


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    """fp16 (round to nearest even) as a [..., 2] little-endian byte array."""
    return v.astype(np.float16).view(np.uint8).reshape(*v.shape, 2)


def _scales(rng: np.random.Generator, shape) -> np.ndarray:
    return np.abs(rng.normal(0.0, SCALE_SIGMA, size=shape)).astype(np.float32)


def make_weights(dtype, N: int, K: int, seed: int) -> np.ndarray:
    """Return a uint8 array [N, row_bytes] of seeded random blocks."""
    f = fmt(dtype)
    if K % f.block_elems:
        raise ValueError(f"K={K} must be a multiple of {f.block_elems} for {f.name}")
    nb = K // f.block_elems
    rng = np.random.default_rng(seed)
    blk = np.empty((N, nb, f.block_bytes), dtype=np.uint8)
    if f.dtype == Q4_0:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:18] = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    elif f.dtype == Q4_1:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:4] = _f16_bytes(rng.normal(0.0, SCALE_SIGMA * 8, size=(N, nb)).astype(np.float32))
        blk[..., 4:20] = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    elif f.dtype == Q8_0:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:34] = rng.integers(-127, 128, size=(N, nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    elif f.dtype == Q4_K:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:4] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 4:144] = rng.integers(0, 256, size=(N, nb, 140), dtype=np.uint8)
    elif f.dtype == Q6_K:
        blk[..., 0:208] = rng.integers(0, 256, size=(N, nb, 208), dtype=np.uint8)
        blk[..., 208:210] = _f16_bytes(_scales(rng, (N, nb)))
    elif f.dtype in (Q5_0, IQ4_NL):
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:] = rng.integers(0, 256, size=(N, nb, f.block_bytes - 2), dtype=np.uint8)
    elif f.dtype == Q5_1:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:4] = _f16_bytes(rng.normal(0.0, SCALE_SIGMA * 8, size=(N, nb)).astype(np.float32))
        blk[..., 4:24] = rng.integers(0, 256, size=(N, nb, 20), dtype=np.uint8)
    elif f.dtype == Q3_K:
        blk[..., 0:108] = rng.integers(0, 256, size=(N, nb, 108), dtype=np.uint8)
        blk[..., 108:110] = _f16_bytes(_scales(rng, (N, nb)))
    elif f.dtype == Q5_K:
        blk[..., 0:2] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 2:4] = _f16_bytes(_scales(rng, (N, nb)))
        blk[..., 4:176] = rng.integers(0, 256, size=(N, nb, 172), dtype=np.uint8)
    else:  # pragma: no cover - fmt() already rejected it
        raise ValueError(dtype)
    return blk.reshape(N, nb * f.block_bytes)


def make_x(M: int, K: int, seed: int) -> np.ndarray:
    """fp32 activations [M, K] drawn N(0, 1)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal(size=(M, K), dtype=np.float32)
