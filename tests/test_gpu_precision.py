"""Activations with outliers INSIDE a 32-element unit: the case the batch-1
and int8 matrix-core kernels' representation handles worst.

Those kernels carry each 32-element unit of x as three int8 limbs under one
power-of-two scale picked from the unit's largest element, so a small element
next to a large one keeps about 2^-21 of the LARGE element's magnitude
(absolute), not 2^-24 of its own.  The MFMA path scales per 64-element chunk
the same way (hi/lo fp16, 22 bits).  These tests put such units on every M
path and both weight layouts and hold the outputs to the path's bar (relative
L2 <= 1e-5, per-row max-abs <= 1e-3 ||x||_2 max|W|) against the exact fp64
product AND against the reference's own fp32 CPU path (oracle/_ref).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from forge_amd import formats as F
from forge_amd import ops, synth
from helpers import assert_close
from test_gpu_parity import dev_weight

pytestmark = pytest.mark.gpu


def outlier_x(M, K, seed, kind):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    u = x.reshape(M, K // 32, 32)
    if kind == "spike":  # one element per unit at ~1e3 x the rest, at a varying slot
        pos = rng.integers(0, 32, size=(M, K // 32))
        sign = rng.choice([-1.0, 1.0], size=(M, K // 32))
        np.put_along_axis(u, pos[..., None], (1e3 * sign)[..., None].astype(np.float32), axis=2)
    elif kind == "mixed":  # every unit mixes 1e-3 and 1e3 magnitudes
        u[..., 0::2] *= np.float32(1e-3)
        u[..., 1::2] *= np.float32(1e3)
    elif kind == "sparse":  # units of tiny values between units of huge ones
        u[:, 0::2, :] *= np.float32(1e4)
        u[:, 1::2, :] *= np.float32(1e-4)
    elif kind == "edge":
        # unit maxima just below and at powers of two (the largest float under
        # 2^j rounds to the top of the representation's range: the 4-bit
        # formats' hex digits then carry a top digit of 4), both signs, with
        # the rest of the unit small and the unit's sign pattern varying
        j = rng.integers(-6, 7, size=(M, K // 32)).astype(np.float32)
        below = np.nextafter(np.float32(1.0), np.float32(0.0)) * np.exp2(j)
        pos = rng.integers(0, 32, size=(M, K // 32))
        sign = rng.choice([-1.0, 1.0], size=(M, K // 32)).astype(np.float32)
        u *= np.float32(0.01) * np.exp2(j)[..., None]
        val = np.where(rng.random((M, K // 32)) < 0.5, below, np.exp2(j)) * sign
        np.put_along_axis(u, pos[..., None], val[..., None].astype(np.float32), axis=2)
        np.put_along_axis(u, ((pos + 16) % 32)[..., None], (-val)[..., None].astype(np.float32),
                          axis=2)
    return np.ascontiguousarray(x)


def check(dtype, w, x, N, K, y, what):
    deq_max = float(np.max(np.abs(oracle.dequant(dtype, w[:2048], min(N, 2048), K))))
    assert_close(y, oracle.matmul_f64(dtype, x, w, N, K), x, np.array([deq_max]),
                 what + " vs exact")
    if oracle.have_ref():
        assert_close(y, oracle.ref_matmul(dtype, x, w, N, K, threads=16), x,
                     np.array([deq_max]), what + " vs reference")


SHAPES = [  # (format, N, K): the 7B and TinyLlama decode shapes, lm_head cut to 8192 rows
    (F.Q4_K, 18944, 3584), (F.Q6_K, 3584, 18944), (F.Q6_K, 8192, 3584),
    (F.Q4_0, 5632, 2048), (F.Q8_0, 2048, 5632), (F.Q4_1, 2048, 2048),
    (F.Q4_0, 3584, 18944), (F.Q4_1, 4096, 4096),
]


@pytest.mark.parametrize("kind", ["spike", "mixed", "sparse", "edge"])
@pytest.mark.parametrize("dtype,N,K", SHAPES, ids=lambda v: str(v))
def test_batch1_gguf_and_packed(dtype, N, K, kind):
    w = synth.make_weights(dtype, N, K, seed=77)
    x = outlier_x(1, K, 78, kind)
    W = dev_weight(dtype, w, N, K)
    xd = torch.from_numpy(x).cuda()
    name = f"{F.fmt(dtype).name} {N}x{K} {kind}"
    check(dtype, w, x, N, K, ops.matmul_transB(xd, W).cpu().numpy(), name + " gguf")
    check(dtype, w, x, N, K, ops.gemv_packed(xd, ops.pack_weights(W)).cpu().numpy().reshape(1, -1),
          name + " packed")


@pytest.mark.parametrize("kind", ["spike", "mixed"])
@pytest.mark.parametrize("M", [2, 3, 5, 8, 16])
@pytest.mark.parametrize("dtype", [F.Q4_K, F.Q6_K, F.Q8_0, F.Q4_0])
def test_small_batch_paths(dtype, M, kind):
    # cfg3-like rows (Q4_K M = 3 runs on the int8 matrix cores, M = 5..16 on
    # the one-pass fp16 MFMA kernel; M = 2 on the batch-1 kernel with two
    # tokens, which takes weights of 8 MB and more, so 4096 rows there)
    N, K = (4096 if M == 2 else 2048), 4096
    w = synth.make_weights(dtype, N, K, seed=80 + M)
    x = outlier_x(M, K, 90 + M, kind)
    y = ops.matmul_transB(torch.from_numpy(x).cuda(), dev_weight(dtype, w, N, K))
    check(dtype, w, x, N, K, y.cpu().numpy(), f"{F.fmt(dtype).name} M={M} {kind}")


@pytest.mark.parametrize("kind", ["spike", "mixed"])
@pytest.mark.parametrize("dtype", [F.Q8_0, F.Q4_0, F.Q4_1, F.Q4_K, F.Q5_0, F.Q5_1])
def test_prefill_path(dtype, kind):
    N, K, M = 1024, 4096, 64
    w = synth.make_weights(dtype, N, K, seed=95)
    x = outlier_x(M, K, 96, kind)
    y = ops.matmul_transB(torch.from_numpy(x).cuda(), dev_weight(dtype, w, N, K))
    check(dtype, w, x, N, K, y.cpu().numpy(), f"{F.fmt(dtype).name} M={M} {kind}")
