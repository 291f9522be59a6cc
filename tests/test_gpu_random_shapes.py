"""Seeded random shapes through ops.matmul_transB against the f64 oracle:
every format, M from 1 to 100 (every dispatch path), N >= 16 with tails, K
any whole number of blocks up to 8192, no bias / row bias / full bias; and
40 shapes of 4 MB and more in the five batch-1 formats (N up to 12289, K up
to 12288).
Bars as in test_gpu_parity.py.

The rel-L2 bar is a ratio to |y|, so it is only asserted on outputs of 16
or more rows: on a single row whose dot product cancels, |y| can be orders
below ||x|| max|w| and the ratio exceeds 1e-5 for the reference's own fp32
CPU path as well (see the numerics notes); the max-abs bar holds there."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from forge_amd import formats as F
from forge_amd import ops, synth
from helpers import assert_close

pytestmark = pytest.mark.gpu

CASES = 160


def _cases():
    rng = np.random.default_rng(20260301)
    out = []
    allf = sorted(F.FORMATS)
    while len(out) < CASES:
        dt = int(rng.choice(allf))
        be = F.fmt(dt).block_elems
        M = int(rng.choice([1, 1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 32, 33, 64, 100]))
        N = int(rng.choice([16, 17, 100, 128, 129, 300, 1000]))
        K = be * int(rng.integers(1, max(2, 8192 // be)))
        if M * N * K > 1.5e8:
            continue
        out.append((dt, M, N, K, int(rng.integers(1 << 30)), float(rng.random())))
    return out


def _large_cases():
    # matrices of 4 MB and more: the K-sliced batch-1 kernel with 1 .. 4
    # tokens (partial K-slices, odd row counts), the band kernel and the
    # prefill kernel on larger row counts
    rng = np.random.default_rng(20261202)
    out = []
    fives = [F.Q4_0, F.Q4_1, F.Q8_0, F.Q4_K, F.Q6_K]
    while len(out) < 40:
        dt = int(rng.choice(fives))
        be = F.fmt(dt).block_elems
        M = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 8, 16, 33, 64]))
        N = int(rng.choice([2049, 4097, 6001, 9000, 12289]))
        K = be * int(rng.integers(max(1, 2048 // be), 12288 // be))
        if M * N * K > 2.0e8 or N * (K // be) * F.fmt(dt).block_bytes < (4 << 20):
            continue
        out.append((dt, M, N, K, int(rng.integers(1 << 30)), float(rng.random())))
    return out


@pytest.mark.parametrize("dt,M,N,K,seed,r", _cases() + _large_cases())
def test_random_shape(dt, M, N, K, seed, r):
    w = synth.make_weights(dt, N, K, seed=seed)
    x = synth.make_x(M, K, seed=seed + 1)
    bias = None
    if r < 0.2:
        bias = torch.from_numpy(synth.make_x(1, N, seed + 2).reshape(N))
    elif r < 0.3:
        bias = torch.from_numpy(synth.make_x(M, N, seed + 3))
    W = ops.QWeight.from_numpy(w, dt, N, K, device="cuda")
    y = ops.matmul_transB(torch.from_numpy(x).cuda(),
                          W, bias.cuda() if bias is not None else None).cpu().numpy()
    y64 = oracle.matmul_f64(dt, x, w, N, K)
    if bias is not None:
        y64 = y64 + bias.numpy().astype(np.float64)
    deq = float(np.max(np.abs(oracle.dequant(dt, w, N, K))))
    assert_close(y, y64, x, np.array([deq]), f"{F.fmt(dt).name} M={M} N={N} K={K}")


def _small_batch_cases():
    rng = np.random.default_rng(20261203)
    out = []
    allf = sorted(F.FORMATS)
    while len(out) < 80:
        dt = int(rng.choice(allf))
        be = F.fmt(dt).block_elems
        M = int(rng.choice([2, 3, 4, 5, 6, 8, 9, 12, 16]))
        N = int(rng.choice([int(rng.integers(1, 3000)), int(rng.integers(3000, 20000))]))
        K = (256 * int(rng.integers(1, 75)) if rng.random() < 0.8
             else be * int(rng.integers(1, 19000 // be)))
        if M * N * K > 4e8 or N * K > 1.2e8:
            continue
        out.append((dt, M, N, K, int(rng.integers(1 << 30)), float(rng.random()),
                    int(rng.choice([0, 0, 2, 16]))))
    return out


@pytest.mark.parametrize("dt,M,N,K,seed,r,off", _small_batch_cases())
def test_random_small_batch(dt, M, N, K, seed, r, off):
    from test_gpu_parity import dev_weight
    w = synth.make_weights(dt, N, K, seed=seed)
    x = synth.make_x(M, K, seed=seed + 1)
    bias = torch.from_numpy(synth.make_x(1, N, seed + 2).reshape(N)) if r < 0.3 else None
    y = ops.matmul_transB(torch.from_numpy(x).cuda(), dev_weight(dt, w, N, K, off),
                          bias.cuda() if bias is not None else None).cpu().numpy()
    y64 = oracle.matmul_f64(dt, x, w, N, K)
    if bias is not None:
        y64 = y64 + bias.numpy().astype(np.float64)
    deq = float(np.max(np.abs(oracle.dequant(dt, w, min(N, 4096), K))))
    assert_close(y, y64, x, np.array([deq]),
                 f"{F.fmt(dt).name} M={M} N={N} K={K} offset {off}")
