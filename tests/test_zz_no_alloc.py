"""fq_matmul_transB_noalloc (fixed device workspace, no allocation) against
fq_matmul_transB on the same inputs: the same kernels and launch plan, so the
outputs are bit-identical.  Two calls in a row, the second smaller, on every
M path; a call beyond the fixed workspace is refused."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import _lib, synth
from forge_amd import formats as F

pytestmark = pytest.mark.gpu


def _call(fn, dtype, x, w, y, M, K, N, bias=None, stream=None):
    b = bias.data_ptr() if bias is not None else None
    nd = bias.dim() if bias is not None else 0
    bl = bias.numel() if bias is not None else 0
    return fn(dtype, x.data_ptr(), w.data_ptr(), b, nd, bl, y.data_ptr(), M, K, N, stream)


def _pair(dtype, M, K, N, seed, bias=False):
    L = _lib.lib()
    w = torch.from_numpy(synth.make_weights(dtype, N, K, seed).reshape(-1)).cuda()
    x = torch.from_numpy(synth.make_x(M, K, seed + 1)).cuda()
    b = torch.randn(M, N, device="cuda") if bias else None
    y0 = torch.full((M, N), float("nan"), device="cuda")
    y1 = torch.full((M, N), float("nan"), device="cuda")
    assert _call(L.fq_matmul_transB, dtype, x, w, y0, M, K, N, b) == 0
    assert _call(L.fq_matmul_transB_noalloc, dtype, x, w, y1, M, K, N, b) == 0
    torch.cuda.synchronize()
    a0, a1 = y0.cpu().numpy(), y1.cpu().numpy()
    assert np.isfinite(a0).all()
    np.testing.assert_array_equal(a1, a0, err_msg=f"{F.fmt(dtype).name} M={M} {N}x{K}")


@pytest.mark.parametrize("dtype", [F.Q4_K, F.Q8_0, F.Q6_K, F.Q4_0])
def test_noalloc_matches_two_calls(dtype):
    # the MFMA path with K-splits (workspace: token operands + partial slabs),
    # then a smaller call that reuses the same array
    _pair(dtype, 16, 4096, 3000, 40)
    _pair(dtype, 12, 2048, 700, 41, bias=True)


def test_noalloc_every_m_path():
    for M in (1, 2, 3, 5, 33):
        _pair(F.Q4_K, M, 2048, 640, 50 + M)
    # the batch-1 kernel with 1 .. 4 tokens (Q6_K always takes it) and the
    # one-pass small-batch kernel on 8 MB of Q4_K
    for M in (1, 2, 3, 4):
        _pair(F.Q6_K, M, 2048, 3000, 70 + M, bias=M == 3)
    _pair(F.Q4_K, 8, 4096, 4096, 80)
    # the batch-1 kernel with K split into slabs (two, then four tokens)
    _pair(F.Q6_K, 2, 18944, 3000, 90, bias=True)
    _pair(F.Q4_0, 4, 18944, 1500, 91)


def test_noalloc_prefill_and_limit():
    _pair(F.Q8_0, 512, 4096, 4096, 60)  # 42 MiB of the 64 MiB: 4 K-splits
    _pair(F.Q4_0, 64, 1024, 512, 61)
    _pair(F.Q6_K, 128, 2048, 1024, 62)  # the rows rewritten into the fixed array too
    L = _lib.lib()
    M, K, N = 1024, 16384, 256  # token operands alone need 272 MiB
    w = torch.zeros(N * (K // 32) * 34, dtype=torch.uint8, device="cuda")
    x = torch.zeros(M, K, device="cuda")
    y = torch.zeros(M, N, device="cuda")
    assert _call(L.fq_matmul_transB_noalloc, F.Q8_0, x, w, y, M, K, N) == _lib.FQ_ERR_WORKSPACE
