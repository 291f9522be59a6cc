"""The per-stream workspace of the M > 1 matrix-core path: reserved up front
it lets a call be captured into a HIP graph (every replay matches the eager
result); during capture a call that would have to grow it fails with
FQ_ERR_WORKSPACE instead of allocating."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import _lib, synth
from forge_amd import formats as F

pytestmark = pytest.mark.gpu


def _mm(L, dtype, x, w, y, M, K, N, stream):
    return L.fq_matmul_transB(dtype, x.data_ptr(), w.data_ptr(), None, 0, 0, y.data_ptr(), M, K,
                              N, stream)


def test_reserved_workspace_graph_replays():
    L = _lib.lib()
    dtype, M, K, N = F.Q4_K, 16, 4096, 2000  # MFMA path with K-splits
    w = torch.from_numpy(synth.make_weights(dtype, N, K, 31).reshape(-1)).cuda()
    x = torch.from_numpy(synth.make_x(M, K, 32)).cuda()
    side = torch.cuda.Stream()
    y_eager = torch.empty(M, N, device="cuda")
    y_graph = torch.empty(M, N, device="cuda")
    with torch.cuda.stream(side):
        assert L.fq_reserve_workspace(M, K, N, side.cuda_stream) == 0
        assert _mm(L, dtype, x, w, y_eager, M, K, N, side.cuda_stream) == 0
    torch.cuda.synchronize()
    ref = y_eager.cpu().numpy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        st = _mm(L, dtype, x, w, y_graph, M, K, N, side.cuda_stream)
    assert st == 0
    for r in range(3):
        y_graph.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y_graph.cpu().numpy(), ref, err_msg=f"replay {r}")
        # eager work on the same workspace between replays
        with torch.cuda.stream(side):
            assert _mm(L, dtype, x * 2, w, y_eager, M, K, N, side.cuda_stream) == 0
        torch.cuda.synchronize()
    del g
    assert L.fq_release_workspace(side.cuda_stream) == 0


def test_growth_under_capture_is_refused():
    L = _lib.lib()
    dtype, M, K, N = F.Q8_0, 24, 2048, 1024
    w = torch.from_numpy(synth.make_weights(dtype, N, K, 33).reshape(-1)).cuda()
    x = torch.from_numpy(synth.make_x(M, K, 34)).cuda()
    y = torch.empty(M, N, device="cuda")
    side = torch.cuda.Stream()  # a fresh stream: no workspace yet
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        st = _mm(L, dtype, x, w, y, M, K, N, side.cuda_stream)
    assert st == _lib.FQ_ERR_WORKSPACE
    assert b"fq_reserve_workspace" in L.fq_status_str(st)
    del g
    # outside capture the same call grows the workspace and runs
    with torch.cuda.stream(side):
        assert _mm(L, dtype, x, w, y, M, K, N, side.cuda_stream) == 0
    torch.cuda.synchronize()
    assert np.isfinite(y.cpu().numpy()).all()


@pytest.mark.parametrize("dtype,M,K,N", [(F.Q8_0, 40, 4096, 256), (F.Q4_0, 512, 1280, 4096),
                                         (F.Q4_K, 16, 4096, 2000), (F.Q8_0, 8, 2048, 3000),
                                         (F.Q6_K, 96, 2048, 1500), (F.Q4_K, 8, 18944, 3584),
                                         (F.Q6_K, 2, 18944, 3584), (F.Q4_0, 3, 18944, 3584),
                                         (F.Q6_K, 8, 18944, 3584), (F.Q8_0, 6, 18944, 3584),
                                         (F.Q4_1, 16, 4096, 1000), (F.Q5_K, 2, 18944, 3584)])
def test_reserve_then_capture_first(dtype, M, K, N):
    # fq_reserve_workspace alone (no eager call first) must cover the call's
    # kernel choice: the prefill kernel (Q8_0 / Q4_0, up to 16 K-splits; Q6_K
    # with its rewritten rows), the MMQ and small-batch paths (the band
    # kernel with K split over four slabs at 3584 x 18944, on Q4_K, Q4_0,
    # Q4_1, Q8_0 and Q6_K) and the batch-1 kernel over two or three tokens
    # with K split into slabs.  Three
    # replays, each checked against the eager call, with eager work between
    # them
    L = _lib.lib()
    w = torch.from_numpy(synth.make_weights(dtype, N, K, 41).reshape(-1)).cuda()
    x = torch.from_numpy(synth.make_x(M, K, 42)).cuda()
    y_graph = torch.empty(M, N, device="cuda")
    y_eager = torch.empty(M, N, device="cuda")
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    assert L.fq_reserve_workspace(M, K, N, side.cuda_stream) == 0
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        st = _mm(L, dtype, x, w, y_graph, M, K, N, side.cuda_stream)
    assert st == 0, L.fq_status_str(st)
    with torch.cuda.stream(side):
        assert _mm(L, dtype, x, w, y_eager, M, K, N, side.cuda_stream) == 0
    torch.cuda.synchronize()
    ref = y_eager.cpu().numpy()
    for _ in range(3):
        y_graph.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y_graph.cpu().numpy(), ref)
        with torch.cuda.stream(side):
            assert _mm(L, dtype, x, w, y_eager, M, K, N, side.cuda_stream) == 0
        torch.cuda.synchronize()
    del g
    assert L.fq_release_workspace(side.cuda_stream) == 0


def test_fused_qkv_small_batch_graph_replays():
    # fused QKV at 8 tokens under capture after fq_reserve_workspace: the
    # band kernel's shared token operands need slot 0 at its largest band
    # size, which the reserve covers; every replay equals the eager call
    from forge_amd import ops
    L = _lib.lib()
    dtype, M, K, ns = F.Q4_K, 8, 4096, (4096, 1024, 1024)
    Ws = [ops.QWeight.from_numpy(synth.make_weights(dtype, n, K, 90 + i), dtype, n, K,
                                 device="cuda") for i, n in enumerate(ns)]
    x = torch.from_numpy(synth.make_x(M, K, 95)).cuda()
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    assert L.fq_reserve_workspace(M, K, max(ns), side.cuda_stream) == 0
    with torch.cuda.stream(side):
        ref = ops.fused_qkv(x, *Ws).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        y = ops.fused_qkv(x, *Ws)
    for _ in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref)
        with torch.cuda.stream(side):
            ops.fused_qkv(x * 2, *Ws)
        torch.cuda.synchronize()
    del g
    assert L.fq_release_workspace(side.cuda_stream) == 0
