"""GPU tests of the aligned device layout (fq_pack_weights / fq_gemv_packed).

The packed layout moves bytes only, so: unpack(pack(w)) == w byte for byte,
dequantizing the unpacked bytes is bit-exact against the oracle, and the
packed GEMV meets the path's tolerance against the oracle's exact product.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from forge_amd import formats as F
from forge_amd import ops, synth
from helpers import assert_close

pytestmark = pytest.mark.gpu

ALL = [F.Q4_0, F.Q4_1, F.Q8_0, F.Q4_K, F.Q6_K]
DEV = "cuda"


def qweight(dtype, N, K, seed):
    w = synth.make_weights(dtype, N, K, seed)
    return w, ops.QWeight.from_numpy(w, dtype, N, K, device=DEV)


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("N,K", [(1, 256), (37, 2048), (130, 3584), (9, 18944),
                                 (65541, 256)])  # Q8_0: the tiled arrangement
def test_pack_roundtrip_bitexact(dtype, N, K):
    w, W = qweight(dtype, N, K, seed=N * 7 + K)
    P = ops.pack_weights(W)
    assert P.data.numel() == N * ops.packed_row_bytes(dtype, K)
    back = ops.unpack_weights(P).data.cpu().numpy()
    assert np.array_equal(back, w.reshape(-1))
    deq = ops.dequantize_weight(ops.unpack_weights(P)).cpu().numpy()
    assert np.array_equal(deq.view(np.uint32), oracle.dequant(dtype, w, N, K).view(np.uint32))


PACKED_SHAPES = [
    ("cfg0-ffn_up", F.Q4_0, 5632, 2048),
    ("cfg1-down-q8", F.Q8_0, 2048, 5632),
    ("cfg2-gate", F.Q4_K, 18944, 3584),
    ("cfg2-down", F.Q6_K, 3584, 18944),
    ("cfg2-lm_head", F.Q6_K, 152064, 3584),
    ("q4_0-7b-up", F.Q4_0, 18944, 3584),
    ("q4_0-7b-down", F.Q4_0, 3584, 18944),
    ("q4_0-7b-lm_head", F.Q4_0, 152064, 3584),
    ("q4_1-4096", F.Q4_1, 4096, 4096),
    ("q8_0-3584", F.Q8_0, 3000, 3584),
]


@pytest.mark.parametrize("name,dtype,N,K", PACKED_SHAPES, ids=[s[0] for s in PACKED_SHAPES])
def test_gemv_packed_configs(name, dtype, N, K):
    w, W = qweight(dtype, N, K, seed=N + K)
    x = synth.make_x(1, K, seed=K)
    P = ops.pack_weights(W)
    y = ops.gemv_packed(torch.from_numpy(x).to(DEV), P).cpu().numpy()
    y64 = oracle.matmul_f64(dtype, x, w, N, K)
    wmax = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
    assert_close(y[None, :], y64, x, np.array([wmax]), name)
    y2 = ops.gemv_packed(torch.from_numpy(x).to(DEV), P).cpu().numpy()
    assert np.array_equal(y, y2)  # deterministic, split-K included


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("N,K", [(1, 256), (7, 512), (65, 8192), (33, 12800),
                                 (65541, 256), (65536, 2048), (66000, 12800)])
def test_gemv_packed_edges(dtype, N, K):
    # 65536 rows and more of Q8_0 take the tiled arrangement (the last tile
    # partial at 65541 and 66000 rows; 66000 x 12800: the rows' records need
    # 16 waves a work-group and the tiles more work-groups than CU slots)
    w, W = qweight(dtype, N, K, seed=3 * N + K)
    x = synth.make_x(1, K, seed=K + 1)
    y = ops.gemv_packed(torch.from_numpy(x).to(DEV), ops.pack_weights(W)).cpu().numpy()
    y64 = oracle.matmul_f64(dtype, x, w, N, K)
    wmax = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
    assert_close(y[None, :], y64, x, np.array([wmax]), f"{N}x{K}")


@pytest.mark.parametrize("dtype", [F.Q4_0, F.Q6_K])
@pytest.mark.parametrize("K", [3584, 18944])
@pytest.mark.parametrize("N", [300, 65600])
def test_gemv_packed_bias(dtype, K, N):
    w, W = qweight(dtype, N, K, seed=5)
    x = torch.from_numpy(synth.make_x(1, K, 6)).to(DEV)
    P = ops.pack_weights(W)
    b = torch.randn(N, device=DEV)
    y0 = ops.gemv_packed(x, P)
    y1 = ops.gemv_packed(x, P, b)
    # the bias joins the first K-slice's partial, so the rounding order differs
    tol = 1e-6 * float(y0.abs().max())
    torch.testing.assert_close(y1, y0 + b, rtol=0, atol=tol)
    bs = torch.randn(100, device=DEV)  # shorter bias: only n < 100
    y2 = ops.gemv_packed(x, P, bs)
    exp = y0.clone()
    exp[:100] += bs
    torch.testing.assert_close(y2, exp, rtol=0, atol=tol)


def test_packed_alignment_and_shape_errors():
    from forge_amd import _lib
    w, W = qweight(F.Q4_0, 8, 512, seed=1)
    buf = torch.empty(8 * ops.packed_row_bytes(F.Q4_0, 512) + 16, dtype=torch.uint8, device=DEV)
    L = _lib.lib()
    st = L.fq_pack_weights(F.Q4_0, W.data.data_ptr(), buf.data_ptr() + 2, 8, 512, None)
    assert st == _lib.FQ_ERR_ALIGN
    st = L.fq_pack_weights(F.Q4_0, W.data.data_ptr(), buf.data_ptr(), 8, 480, None)
    assert st == _lib.FQ_ERR_SHAPE


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_gemv_packed_q6k_limb_chain_extremes(sign):
    # every 6-bit code at 63 and every activation at 1.99 (limbs a1 = 127,
    # a2 = 46): each 16-quant group's int32 limb chain reaches ~2.10e9, just
    # under 2^31; each row's sub-scales all at one int8 extreme
    N, K = 64, 3584
    f = F.fmt(F.Q6_K)
    w = synth.make_weights(F.Q6_K, N, K, seed=41).reshape(N, K // 256, f.block_bytes)
    w[:, :, 0:192] = 0xFF                                   # ql, qh: q = 63
    w[0::2, :, 192:208] = np.uint8(127)                      # sub-scales +127
    w[1::2, :, 192:208] = np.array([-128], np.int8).view(np.uint8)[0]  # and -128
    w = w.reshape(N, -1)
    x = np.full((1, K), sign * 1.99, np.float32)
    P = ops.pack_weights(ops.QWeight.from_numpy(w, F.Q6_K, N, K, device=DEV))
    y = ops.gemv_packed(torch.from_numpy(x).to(DEV), P).cpu().numpy()
    y64 = oracle.matmul_f64(F.Q6_K, x, w, N, K)
    wmax = float(np.max(np.abs(oracle.dequant(F.Q6_K, w, N, K))))
    assert_close(y[None, :], y64, x, np.array([wmax]), f"q6_k extremes sign {sign}")
