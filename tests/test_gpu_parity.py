"""GPU parity of the HIP path against the oracle and the reference's goldens.

Every test calls libforge_q.so through the C ABI (forge_amd.ops wraps the
ctypes calls; torch only holds device memory).  Bars:
  * dequantized weights: bit-exact;
  * matmul outputs: rel-L2 <= 1e-5 and per-row max-abs <= 1e-3*||x||_2*max|W|
    against the oracle's exact (fp64) product over the bit-exact dequantized W.
Shapes are the benchmark configurations at full size where the oracle runs in
seconds; the M = 512 prefill compares a subset of token rows and checks
size-independent properties (linearity, batch consistency) on the rest.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from forge_amd import formats as F
from forge_amd import ops, synth
from helpers import assert_close, golden_files, load_golden

pytestmark = pytest.mark.gpu

ALL = sorted(F.FORMATS)
DEV = "cuda"


def dev_weight(dtype, w_np, N, K, offset=0):
    """Upload block bytes; ``offset`` shifts the base address (alignment test)."""
    flat = np.ascontiguousarray(w_np).reshape(-1)
    buf = torch.empty(flat.size + offset, dtype=torch.uint8, device=DEV)
    buf[offset:] = torch.from_numpy(flat).to(DEV)
    return ops.QWeight(buf[offset:], int(dtype), int(N), int(K))


def run(dtype, w_np, x_np, N, K, offset=0, bias=None):
    w = dev_weight(dtype, w_np, N, K, offset)
    x = torch.from_numpy(np.ascontiguousarray(x_np, np.float32)).to(DEV)
    y = ops.matmul_transB(x, w, bias)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check_shape(dtype, N, K, M, seed, what=""):
    w = synth.make_weights(dtype, N, K, seed)
    x = synth.make_x(M, K, seed + 1)
    y = run(dtype, w, x, N, K)
    y64 = oracle.matmul_f64(dtype, x, w, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
    return assert_close(y, y64, x, np.array([deq_max]), what or f"{F.fmt(dtype).name} {N}x{K} M={M}")


# ------------------------------------------------------------ dequant
@pytest.mark.parametrize("path", golden_files(), ids=lambda p: p.rsplit("_", 1)[-1][:-4])
def test_dequant_golden_bitexact(path):
    dtype, cases = load_golden(path)
    for name, c in cases.items():
        w, K = c["w"], int(c["K"])
        N = w.shape[0]
        out = ops.dequantize_weight(dev_weight(dtype, w, N, K)).cpu().numpy()
        assert np.array_equal(out.view(np.uint32), c["deq"].view(np.uint32)), name


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("N,K", [(1, 256), (37, 2048), (300, 3584), (64, 18944)])
def test_dequant_random_bitexact(dtype, N, K):
    w = synth.make_weights(dtype, N, K, seed=N + K)
    out = ops.dequantize_weight(dev_weight(dtype, w, N, K)).cpu().numpy()
    ref = oracle.dequant(dtype, w, N, K)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------ goldens
@pytest.mark.parametrize("path", golden_files(), ids=lambda p: p.rsplit("_", 1)[-1][:-4])
def test_matmul_golden(path):
    dtype, cases = load_golden(path)
    for name in ("rand", "edge"):
        c = cases[name]
        w, K = c["w"], int(c["K"])
        N = w.shape[0]
        for xk in ("x1", "x3"):
            x = c[xk]
            y = run(dtype, w, x, N, K)
            y64 = oracle.matmul_f64(dtype, x, w, N, K)
            assert_close(y, y64, x, c["deq"], f"{name}/{xk} vs oracle")
            assert_close(y, c["y_" + xk], x, c["deq"], f"{name}/{xk} vs reference")


# ------------------------------------------------------------ configs
CONFIG_GEMV = [
    # config 0: TinyLlama FFN up, Q4_0
    ("cfg0-ffn_up", F.Q4_0, 5632, 2048),
    # config 1: one TinyLlama layer, Q4_0 and Q8_0 variants
    *[(f"cfg1-{n}-{F.fmt(dt).name}", dt, N, K)
      for dt in (F.Q4_0, F.Q8_0)
      for n, N, K in [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
                      ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]],
    # config 2: Qwen2.5-7B Q4_K_M mix
    ("cfg2-gate", F.Q4_K, 18944, 3584),
    ("cfg2-down", F.Q6_K, 3584, 18944),
    ("cfg2-lm_head", F.Q6_K, 152064, 3584),
    # Qwen2.5-7B in Q4_0, the reference's published decode workload: ffn up,
    # ffn down (K = 18944) and the >= 64k-row lm_head, on GGUF bytes (the
    # latter two take the batch-1 kernel's two-units-per-lane forms)
    ("q4_0-7b-up", F.Q4_0, 18944, 3584),
    ("q4_0-7b-down", F.Q4_0, 3584, 18944),
    ("q4_0-7b-lm_head", F.Q4_0, 152064, 3584),
]


@pytest.mark.parametrize("name,dtype,N,K", CONFIG_GEMV, ids=[c[0] for c in CONFIG_GEMV])
def test_gemv_configs(name, dtype, N, K):
    check_shape(dtype, N, K, 1, seed=1000 + N + K, what=name)


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
def test_q4_0_lm_head_vs_reference():
    # Q4_0 152064 x 3584 lm_head (the reference's output_proj_q4_0_kernel,
    # cuda_fused.cu:844-922) against the reference's own CPU matmul_transB on
    # a row subset: the first, a middle and the last 2048 rows
    N, K = 152064, 3584
    w = synth.make_weights(F.Q4_0, N, K, 1000 + N + K)
    x = synth.make_x(1, K, 1001 + N + K)
    y = run(F.Q4_0, w, x, N, K)
    for r0 in (0, N // 2 - 1024, N - 2048):
        ws = np.ascontiguousarray(w[r0:r0 + 2048])
        yr = oracle.ref_matmul(F.Q4_0, x, ws, 2048, K, threads=16)
        deq_max = float(np.max(np.abs(oracle.dequant(F.Q4_0, ws, 2048, K))))
        assert_close(y[:, r0:r0 + 2048], yr, x, np.array([deq_max]), f"rows {r0}+2048 vs reference")


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("N,K", [(1, 256), (7, 512), (17, 1024), (33, 4352), (5, 32768)])
def test_gemv_edge_shapes(dtype, N, K):
    check_shape(dtype, N, K, 1, seed=7 * N + K)


@pytest.mark.parametrize("dtype,N,K", [
    (F.Q4_0, 4099, 4160), (F.Q4_1, 4099, 4160), (F.Q8_0, 2051, 2080),
    (F.Q4_K, 4097, 4352), (F.Q6_K, 1001, 4352), (F.Q4_0, 1025, 18944 + 32),
])
def test_batch1_ragged_k_slices(dtype, N, K):
    # M = 1 on the K-sliced kernel (4 MB of weights and more, every Q6_K): the
    # last K-slice of each row is partial (Q4_0 4160: 130 blocks in slices of
    # 128, Q8_0 2080: 65 in slices of 64, Q4_K / Q6_K 4352: 68 / 68 lane units
    # of 64), the row count odd, so the last rows' loads run past the
    # matrix's end into the buffer bound (zeros) and the idle lanes are
    # masked out of the row sums
    check_shape(dtype, N, K, 1, seed=N + K, what=f"{F.fmt(dtype).name} {N}x{K} gguf")
    if K % 256 == 0:
        w = synth.make_weights(dtype, N, K, N + K)
        x = synth.make_x(1, K, N + K + 1)
        y = ops.gemv_packed(torch.from_numpy(x).to(DEV),
                            ops.pack_weights(dev_weight(dtype, w, N, K))).cpu().numpy()
        deq_max = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
        assert_close(y.reshape(1, -1), oracle.matmul_f64(dtype, x, w, N, K), x,
                     np.array([deq_max]), f"{F.fmt(dtype).name} {N}x{K} aligned")


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16, 32])
def test_small_batch_config3(M):
    # config 3: Llama-3-8B FFN up, Q4_K, speculative-verify batch sizes
    check_shape(F.Q4_K, 14336, 4096, M, seed=3000 + M, what=f"cfg3 M={M}")


@pytest.mark.parametrize("M", [3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("N,K", [(3584, 18944), (1000, 4096), (4099, 2048), (131072, 256)])
@pytest.mark.parametrize("dtype", [F.Q4_0, F.Q4_1, F.Q8_0])
def test_block_formats_small_batch_band_kernel(dtype, N, K, M):
    # Q4_0 / Q4_1 / Q8_0, 4..16 tokens (M = 4 from 16 MB, M = 3 from 16 MB at
    # K >= 14336 for Q4_0 and Q4_1; otherwise the other kernels): the fp16
    # band kernel over groups of eight blocks (144 / 160 / 272 bytes; 3584 x 18944: K split into slabs;
    # 4099 rows: a ragged last tile; 131072 rows: eight bands and more per
    # CU), each bias form added after the sum; at a 2-byte offset base or K =
    # 4096 + 32 the rows are not 16-byte aligned and the call takes the other
    # kernels
    name = F.fmt(dtype).name
    w = synth.make_weights(dtype, N, K, seed=N + M)
    x = synth.make_x(M, K, N + M + 1)
    y = run(dtype, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
    assert_close(y, oracle.matmul_f64(dtype, x, w, N, K), x, np.array([deq_max]),
                 f"{name} M={M} {N}x{K}")
    b1 = torch.linspace(-1, 1, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b1), y + b1.numpy(), rtol=1e-6,
                               atol=1e-6)
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6,
                               atol=1e-6)
    if K == 4096:
        y2 = run(dtype, w, x, N, K, offset=2)
        assert_close(y2, oracle.matmul_f64(dtype, x, w, N, K), x, np.array([deq_max]),
                     f"{name} M={M} {N}x{K} offset 2")
        K2 = K + 32
        w2 = synth.make_weights(dtype, N, K2, seed=N + M + 2)
        x2 = synth.make_x(M, K2, N + M + 3)
        assert_close(run(dtype, w2, x2, N, K2), oracle.matmul_f64(dtype, x2, w2, N, K2), x2,
                     np.array([float(np.max(np.abs(oracle.dequant(dtype, w2, N, K2))))]),
                     f"{name} M={M} {N}x{K2}")


@pytest.mark.parametrize("M", [4, 5, 9, 16])
@pytest.mark.parametrize("N,K", [(3584, 18944), (1000, 4096), (4099, 2048), (700, 256),
                                 (17000, 2048)])
def test_q6k_small_batch_band_kernel(N, K, M):
    # Q6_K, 5..16 tokens (and 4 on at most 16384 rows or under 24 MB):
    # the fp16 band kernel over
    # 210-byte super-blocks loaded from each row's aligned-down start and
    # read at the row's byte shift, four 16-element sub-blocks per chunk
    # (3584 x 18944: K split into slabs; 4099 rows: a ragged last tile), each
    # bias form after the sum; at a 2-byte offset base every row's shift
    # changes and the results stay bit-identical
    w = synth.make_weights(F.Q6_K, N, K, seed=N + M + 7)
    x = synth.make_x(M, K, N + M + 8)
    y = run(F.Q6_K, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(F.Q6_K, w, min(N, 4096), K))))
    assert_close(y, oracle.matmul_f64(F.Q6_K, x, w, N, K), x, np.array([deq_max]),
                 f"Q6_K M={M} {N}x{K}")
    np.testing.assert_array_equal(run(F.Q6_K, w, x, N, K, offset=2), y)
    b1 = torch.linspace(-1, 1, N)
    np.testing.assert_allclose(run(F.Q6_K, w, x, N, K, bias=b1), y + b1.numpy(), rtol=1e-6,
                               atol=1e-6)
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(F.Q6_K, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6,
                               atol=1e-6)


@pytest.mark.parametrize("M", [2, 3, 4, 7, 16])
@pytest.mark.parametrize("N,K", [(3584, 18944), (4099, 2048), (17001, 512)])
@pytest.mark.parametrize("dtype", [F.Q5_K, F.Q5_0, F.Q5_1, F.IQ4_NL, F.Q3_K])
def test_q5k_small_batch_band_kernel(dtype, N, K, M):
    # Q5_K, Q5_0, Q5_1, IQ4_NL and Q3_K at 2..16 tokens: the fp16 band kernel
    # where the format's rule takes it (Q5_K: the Q4_K panels plus the
    # fifth-bit plane; Q5_0, Q5_1, IQ4_NL eight blocks per panel row, rows
    # 16-byte aligned; Q3_K rows read at their byte shift; long K for all,
    # one round of bands for Q5_K, Q5_0, IQ4_NL, Q3_K), the other kernels
    # elsewhere and, except Q3_K, at a 2-byte offset base; all within the
    # same bar
    name = F.fmt(dtype).name
    w = synth.make_weights(dtype, N, K, seed=N + M + 11)
    x = synth.make_x(M, K, N + M + 12)
    y = run(dtype, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(dtype, w, min(N, 4096), K))))
    ref = oracle.matmul_f64(dtype, x, w, N, K)
    assert_close(y, ref, x, np.array([deq_max]), f"{name} M={M} {N}x{K}")
    assert_close(run(dtype, w, x, N, K, offset=2), ref, x, np.array([deq_max]),
                 f"{name} M={M} {N}x{K} offset 2")
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6,
                               atol=1e-6)


@pytest.mark.parametrize("M", [8, 9, 16])
def test_q4k_wide_small_batch(M):
    # Q4_K on more rows than one four-tile band per CU: the int8 kernel up to
    # 8 tokens, the band kernel above (K = 4352: 17 super-blocks)
    N, K = 17001, 4352
    w = synth.make_weights(F.Q4_K, N, K, seed=M + 90)
    x = synth.make_x(M, K, M + 91)
    y = run(F.Q4_K, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(F.Q4_K, w, 4096, K))))
    assert_close(y, oracle.matmul_f64(F.Q4_K, x, w, N, K), x, np.array([deq_max]),
                 f"Q4_K M={M} {N}x{K}")
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(F.Q4_K, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6,
                               atol=1e-6)


@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("dtype", [F.Q4_0, F.Q4_1, F.Q8_0, F.Q4_K, F.Q6_K])
@pytest.mark.parametrize("N,K", [(4099, 4096), (2113, 7168), (1500, 18944)])
def test_few_tokens_batch1_kernel(dtype, N, K, M):
    # M = 2 .. 4 on weights of 8 MB and more (every Q6_K; below that M = 1 and
    # M > 1 take other kernels): the batch-1 kernel
    # dots each weight unit with every token's limbs (Q4_K and Q6_K: up to
    # three tokens).  Q4_0 and Q4_1 rows of 65-192 blocks take two lane units
    # per lane at one and two tokens, one at three (so those rows' K-slices,
    # and their summation order, differ from the M = 1 call's), and other
    # kernels at four.
    # Otherwise each token's arithmetic and summation order are the batch-1
    # kernel's, so token t's row equals the M = 1 result bit for bit; the
    # oracle pins every case.  Every bias form is added after the
    # sum.  At K = 18944 the tokens' records need more LDS than there is: the
    # kernel splits K and a second pass adds the slabs, in another order than
    # the M = 1 sum.
    w = synth.make_weights(dtype, N, K, seed=50 + dtype)
    x = synth.make_x(M, K, 51 + N + M)
    y = run(dtype, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(dtype, w, N, K))))
    assert_close(y, oracle.matmul_f64(dtype, x, w, N, K), x, np.array([deq_max]),
                 f"{F.fmt(dtype).name} M={M} {N}x{K}")
    fm = F.fmt(dtype)
    units = K // 32  # 32-element units
    big = dtype == F.Q6_K or N * (K // fm.block_elems) * fm.block_bytes >= 8 << 20
    # (Q4_0 / Q8_0 from 16 MB at M = 4: the band kernel)
    band = (dtype in (F.Q4_0, F.Q4_1, F.Q8_0) and M == 4 and K % 256 == 0
            and N * (K // fm.block_elems) * fm.block_bytes >= 16 << 20)
    batch1 = (big and not band and K != 18944 and not (M == 4 and dtype in (F.Q4_K, F.Q6_K))
              and not (M > 2 and dtype in (F.Q4_0, F.Q4_1) and units > 64))
    if batch1:
        for t in range(M):
            np.testing.assert_array_equal(y[t], run(dtype, w, x[t:t + 1], N, K)[0])
    b1 = torch.linspace(-1, 1, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b1), y + b1.numpy(), rtol=1e-6, atol=1e-6)
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [F.Q4_0, F.Q4_1, F.Q8_0, F.Q6_K, F.Q5_0, F.Q5_1, F.Q3_K,
                                   F.Q5_K, F.IQ4_NL])
@pytest.mark.parametrize("M", [2, 5, 16])
def test_small_batch_formats(dtype, M):
    check_shape(dtype, 1000, 2048 if F.fmt(dtype).block_elems == 32 else 2560, M, seed=M + dtype)


@pytest.mark.parametrize("dtype", [F.Q8_0, F.Q4_0])
@pytest.mark.parametrize("N", [4096, 14336])
def test_prefill_config4(dtype, N):
    # config 4: M = 512 prefill.  The oracle checks 16 token rows; the other
    # rows are checked through batch consistency against the same rows run
    # through the small-batch path.
    K, M = 4096, 512
    w = synth.make_weights(dtype, N, K, seed=4000 + N + dtype)
    x = synth.make_x(M, K, seed=4001 + N)
    y = run(dtype, w, x, N, K)
    rows = np.r_[0:4, 250:254, 508:512, np.random.default_rng(0).integers(0, M, 4)]
    y64 = oracle.matmul_f64(dtype, x[rows], w, N, K)
    wmax = float(np.max(np.abs(oracle.dequant(dtype, w, N, K))))
    assert_close(y[rows], y64, x[rows], np.array([wmax]), f"prefill {N} rows")
    # batch consistency: a 32-row slice through the M <= 32 path
    sl = slice(100, 132)
    ys = run(dtype, w, x[sl], N, K)
    assert_close(y[sl], ys, x[sl], np.array([wmax]), "prefill vs batch")


# ------------------------------------------------------------ properties
@pytest.mark.parametrize("dtype", ALL)
def test_onehot_pins_unpack_through_gemv(dtype):
    """x = e_k selects column k of W.  For every format but Q6_K the kernel's
    arithmetic on a one-hot x is exact, so y must equal the dequantized
    column bit for bit (up to the sign of zero: Q3_K's signed scales give the
    reference -0 where the kernel's sum gives +0); Q6_K's offset term rounds
    once more (tolerance)."""
    N, K = 96, 4096
    w = synth.make_weights(dtype, N, K, seed=55 + dtype)
    deq = oracle.dequant(dtype, w, N, K)
    W = dev_weight(dtype, w, N, K)
    for k in (0, 1, 17, 31, 32, 255, 256, 1000, 4095):
        x = torch.zeros((1, K), dtype=torch.float32, device=DEV)
        x[0, k] = 1.0
        y = ops.matmul_transB(x, W).cpu().numpy()[0]
        if dtype == F.Q6_K:
            # the offset term adds one rounding of (d*sc)*(q+32) before - 32*d*sc
            np.testing.assert_allclose(y, deq[:, k], rtol=0, atol=4e-6 * np.abs(deq).max())
        else:
            want = deq[:, k] + np.float32(0.0)  # -0 -> +0
            assert np.array_equal((y + np.float32(0.0)).view(np.uint32), want.view(np.uint32)), k


@pytest.mark.parametrize("dtype", ALL)
def test_zero_linearity_determinism(dtype):
    N, K = 2048, 4096
    w = synth.make_weights(dtype, N, K, seed=66 + dtype)
    W = dev_weight(dtype, w, N, K)
    x1 = torch.from_numpy(synth.make_x(1, K, 1)).to(DEV)
    x2 = torch.from_numpy(synth.make_x(1, K, 2)).to(DEV)
    z = ops.matmul_transB(torch.zeros_like(x1), W)
    assert not torch.any(z)
    ya, yb = ops.matmul_transB(x1, W), ops.matmul_transB(x1, W)
    assert torch.equal(ya, yb)  # deterministic: no atomics
    y2 = ops.matmul_transB(x2, W)
    ylin = ops.matmul_transB(2.0 * x1 - 0.5 * x2, W)
    ref = (2.0 * ya.double() - 0.5 * y2.double())
    rel = (torch.linalg.norm(ylin.double() - ref) / torch.linalg.norm(ref)).item()
    assert rel < 1e-5


@pytest.mark.parametrize("dtype", [F.Q4_0, F.Q6_K])
def test_unaligned_weight_base(dtype):
    N, K = 257, 2048 if dtype == F.Q4_0 else 2560
    w = synth.make_weights(dtype, N, K, seed=9)
    x = synth.make_x(3, K, 10)
    y0 = run(dtype, w, x, N, K, offset=0)
    y2 = run(dtype, w, x, N, K, offset=2)  # GGUF blocks are only 2-byte aligned
    assert np.array_equal(y0, y2)


@pytest.mark.parametrize("M", [4])
def test_q6k_four_five_tokens_in_groups(M):
    # four Q6_K tokens on 24 MB and more of more than 16384 rows run as three
    # tokens on the batch-1 kernel, then the fourth: the rows equal those
    # separate calls bit for bit, with each bias form
    N, K = 17000, 2048
    w = synth.make_weights(F.Q6_K, N, K, seed=M + 80)
    x = synth.make_x(M, K, M + 81)
    y = run(F.Q6_K, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(F.Q6_K, w, N, K))))
    assert_close(y, oracle.matmul_f64(F.Q6_K, x, w, N, K), x, np.array([deq_max]),
                 f"Q6_K M={M} {N}x{K}")
    np.testing.assert_array_equal(y[:3], run(F.Q6_K, w, x[:3], N, K))
    np.testing.assert_array_equal(y[3:], run(F.Q6_K, w, x[3:], N, K))
    b1 = torch.linspace(-1, 1, N)
    np.testing.assert_allclose(run(F.Q6_K, w, x, N, K, bias=b1), y + b1.numpy(), rtol=1e-6,
                               atol=1e-6)
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(F.Q6_K, w, x, N, K, bias=b2), y + b2.numpy(), rtol=1e-6,
                               atol=1e-6)


@pytest.mark.parametrize("N,K", [(4096, 3584), (1100, 18944)])
def test_q4k_gguf_unaligned_base(N, K):
    # batch 1 on Q4_K GGUF rows at 16-byte aligned and 2-byte offset bases
    # (K = 3584 is one partial K-slice, 18944 ends in one): each K-slice is
    # staged through LDS from the aligned superset of its bytes, so the base's
    # alignment changes only the staging offset and the outputs are
    # bit-identical
    w = synth.make_weights(F.Q4_K, N, K, seed=N + 5)
    x = synth.make_x(1, K, N + 6)
    b = torch.linspace(-1, 1, N)
    ys = [run(F.Q4_K, w, x, N, K, offset=o, bias=b) for o in (0, 16, 2)]
    np.testing.assert_array_equal(ys[0], ys[1])
    np.testing.assert_array_equal(ys[0], ys[2])
    y = run(F.Q4_K, w, x, N, K)
    deq_max = float(np.max(np.abs(oracle.dequant(F.Q4_K, w, N, K))))
    assert_close(y, oracle.matmul_f64(F.Q4_K, x, w, N, K), x, np.array([deq_max]),
                 f"Q4_K {N}x{K}")
    np.testing.assert_allclose(ys[0], y + b.numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype,N,K", [(F.Q4_0, 4608, 2048), (F.Q4_0, 300, 2048),
                                       (F.Q4_K, 2048, 4096), (F.Q6_K, 700, 4352),
                                       (F.Q8_0, 2100, 2048)])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 40])
def test_activation_base_4_byte_aligned(dtype, N, K, M):
    # x at a 4-byte (not 16-byte) offset, as a slice of a larger tensor can
    # place it: every path (batch-1, few-token, band, MMQ, prefill)
    # reads x in 16-byte pieces, which gfx950 serves at any 4-byte alignment;
    # the result is bit-identical to the aligned call's
    w = synth.make_weights(dtype, N, K, seed=71)
    x = synth.make_x(M, K, 72)
    W = dev_weight(dtype, w, N, K)
    xa = torch.from_numpy(x).to(DEV)
    xo = torch.empty(M * K + 1, device=DEV)[1:].view(M, K)
    xo.copy_(xa)
    assert xo.data_ptr() % 16 == 4
    np.testing.assert_array_equal(ops.matmul_transB(xo, W).cpu().numpy(),
                                  ops.matmul_transB(xa, W).cpu().numpy())


@pytest.mark.parametrize("dtype,M", [(F.Q4_K, 1), (F.Q4_K, 2), (F.Q4_K, 3), (F.Q6_K, 2),
                                     (F.Q8_0, 2), (F.Q4_K, 40)])
def test_bias_modes(dtype, M):
    # every M path: batch 1, two tokens on the row-step kernel, the int8
    # matrix cores (Q4_K, 3..8), the fp16 MFMA path
    N, K = 300, 1024
    w = synth.make_weights(dtype, N, K, seed=11)
    x = synth.make_x(M, K, 12)
    base = run(dtype, w, x, N, K)
    b1 = torch.linspace(-1, 1, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b1), base + b1.numpy(), rtol=1e-6, atol=1e-6)
    b1s = torch.linspace(-1, 1, 100)  # shorter 1-D bias: only n < 100 (apply_bias)
    exp = base.copy()
    exp[:, :100] += b1s.numpy()
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b1s), exp, rtol=1e-6, atol=1e-6)
    b2 = torch.randn(M, N)
    np.testing.assert_allclose(run(dtype, w, x, N, K, bias=b2), base + b2.numpy(), rtol=1e-6, atol=1e-6)
    # M = 1 with a K-split (long K) adds the bias in the finalize pass
    w2 = synth.make_weights(dtype, 64, 18944, seed=13)
    x2 = synth.make_x(1, 18944, 14)
    b = torch.randn(64)
    np.testing.assert_allclose(run(dtype, w2, x2, 64, 18944, bias=b),
                               run(dtype, w2, x2, 64, 18944) + b.numpy(), rtol=1e-6, atol=1e-6)


def test_operator_errors():
    W = dev_weight(F.Q4_0, synth.make_weights(F.Q4_0, 8, 64, 1), 8, 64)
    with pytest.raises(RuntimeError, match="dimension mismatch"):
        ops.matmul_transB(torch.zeros((1, 32), device=DEV), W)
    with pytest.raises(RuntimeError, match="expects 2D"):
        ops.matmul_transB(torch.zeros((64,), device=DEV), W)
    bad = ops.QWeight(W.data, 10, 8, 64)  # Q2_K: not implemented on this path
    with pytest.raises(RuntimeError, match="Unsupported quantized type"):
        ops.matmul_transB(torch.zeros((1, 64), device=DEV), bad)


def test_empty_shapes():
    W = dev_weight(F.Q4_0, synth.make_weights(F.Q4_0, 8, 64, 1), 8, 64)
    y = ops.matmul_transB(torch.zeros((0, 64), device=DEV), W)
    assert tuple(y.shape) == (0, 8)
