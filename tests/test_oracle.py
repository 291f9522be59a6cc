"""CPU tests pinning the oracle (oracle/fq_oracle.c).

Each oracle function is checked against something it does not restate:
  * the golden vectors written by the reference's own compiled CPU code
    (tests/golden/gen_golden.py over oracle/_ref/libforge_ref.so);
  * closed forms: numpy's IEEE float16 conversion, an independent encoder
    that packs known codes/scales from the GGUF format definition (element e
    of a super-block uses sub-block e//32 for Q4_K and e//16 for Q6_K), and
    brute-force products on tiny inputs.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import oracle
from forge_amd import formats as F
from forge_amd import synth
from helpers import assert_close, golden_files, load_golden

ALL = sorted(F.FORMATS)

# IQ4_NL code -> value table of the format definition (matmul.cpp:849-851)
IQ4_NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10,
                          1, 13, 25, 38, 53, 69, 89, 113], np.float32)


# ---------------------------------------------------------------- fp16
def test_fp16_all_codes(oracle_lib):
    codes = np.arange(65536, dtype=np.uint16)
    got = np.array([oracle_lib.fqo_fp16_to_fp32(int(c)) for c in codes], np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    exp = (codes >> 10) & 31
    man = (codes & 0x3FF).astype(np.float64)
    sign = np.where(codes >> 15, -1.0, 1.0)
    finite = exp != 31
    # finite codes: exact IEEE conversion except that -0 maps to +0
    nz = finite & ((codes & 0x7FFF) != 0)
    assert np.array_equal(got[nz].view(np.uint32), ref[nz].view(np.uint32))
    zero = (codes & 0x7FFF) == 0
    assert np.all(got[zero].view(np.uint32) == 0)  # both +0 and -0 -> +0
    # exponent 31 codes: the reference's formula gives (1 + m/1024) * 2^16
    inf_nan = ~finite
    want = (sign * (1.0 + man / 1024.0) * 65536.0).astype(np.float32)
    assert np.array_equal(got[inf_nan], want[inf_nan])


# ---------------------------------------------------------------- golden
@pytest.mark.parametrize("path", golden_files(), ids=lambda p: p.rsplit("_", 1)[-1][:-4])
def test_oracle_matches_reference_golden(path):
    dtype, cases = load_golden(path)
    assert set(cases) >= {"rand", "edge", "specialf16", "ragged"}
    for name, c in cases.items():
        w, K = c["w"], int(c["K"])
        N = w.shape[0]
        deq = oracle.dequant(dtype, w, N, K)
        assert np.array_equal(deq.view(np.uint32), c["deq"].view(np.uint32)), name
        for xk in ("x1", "x3"):
            if xk not in c:
                continue
            y64 = oracle.matmul_f64(dtype, c[xk], w, N, K)
            # the reference's fp32 AVX2 sums agree with the exact product
            assert_close(c["y_" + xk], y64, c[xk], deq, f"{name}/{xk}")


def test_golden_covers_every_format():
    got = sorted(load_golden(p)[0] for p in golden_files())
    assert got == sorted(ALL)


# ---------------------------------------------------------------- encoder
def _f16(v):
    return np.asarray(v, np.float32).astype(np.float16)


def encode(dtype, codes, d, extra=None):
    """Pack integer codes [N, K] (and per-block/sub-block scales) into blocks.

    Written from the GGUF format definition, independently of the oracle's
    loops.  Returns (blocks uint8 [N, row_bytes], expected fp32 [N, K]).
    """
    N, K = codes.shape
    f = F.fmt(dtype)
    nb = K // f.block_elems
    out = np.zeros((N, nb, f.block_bytes), np.uint8)
    c = codes.reshape(N, nb, f.block_elems)
    dh = _f16(d).reshape(N, nb)
    df = dh.astype(np.float32)[..., None]
    if dtype in (F.Q4_0, F.Q4_1):
        off = 2 if dtype == F.Q4_0 else 4
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., off:off + 16] = (c[..., :16] | (c[..., 16:] << 4)).astype(np.uint8)
        if dtype == F.Q4_0:
            want = (c.astype(np.float32) - 8.0) * df
        else:
            mh = _f16(extra).reshape(N, nb)
            out[..., 2:4] = mh.view(np.uint8).reshape(N, nb, 2)
            want = c.astype(np.float32) * df + mh.astype(np.float32)[..., None]
    elif dtype == F.Q8_0:
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., 2:34] = c.astype(np.int8).view(np.uint8)
        want = c.astype(np.float32) * df
    elif dtype == F.Q4_K:
        dmin_h = _f16(extra["dmin"]).reshape(N, nb)
        sc, mn = extra["sc"], extra["m"]  # [N, nb, 8] 6-bit
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., 2:4] = dmin_h.view(np.uint8).reshape(N, nb, 2)
        s = np.zeros((N, nb, 12), np.uint16)
        s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
        s[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
        s[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
        out[..., 4:16] = s.astype(np.uint8)
        cc = c.reshape(N, nb, 4, 2, 32)  # [.., pair g, sub 0/1, 32]
        out[..., 16:144] = (cc[..., 0, :] | (cc[..., 1, :] << 4)).reshape(N, nb, 128)
        sub = np.repeat(np.arange(8), 32)  # element e -> sub-block e // 32
        d1 = df * sc[..., sub].astype(np.float32)
        m1 = dmin_h.astype(np.float32)[..., None] * mn[..., sub].astype(np.float32)
        want = d1 * c.astype(np.float32) - m1
    elif dtype == F.Q6_K:
        sc = extra["sc"]  # [N, nb, 16] int8
        e = np.arange(256)
        half, r = e // 128, e % 128
        grp, l = r // 32, r % 32
        ql_idx = 64 * half + l + 32 * (grp & 1)
        ql_shift = 4 * (grp >> 1)
        qh_idx = 32 * half + l
        qh_shift = 2 * grp
        ql = np.zeros((N, nb, 128), np.int64)
        qh = np.zeros((N, nb, 64), np.int64)
        for i in range(256):
            ql[..., ql_idx[i]] |= (c[..., i] & 15) << ql_shift[i]
            qh[..., qh_idx[i]] |= ((c[..., i] >> 4) & 3) << qh_shift[i]
        out[..., 0:128] = ql.astype(np.uint8)
        out[..., 128:192] = qh.astype(np.uint8)
        out[..., 192:208] = sc.astype(np.int8).view(np.uint8)
        out[..., 208:210] = dh.view(np.uint8).reshape(N, nb, 2)
        dsc = df * sc[..., e // 16].astype(np.float32)  # element e -> sub-block e // 16
        want = dsc * (c.astype(np.float32) - 32.0)
    elif dtype in (F.Q5_0, F.Q5_1):
        qs_off = 6 if dtype == F.Q5_0 else 8
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., qs_off:qs_off + 16] = ((c[..., :16] & 15) | ((c[..., 16:] & 15) << 4)).astype(np.uint8)
        qh = np.zeros((N, nb), np.uint64)
        for j in range(32):  # bit j of the 32-bit qh word is bit 4 of element j
            qh |= ((c[..., j] >> 4) & 1).astype(np.uint64) << np.uint64(j)
        out[..., qs_off - 4:qs_off] = qh.astype("<u4").view(np.uint8).reshape(N, nb, 4)
        if dtype == F.Q5_0:
            want = (c.astype(np.float32) - 16.0) * df
        else:
            mh = _f16(extra).reshape(N, nb)
            out[..., 2:4] = mh.view(np.uint8).reshape(N, nb, 2)
            want = c.astype(np.float32) * df + mh.astype(np.float32)[..., None]
    elif dtype == F.IQ4_NL:
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., 2:18] = (c[..., :16] | (c[..., 16:] << 4)).astype(np.uint8)
        want = df * IQ4_NL_VALUES[c]
    elif dtype == F.Q3_K:
        sc = extra["sc"]  # [N, nb, 16] in -32..31
        hm = np.zeros((N, nb, 32), np.int64)
        qs = np.zeros((N, nb, 64), np.int64)
        for e in range(256):  # 128-element halves, 32-element rows of 2-bit planes
            n, j, l = e // 128, (e % 128) // 32, e % 32
            qs[..., 32 * n + l] |= (c[..., e] & 3) << (2 * j)  # c in -4..3, two's complement
            hm[..., l] |= (c[..., e] >= 0).astype(np.int64) << (4 * n + j)
        raw = np.zeros((N, nb, 12), np.int64)
        for j in range(16):  # scale j + 32 as 6 bits: low nibbles, then 2-bit high parts
            v = sc[..., j] + 32
            if j < 8:
                raw[..., j] |= v & 15
            else:
                raw[..., j - 8] |= (v & 15) << 4
            raw[..., 8 + j % 4] |= (v >> 4) << (2 * (j // 4))
        out[..., 0:32] = hm.astype(np.uint8)
        out[..., 32:96] = qs.astype(np.uint8)
        out[..., 96:108] = raw.astype(np.uint8)
        out[..., 108:110] = dh.view(np.uint8).reshape(N, nb, 2)
        dl = df * sc[..., np.arange(256) // 16].astype(np.float32)  # 16-element sub-blocks
        want = dl * c.astype(np.float32)
    elif dtype == F.Q5_K:
        dmin_h = _f16(extra["dmin"]).reshape(N, nb)
        sc, mn = extra["sc"], extra["m"]
        out[..., 0:2] = dh.view(np.uint8).reshape(N, nb, 2)
        out[..., 2:4] = dmin_h.view(np.uint8).reshape(N, nb, 2)
        s = np.zeros((N, nb, 12), np.uint16)
        s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
        s[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
        s[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
        out[..., 4:16] = s.astype(np.uint8)
        cc = c.reshape(N, nb, 4, 2, 32)  # [.., pair g, sub 0/1, 32]
        out[..., 48:176] = ((cc[..., 0, :] & 15) | ((cc[..., 1, :] & 15) << 4)).reshape(N, nb, 128)
        qh = np.zeros((N, nb, 32), np.int64)
        for g in range(4):
            for h in range(2):
                qh |= ((cc[..., g, h, :] >> 4) & 1) << (2 * g + h)
        out[..., 16:48] = qh.astype(np.uint8)
        sub = np.repeat(np.arange(8), 32)
        d1 = df * sc[..., sub].astype(np.float32)
        m1 = dmin_h.astype(np.float32)[..., None] * mn[..., sub].astype(np.float32)
        want = d1 * c.astype(np.float32) - m1
    return out.reshape(N, -1), want.reshape(N, K).astype(np.float32)


def random_codes(dtype, N, K, rng):
    f = F.fmt(dtype)
    nb = K // f.block_elems
    d = np.abs(rng.normal(0, 0.05, size=(N, nb)))
    extra = None
    if dtype in (F.Q4_0, F.Q4_1, F.Q4_K, F.IQ4_NL):
        codes = rng.integers(0, 16, size=(N, K))
    elif dtype == F.Q8_0:
        codes = rng.integers(-128, 128, size=(N, K))
    elif dtype in (F.Q5_0, F.Q5_1, F.Q5_K):
        codes = rng.integers(0, 32, size=(N, K))
    elif dtype == F.Q3_K:
        codes = rng.integers(-4, 4, size=(N, K))
    else:
        codes = rng.integers(0, 64, size=(N, K))
    if dtype in (F.Q4_1, F.Q5_1):
        extra = rng.normal(0, 0.3, size=(N, nb))
    elif dtype == F.Q3_K:
        extra = dict(sc=rng.integers(-32, 32, size=(N, nb, 16)))
    elif dtype in (F.Q4_K, F.Q5_K):
        extra = dict(dmin=np.abs(rng.normal(0, 0.05, size=(N, nb))),
                     sc=rng.integers(0, 64, size=(N, nb, 8)),
                     m=rng.integers(0, 64, size=(N, nb, 8)))
    elif dtype == F.Q6_K:
        extra = dict(sc=rng.integers(-128, 128, size=(N, nb, 16)))
    return codes, d, extra


@pytest.mark.parametrize("dtype", ALL)
def test_oracle_dequant_matches_independent_encoder(dtype):
    rng = np.random.default_rng(dtype)
    N, K = 6, 512
    codes, d, extra = random_codes(dtype, N, K, rng)
    blocks, want = encode(dtype, codes, d, extra)
    got = oracle.dequant(dtype, blocks, N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", ALL)
def test_oracle_matmul_brute_force(dtype):
    rng = np.random.default_rng(10 + dtype)
    f = F.fmt(dtype)
    N, K, M = 5, f.block_elems * 2, 3
    codes, d, extra = random_codes(dtype, N, K, rng)
    blocks, want = encode(dtype, codes, d, extra)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = oracle.matmul_f64(dtype, x, blocks, N, K)
    brute = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            brute[m, n] = sum(float(x[m, k]) * float(want[n, k]) for k in range(K))
    np.testing.assert_allclose(y, brute, rtol=1e-12, atol=1e-12)
    y32 = oracle.matmul_f32(dtype, x, blocks, N, K)
    assert_close(y32, brute, x, want, "f32 order")


def test_invariants():
    rng = np.random.default_rng(7)
    N, K = 3, 256
    # Q4_0 with every nibble 8 dequantizes to exactly zero
    codes = np.full((N, K), 8)
    blocks, _ = encode(F.Q4_0, codes, np.abs(rng.normal(0, 0.05, (N, K // 32))))
    assert not np.any(oracle.dequant(F.Q4_0, blocks, N, K))
    # d = 0 gives zero for every format with a multiplicative scale
    for dt in (F.Q4_0, F.Q8_0, F.Q6_K):
        codes, d, extra = random_codes(dt, N, K, rng)
        blocks, _ = encode(dt, codes, np.zeros_like(d), extra)
        assert not np.any(oracle.dequant(dt, blocks, N, K))
    # Q4_K with dmin = 0 reduces to d * sc * q
    codes, d, extra = random_codes(F.Q4_K, N, K, rng)
    extra["dmin"] = np.zeros_like(extra["dmin"])
    blocks, want = encode(F.Q4_K, codes, d, extra)
    got = oracle.dequant(F.Q4_K, blocks, N, K)
    sub = np.repeat(np.arange(8), 32)
    dsc = _f16(d).astype(np.float32)[..., None] * extra["sc"][..., sub].astype(np.float32)
    expect = (dsc * codes.reshape(N, 1, K).astype(np.float32)).reshape(N, K)
    assert np.array_equal(got, expect)


def test_oracle_rejects_unsupported(oracle_lib):
    out = np.zeros(4, np.float32)
    w = np.zeros(64, np.uint8)
    P = ctypes.c_void_p
    assert oracle_lib.fqo_dequant_rows(1, w.ctypes.data_as(P), out.ctypes.data_as(P), 1, 4) == -1


def test_synth_distributions():
    w = synth.make_weights(F.Q4_0, 64, 2048, seed=1).reshape(64, 64, 18)
    d = w[..., 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.01 < float(np.mean(d)) < 0.02  # |N(0,0.02)| mean 0.016
    q8 = synth.make_weights(F.Q8_0, 64, 1024, seed=2).reshape(64, 32, 34)[..., 2:].view(np.int8)
    assert q8.min() >= -127 and q8.max() <= 127
    a = synth.make_weights(F.Q4_K, 4, 512, seed=3)
    b = synth.make_weights(F.Q4_K, 4, 512, seed=3)
    assert np.array_equal(a, b)


def test_fused_goldens_against_exact_products():
    """golden_fused.npz holds the reference's fused CPU operators
    (ffn_up_fused, fused QKV / gate+up / down+residual); each output agrees
    with the exact product from the oracle's fp64 matmul at the path's bar:
    the fixture is consistent and pins what the fused GPU ops must match."""
    from helpers import GOLDEN, assert_close, assert_close_silu_mul
    z = np.load(os.path.join(GOLDEN, "golden_fused.npz"), allow_pickle=False)
    keys = set(z.files)
    seen = 0
    for k in sorted(keys):
        if not k.endswith("/y"):
            continue
        op, f, m = k.split("/")[:3]
        base = f"{op}/{f}"
        dt = int(z[f"{base}/dtype"])
        x, y = z[f"{base}/{m}/x"], z[k]
        K = x.shape[1]

        def deq_max(*ws):
            return max(float(np.max(np.abs(oracle.dequant(dt, w, w.shape[0], K)))) for w in ws)

        if op in ("ffn_up_fused", "fused_ffn_up"):
            wg, wu = z[f"{base}/wg"], z[f"{base}/wu"]
            g = oracle.matmul_f64(dt, x, wg, wg.shape[0], K)
            u = oracle.matmul_f64(dt, x, wu, wu.shape[0], K)
            assert_close_silu_mul(y, g, u, x, deq_max(wg, wu), k)
        elif op == "fused_qkv":
            ws = [z[f"{base}/w{c}"] for c in "qkv"]
            ref = np.concatenate([oracle.matmul_f64(dt, x, w, w.shape[0], K) for w in ws], axis=1)
            assert_close(y, ref, x, np.array([deq_max(*ws)]), k)
        else:
            w, r = z[f"{base}/w"], z[f"{base}/{m}/r"]
            ref = oracle.matmul_f64(dt, x, w, w.shape[0], K) + r
            assert_close(y, ref, x, np.array([deq_max(w)]), k)
        seen += 1
    assert seen == 20


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
def test_reference_silu_multiply_range():
    """A reference behaviour the fused goldens avoid: the reference's AVX2
    silu_multiply (elementwise.cpp:100-160) forms exp(-g) from a 2^n exponent
    it never clamps, so for |g| beyond about 87 its result is garbage, while
    for moderate g it is accurate.  (The GPU path computes silu exactly.)"""
    L = oracle.load_ref()
    K, N = 256, 8
    w = synth.make_weights(F.Q8_0, N, K, seed=5)
    deq = oracle.dequant(F.Q8_0, w, N, K).astype(np.float64)
    for scale, ok in ((1e-2, True), (1e3, False)):
        x = (synth.make_x(1, K, 6) * np.float32(scale)).astype(np.float32)
        y = np.zeros((1, N), np.float32)
        assert L.fqr_ffn_up_fused(F.Q8_0, oracle._p(x), oracle._p(w), oracle._p(w),
                                  oracle._p(y), 1, K, N, 1) == 0
        g = x.astype(np.float64) @ deq.T
        exact = g * 0.5 * (1.0 + np.tanh(0.5 * g)) * g
        close = np.allclose(y, exact, rtol=1e-4, atol=1e-6 * np.max(np.abs(exact)))
        assert close == ok, (scale, float(np.max(np.abs(g))))
