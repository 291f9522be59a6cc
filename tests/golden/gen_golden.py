"""Write the golden vectors for the quantized-matmul hot path.

Runs the reference's OWN compiled CPU code (oracle/_ref/libforge_ref.so, built
by ``make -C oracle ref`` from the reference sources in place) on seeded
inputs and stores inputs and outputs as small .npz fixtures beside this
script.  The fixtures are data: block bytes, activations, the reference's
dequantized rows and the reference's ops::matmul_transB outputs.

Usage:  python tests/golden/gen_golden.py [format ... | fused]   (default: all)

``fused`` writes golden_fused.npz: the reference's fused decode operators
(ffn_up_fused, the fused QKV, gate+up and down+residual CPU kernels) on
seeded inputs.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from forge_amd import formats as F  # noqa: E402
from forge_amd import synth  # noqa: E402

P = ctypes.c_void_p

# fp16 bit patterns for scale fields in the edge cases: +-0, smallest and
# largest subnormal, smallest normal, 1.0, largest finite, and the Inf/NaN
# codes the reference's scalar converter maps to finite values.
SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xFBFF,
               0x8001, 0xBC00, 0x7C00, 0xFC00, 0x7E00]
FINITE_F16 = [h for h in SPECIAL_F16 if (h & 0x7C00) != 0x7C00]

SCALE_OFFSETS = {  # byte offsets of fp16 fields inside a block
    F.Q4_0: [0], F.Q4_1: [0, 2], F.Q8_0: [0], F.Q4_K: [0, 2], F.Q6_K: [208],
    F.Q5_0: [0], F.Q5_1: [0, 2], F.Q3_K: [108], F.Q5_K: [0, 2], F.IQ4_NL: [0],
}
# byte range [lo, hi) of the quant payload (everything but the fp16 fields)
PAYLOAD = {
    F.Q4_0: (2, 18), F.Q4_1: (4, 20), F.Q8_0: (2, 34), F.Q4_K: (4, 144), F.Q6_K: (0, 208),
    F.Q5_0: (2, 22), F.Q5_1: (4, 24), F.Q3_K: (0, 108), F.Q5_K: (4, 176), F.IQ4_NL: (2, 18),
}


def lib():
    path = os.path.join(ROOT, "oracle", "_ref", "libforge_ref.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} missing: run `make -C oracle ref` first")
    return ctypes.CDLL(path)


def ref_dequant(L, dt, w, N, K):
    out = np.zeros((N, K), np.float32)
    assert L.fqr_dequant_rows(dt, w.ctypes.data_as(P), out.ctypes.data_as(P), N, K) == 0
    return out


def ref_matmul(L, dt, x, w, M, K, N):
    y = np.zeros((M, N), np.float32)
    rc = L.fqr_matmul_transB(dt, x.ctypes.data_as(P), w.ctypes.data_as(P),
                             y.ctypes.data_as(P), M, K, N, 4)
    assert rc == 0, rc
    return y


def set_scales(w, f, K, patterns):
    nb = -(-K // f.block_elems)
    blk = w.reshape(w.shape[0], nb, f.block_bytes)
    i = 0
    for n in range(blk.shape[0]):
        for b in range(nb):
            for off in SCALE_OFFSETS[f.dtype]:
                h = patterns[i % len(patterns)]
                blk[n, b, off] = h & 0xFF
                blk[n, b, off + 1] = h >> 8
                i += 1


def extreme_payload(w, f, K):
    """Saturate the quant payload of every other row (all-0 / all-1 bits)."""
    nb = -(-K // f.block_elems)
    blk = w.reshape(w.shape[0], nb, f.block_bytes)
    lo, hi = PAYLOAD[f.dtype]
    blk[0::4, :, lo:hi] = 0x00
    blk[1::4, :, lo:hi] = 0xFF
    if f.dtype == F.Q8_0:
        blk[2::4, :, lo:hi] = 0x80  # int8 -128, outside the synthetic range
        blk[3::4, :, lo:hi] = 0x7F


def _in_silu_range(dt, x, wg, K):
    """x scaled by a power of two so that every gate value stays within
    |g| <= 32.  The reference's AVX2 silu_multiply (elementwise.cpp:100-160)
    builds exp(-g) from a 2^n exponent without clamping n, so for |g| above
    about 87 it returns garbage (e.g. silu(-129) * u = -3.3e4); the synthetic
    K-quant weights give gate values in the hundreds at x ~ N(0, 1)."""
    d = np.zeros((wg.shape[0], K), np.float32)
    assert lib().fqr_dequant_rows(dt, wg.ctypes.data_as(P), d.ctypes.data_as(P),
                                  wg.shape[0], K) == 0
    gmax = float(np.max(np.abs(x.astype(np.float64) @ d.T.astype(np.float64))))
    k = 0
    while gmax / 2.0 ** k > 32.0:
        k += 1
    return np.ascontiguousarray((x * np.float32(2.0 ** -k)).astype(np.float32))


def fused_goldens(L):
    """The reference's fused operators (its own compiled CPU code) on small
    seeded inputs: weights under "<op>/<fmt>/<w...>", per token count
    "<op>/<fmt>/M<m>/{x,r,y}"."""
    out = {}

    def arr(a):
        return np.ascontiguousarray(a)

    for dt in (F.Q4_0, F.Q4_K, F.Q6_K, F.Q8_0):
        f = F.fmt(dt)
        K = 512
        N = 21
        wg = synth.make_weights(dt, N, K, seed=900 + dt)
        wu = synth.make_weights(dt, N, K, seed=950 + dt)
        for M in (1, 3):
            x = _in_silu_range(dt, synth.make_x(M, K, seed=1000 + 10 * dt + M), wg, K)
            y = np.zeros((M, N), np.float32)
            assert L.fqr_ffn_up_fused(dt, arr(x).ctypes.data_as(P), wg.ctypes.data_as(P),
                                      wu.ctypes.data_as(P), y.ctypes.data_as(P), M, K, N, 4) == 0
            key = f"ffn_up_fused/{f.name}"
            out.update({f"{key}/M{M}/x": x, f"{key}/wg": wg, f"{key}/wu": wu,
                        f"{key}/M{M}/y": y, f"{key}/dtype": np.int64(dt)})
    for dt in (F.Q4_0, F.Q4_K):
        f = F.fmt(dt)
        K = 512
        Nq, Nk, Nv = 36, 12, 12
        wq = synth.make_weights(dt, Nq, K, seed=1100 + dt)
        wk = synth.make_weights(dt, Nk, K, seed=1150 + dt)
        wv = synth.make_weights(dt, Nv, K, seed=1175 + dt)
        wg = synth.make_weights(dt, 22, K, seed=1200 + dt)
        wu = synth.make_weights(dt, 22, K, seed=1250 + dt)
        for M in (1, 2):
            x = _in_silu_range(dt, synth.make_x(M, K, seed=1300 + 10 * dt + M), wg, K)
            y = np.zeros((M, Nq + Nk + Nv), np.float32)
            assert L.fqr_fused_qkv(dt, arr(x).ctypes.data_as(P), wq.ctypes.data_as(P),
                                   wk.ctypes.data_as(P), wv.ctypes.data_as(P),
                                   y.ctypes.data_as(P), M, K, Nq, Nk, Nv, 4) == 0
            key = f"fused_qkv/{f.name}"
            out.update({f"{key}/M{M}/x": x, f"{key}/wq": wq, f"{key}/wk": wk, f"{key}/wv": wv,
                        f"{key}/M{M}/y": y, f"{key}/dtype": np.int64(dt)})
            y = np.zeros((M, 22), np.float32)
            assert L.fqr_fused_ffn_up(dt, arr(x).ctypes.data_as(P), wg.ctypes.data_as(P),
                                      wu.ctypes.data_as(P), y.ctypes.data_as(P), M, K, 22, 4) == 0
            key = f"fused_ffn_up/{f.name}"
            out.update({f"{key}/M{M}/x": x, f"{key}/wg": wg, f"{key}/wu": wu,
                        f"{key}/M{M}/y": y, f"{key}/dtype": np.int64(dt)})
    for dt in (F.Q4_0, F.Q6_K):
        f = F.fmt(dt)
        K = 512
        N = 24
        w = synth.make_weights(dt, N, K, seed=1400 + dt)
        for M in (1, 2):
            x = synth.make_x(M, K, seed=1500 + 10 * dt + M)
            r = synth.make_x(M, N, seed=1600 + 10 * dt + M)
            y = np.zeros((M, N), np.float32)
            assert L.fqr_fused_down_residual(dt, arr(x).ctypes.data_as(P), w.ctypes.data_as(P),
                                             arr(r).ctypes.data_as(P), y.ctypes.data_as(P), M, K,
                                             N, 4) == 0
            key = f"fused_down_residual/{f.name}"
            out.update({f"{key}/M{M}/x": x, f"{key}/w": w, f"{key}/M{M}/r": r,
                        f"{key}/M{M}/y": y, f"{key}/dtype": np.int64(dt)})
    path = os.path.join(HERE, "golden_fused.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} B)")


def main():
    L = lib()
    if sys.argv[1:] == ["fused"]:
        fused_goldens(L)
        return
    only = {F.fmt(a).dtype for a in sys.argv[1:]}
    for dt, f in F.FORMATS.items():
        if only and dt not in only:
            continue
        cases = {}
        K = 512 if f.block_elems == 32 else 1024
        N = 7  # not a multiple of the reference's 4-row decode tile
        w = synth.make_weights(dt, N, K, seed=100 + dt)
        x1 = synth.make_x(1, K, seed=200 + dt)
        x3 = synth.make_x(3, K, seed=300 + dt)
        cases["rand"] = dict(w=w, K=K, x1=x1, x3=x3)

        we = synth.make_weights(dt, 8, K, seed=400 + dt)
        extreme_payload(we, f, K)
        set_scales(we, f, K, FINITE_F16)
        cases["edge"] = dict(w=we, K=K, x1=synth.make_x(1, K, seed=500 + dt),
                             x3=synth.make_x(3, K, seed=600 + dt))

        wi = synth.make_weights(dt, 4, K, seed=700 + dt)
        set_scales(wi, f, K, SPECIAL_F16)
        cases["specialf16"] = dict(w=wi, K=K)  # dequant only (Inf/NaN codes)

        # Ragged K (not a multiple of the block): dequant only.
        Kr = 80 if f.block_elems == 32 else 300
        nbr = -(-Kr // f.block_elems)
        rng = np.random.default_rng(800 + dt)
        wr = rng.integers(0, 256, size=(5, nbr * f.block_bytes), dtype=np.uint8)
        set_scales(wr, f, Kr, FINITE_F16)
        cases["ragged"] = dict(w=wr, K=Kr)

        out = {}
        for name, c in cases.items():
            w, K = c["w"], c["K"]
            N = w.shape[0]
            out[f"{name}/w"] = w
            out[f"{name}/K"] = np.int64(K)
            out[f"{name}/deq"] = ref_dequant(L, dt, w, N, K)
            for xk in ("x1", "x3"):
                if xk in c:
                    x = c[xk]
                    out[f"{name}/{xk}"] = x
                    out[f"{name}/y_{xk}"] = ref_matmul(L, dt, x, w, x.shape[0], K, N)
        path = os.path.join(HERE, f"golden_{f.name}.npz")
        np.savez_compressed(path, dtype=np.int64(dt), **out)
        print(f"wrote {path} ({os.path.getsize(path)} B)")


if __name__ == "__main__":
    main()
