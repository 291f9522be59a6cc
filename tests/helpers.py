"""Shared helpers for the parity tests: golden fixtures and the tolerance."""
from __future__ import annotations

import glob
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")

# Tolerance of the hot path (floating point outputs):
#   relative L2 error        <= 1e-5
#   max abs error (per row)  <= 1e-3 * ||x_m||_2 * max|W|
REL_L2 = 1e-5
MAX_ABS_FACTOR = 1e-3


def golden_files():
    """The per-format fixtures (golden_<format>.npz); golden_fused.npz holds
    the fused operators and is read by its own tests."""
    return sorted(p for p in glob.glob(os.path.join(GOLDEN, "golden_*.npz"))
                  if not p.endswith("golden_fused.npz"))


def load_golden(path):
    z = np.load(path, allow_pickle=False)
    dtype = int(z["dtype"])
    cases = {}
    for key in z.files:
        if "/" not in key:
            continue
        case, field = key.split("/", 1)
        cases.setdefault(case, {})[field] = z[key]
    return dtype, cases


def assert_close(y, y_ref, x, w_deq, what=""):
    """rel-L2 and per-row max-abs check of y [M, N] against y_ref [M, N]."""
    y = np.asarray(y, np.float64).reshape(y_ref.shape)
    y_ref = np.asarray(y_ref, np.float64)
    x = np.asarray(x, np.float64).reshape(y_ref.shape[0], -1)
    denom = np.linalg.norm(y_ref)
    err = np.linalg.norm(y - y_ref)
    rel = err / denom if denom > 0 else err
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e} > {REL_L2}"
    wmax = float(np.max(np.abs(w_deq))) if np.size(w_deq) else 0.0
    for m in range(y_ref.shape[0]):
        bound = MAX_ABS_FACTOR * np.linalg.norm(x[m]) * wmax
        mx = float(np.max(np.abs(y[m] - y_ref[m]))) if y_ref.shape[1] else 0.0
        assert mx <= bound, f"{what}: row {m} max-abs {mx:.3e} > {bound:.3e}"
    return rel


def silu(v):
    """silu(v) = v * sigmoid(v) in fp64, without overflow."""
    v = np.asarray(v, np.float64)
    return v * 0.5 * (1.0 + np.tanh(0.5 * v))


def assert_close_silu_mul(y, g, u, x, wmax, what="", y_ref=None):
    """The gate/up product y = silu(g) * u against the exact product of the
    exact matmuls g, u [M, N] (or against y_ref when given), at the path's
    bar carried through the product: relative L2 <= 1e-5, and per element
    |dy| <= E (1.1 |u| + |silu(g)|) with E = 1e-3 ||x_m||_2 max|W| the matmul
    bar on g and u (first order; |silu'| <= 1.1)."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    ref = silu(g) * u if y_ref is None else np.asarray(y_ref, np.float64).reshape(g.shape)
    y = np.asarray(y, np.float64).reshape(ref.shape)
    x = np.asarray(x, np.float64).reshape(ref.shape[0], -1)
    denom = np.linalg.norm(ref)
    rel = np.linalg.norm(y - ref) / denom if denom > 0 else np.linalg.norm(y - ref)
    assert rel <= REL_L2, f"{what}: rel-L2 {rel:.3e} > {REL_L2}"
    E = MAX_ABS_FACTOR * np.linalg.norm(x, axis=1, keepdims=True) * wmax
    bound = E * (1.1 * np.abs(u) + np.abs(silu(g))) + 1e-30
    bad = np.abs(y - ref) > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements over the propagated bar, "
                           f"worst ratio {float(np.max(np.abs(y - ref) / bound)):.3g}")
    return rel
