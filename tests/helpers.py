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
    return sorted(glob.glob(os.path.join(GOLDEN, "golden_*.npz")))


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
