"""Parity metrics between a device result and the oracle.

The stated bar for layer outputs: max|d| <= 2e-3 * ||y||_inf and cosine >= 0.9999;
top-k expert indices must be identical.
"""
import numpy as np

MAX_REL = 2e-3
MIN_COS = 0.9999


def metrics(got, ref):
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    yinf = np.abs(r).max()
    return {
        "max_rel": float(np.abs(g - r).max() / yinf) if yinf > 0 else float(np.abs(g - r).max()),
        "cos": float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r))) if yinf > 0 else 1.0,
        "bit_identical": float(np.mean(np.asarray(got, np.float32).view(np.uint32).ravel()
                                       == np.asarray(ref, np.float32).view(np.uint32).ravel())),
    }


def assert_parity(got, ref, what=""):
    m = metrics(got, ref)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert m["max_rel"] <= MAX_REL and m["cos"] >= MIN_COS, f"{what}: {m}"
    return m
