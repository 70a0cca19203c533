"""Tolerances of the parity contract.

* north star: sign exact on non-singular inputs; logabs within
  1e-5 * max(1, |logabs|) + 1e-6 * n; gradients within 1e-4 relative Frobenius error;
  singular inputs give (0, -inf) and finite gradients.
* reference tests (tests/test_fermix.py:62-70): float32 logabs within
  2e-3 * max(1, n / 64) absolute, gradients within 1e-4 max-abs relative error on
  well-conditioned inputs.
"""

import numpy as np


def logabs_tol(logabs_ref, n):
    return 1e-5 * np.maximum(1.0, np.abs(logabs_ref)) + 1e-6 * n


def ref_log_tol(n):
    return 2e-3 * max(1.0, n / 64)


def rel_fro(x, ref):
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref.reshape(ref.shape[0], -1), axis=1)
    num = np.linalg.norm((x - ref).reshape(ref.shape[0], -1), axis=1)
    return num / np.maximum(den, 1e-300)


def relerr(x, ref):
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(x - ref)) / max(np.max(np.abs(ref)), 1e-30))


def assert_logabs(l, lref, n, what=""):
    l = np.asarray(l, np.float64)
    lref = np.asarray(lref, np.float64)
    fin = np.isfinite(lref)
    assert np.array_equal(np.isneginf(l), np.isneginf(lref)), (what, l, lref)
    err = np.abs(l[fin] - lref[fin])
    tol = logabs_tol(lref[fin], n)
    assert np.all(err <= tol), (what, float(err.max()) if err.size else 0.0)
