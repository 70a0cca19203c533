"""Float64 truth from the mathematics -- TEST INFRASTRUCTURE (pins ``oracle.generic``
and checks the GPU results). Written from the definitions, independent of the
algorithms under test where possible:

* ``slogdet64`` -- numpy's LAPACK slogdet in float64 / complex128 (the reference's own
  tests use it, ``tests/test_fermix.py:153-155``);
* ``pf_brute`` -- the Pfaffian as a signed sum over perfect matchings (expansion along
  the first row), exact up to float64 rounding, n <= 10;
* ``pf_pr64`` -- a float64 Parlett-Reid (the textbook algorithm, cross-checked against
  ``pf_brute`` and pf^2 = det);
* ``adjT_brute`` -- d det / dA = adj(A)^T by cofactors;
* ``adjT_svd`` -- the same from the SVD, A = U diag(sig) V^T:
  adj(A)^T = det(U) det(V) U diag(prod_{j != i} sig_j) V^T (any n, exact continuation
  to singular A; pinned against ``adjT_brute``);
* ``pf_grad_brute`` -- d pf / dS by minor Pfaffians;
* ``pf_grad64`` -- the same with the minors' Pfaffians from ``pf64`` (larger n), and
  ``pf_grad64_rows`` for the entries in given rows only.
"""

import math
import numpy as np


def _wide(x):
    """float64, or complex128 for complex input."""
    x = np.asarray(x)
    return x.astype(np.complex128 if np.iscomplexobj(x) else np.float64)


def slogdet64(A):
    s, l = np.linalg.slogdet(_wide(A))
    return s, l


def pf_brute(S):
    """Pfaffian of one skew matrix by the perfect-matching expansion
    pf(S) = sum_j (-1)^(j+1) s_0j pf(S without rows/cols 0, j) (0-based j >= 1); float64
    or complex128."""
    S = _wide(S)
    n = S.shape[0]
    if n % 2:
        return 0.0
    if n == 0:
        return 1.0
    total = 0.0
    rest = list(range(1, n))
    for t, j in enumerate(rest):
        if S[0, j] == 0.0:
            continue
        keep = [k for k in rest if k != j]
        total += (-1) ** t * S[0, j] * pf_brute(S[np.ix_(keep, keep)])
    return total


def pf_pr64(S):
    """(sign, log|pf|) of one skew matrix by Parlett-Reid with partial pivoting in
    float64 (complex128 for complex S, the sign then the unit phase): pivot the largest
    |entry| of column k below row k into row/col k+1."""
    A = _wide(S).copy()
    cplx = np.iscomplexobj(A)
    n = A.shape[0]
    if n % 2:
        return 0.0, -math.inf
    sign, log = (1.0 + 0.0j if cplx else 1.0), 0.0
    for k in range(0, n - 1, 2):
        kp = k + 1 + int(np.argmax(np.abs(A[k + 1 :, k])))
        if kp != k + 1:
            A[[k + 1, kp], :] = A[[kp, k + 1], :]
            A[:, [k + 1, kp]] = A[:, [kp, k + 1]]
            sign = -sign
        d = A[k, k + 1]
        if d == 0.0:
            return 0.0, -math.inf
        sign *= d / abs(d) if cplx else math.copysign(1.0, d)
        log += math.log(abs(d))
        x = A[k + 2 :, k].copy()
        y = A[k + 2 :, k + 1].copy()
        A[k + 2 :, k + 2 :] += (np.outer(y, x) - np.outer(x, y)) / d
    return sign, log


def pf64(S):
    s, l = pf_pr64(S)
    return s * math.exp(l) if np.isfinite(l) else 0.0


def slogpf64(Sb):
    """Batched (sign, log|pf|) in float64 (complex128 sign for complex input)."""
    out = [pf_pr64(S) for S in np.asarray(Sb)]
    return np.array([o[0] for o in out]), np.array([o[1] for o in out], np.float64)


def adjT_brute(A):
    """d det / dA = adj(A)^T by cofactors, float64 (complex128 for complex A: the
    holomorphic derivative, no conjugation)."""
    A = _wide(A)
    n = A.shape[0]
    G = np.zeros((n, n), A.dtype)
    for i in range(n):
        for j in range(n):
            M = np.delete(np.delete(A, i, 0), j, 1)
            G[i, j] = (-1) ** (i + j) * (np.linalg.det(M) if n > 1 else 1.0)
    return G


def pf_grad_brute(S):
    """d pf / dS with the skew extension G = (D - D^T)/2,
    D_ij = (-1)^(i+j+1) pf(S without rows/cols i, j) for i < j (brute force); float64 or
    complex128 (the holomorphic derivative)."""
    S = _wide(S)
    n = S.shape[0]
    D = np.zeros((n, n), S.dtype)
    for i in range(n):
        for j in range(i + 1, n):
            keep = [k for k in range(n) if k not in (i, j)]
            D[i, j] = (-1) ** (i + j + 1) * pf_brute(S[np.ix_(keep, keep)])
    return 0.5 * (D - D.T)


def inv64(A):
    return np.linalg.inv(np.asarray(A, np.float64))


def adjT_svd(A):
    """d det / dA = adj(A)^T from the SVD (float64, or complex128 for complex A): with
    A = U diag(sig) Vt (U, Vt unitary, adj(U) = det(U) U^H), adj(A) = adj(Vt) adj(diag(sig))
    adj(U) = det(Vt) det(U) Vt^H diag(p) U^H, p_i = prod_{j != i} sig_j, so adj(A)^T =
    det(U) det(Vt) conj(U) diag(p) conj(Vt) (U diag(p) Vt for real A). The products are
    formed in logs (sig_j = 0 contributes an exact zero)."""
    A = _wide(A)
    n = A.shape[0]
    if n == 0:
        return np.zeros((0, 0), A.dtype)
    U, sig, Vt = np.linalg.svd(A)
    with np.errstate(divide="ignore"):
        lg = np.log(sig)
    p = np.empty(n)
    for i in range(n):
        others = np.delete(lg, i)
        p[i] = 0.0 if np.any(np.isneginf(others)) else math.exp(float(np.sum(others)))
    return np.linalg.det(U) * np.linalg.det(Vt) * (U.conj() * p[None, :]) @ Vt.conj()


def pf_grad64(S):
    """d pf / dS as in ``pf_grad_brute`` with each minor's Pfaffian from ``pf64``."""
    S = _wide(S)
    n = S.shape[0]
    D = np.zeros((n, n), S.dtype)
    for i in range(n):
        for j in range(i + 1, n):
            keep = [k for k in range(n) if k not in (i, j)]
            D[i, j] = (-1) ** (i + j + 1) * pf64(S[np.ix_(keep, keep)])
    return 0.5 * (D - D.T)


def pf_grad64_rows(S, rows):
    """d pf / dS restricted to the entries (i, j) with i or j in ``rows`` (the rest set to
    zero): for S whose every other minor Pfaffian vanishes -- e.g. S with the rows and
    columns ``rows`` exactly zero -- this is the whole gradient, at O(n |rows|) minors."""
    S = _wide(S)
    n = S.shape[0]
    D = np.zeros((n, n), S.dtype)
    for i in range(n):
        for j in range(i + 1, n):
            if i not in rows and j not in rows:
                continue
            keep = [k for k in range(n) if k not in (i, j)]
            D[i, j] = (-1) ** (i + j + 1) * pf64(S[np.ix_(keep, keep)])
    return 0.5 * (D - D.T)
