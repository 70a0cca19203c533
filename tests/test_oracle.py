"""Pin the CPU oracle (oracle.generic, the restated generic path of the reference)
against float64 truth, closed forms and brute force -- before anything is compared
with it. Every check is chosen so that a plausible mistake (a dropped term, a wrong
sign or index, a transposed operand) fails; test_planted_mistakes_are_caught shows a
few such mistakes, planted in copies of the oracle, being caught."""

import itertools
import math

import numpy as np
import pytest

from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_logabs, rel_fro, relerr

rng = np.random.default_rng(7)


def randn(shape, dtype=np.float32):
    return rng.standard_normal(shape).astype(dtype)


def skew(A):
    return (A - np.swapaxes(A, -1, -2)).astype(A.dtype)


# --------------------------------------------------------------- reductions
def test_pairwise_tree_order():
    x = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    # (x0 + x2) + (x1 + x3) = 0 + 2, where a left-to-right float32 sum gives 1
    assert g.pairwise(x, np.add, 0) == np.float32(2.0)
    y = np.arange(1, 8, dtype=np.float64)
    assert g.pairwise(y, np.add, 0) == 28.0
    assert g.pairwise(np.array([-1.0, 2.0, -3.0]), np.multiply, 1) == 6.0


# --------------------------------------------------------------- slogdet
@pytest.mark.parametrize("n", [1, 3, 8, 40, 96])
def test_slogdet_generic_vs_float64(n):
    A = randn((6, n, n))
    s, l = g.slogdet_generic(A)
    s64, l64 = ref64.slogdet64(A)
    assert s.dtype == np.float32 and l.dtype == np.float32
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, "oracle", A)


def test_slogdet_generic_permutations_exact():
    n = 9
    for _ in range(20):
        p = rng.permutation(n)
        P = np.eye(n, dtype=np.float32)[p]
        s, l = g.slogdet_generic(P[None])
        inv = sum(1 for i, j in itertools.combinations(range(n), 2) if p[i] > p[j])
        assert s[0] == (-1.0) ** inv and l[0] == 0.0


def test_slogdet_generic_triangular_closed_form():
    n = 12
    for _ in range(10):
        d = randn(n)
        U = np.triu(randn((n, n)), 1) + np.diag(d)
        p = rng.permutation(n)
        A = U[p].astype(np.float32)
        inv = sum(1 for i, j in itertools.combinations(range(n), 2) if p[i] > p[j])
        s, l = g.slogdet_generic(A[None])
        assert s[0] == (-1.0) ** inv * np.prod(np.sign(d))
        assert abs(l[0] - np.sum(np.log(np.abs(d.astype(np.float64))))) < 1e-4


def test_slogdet_generic_singular():
    A = randn((3, 10, 10))
    A[0, :, 4] = 0.0
    A[1, 7, :] = 0.0
    s, l = g.slogdet_generic(A)
    assert s[0] == 0 and s[1] == 0 and np.isneginf(l[0]) and np.isneginf(l[1])
    assert np.isfinite(l[2])


# --------------------------------------------------------------- slogpf
@pytest.mark.parametrize("n", [2, 4, 6, 8, 10])
def test_slogpf_generic_vs_brute_force(n):
    S = skew(randn((5, n, n)))
    s, l = g.slogpf_generic(S)
    brute = np.array([ref64.pf_brute(x) for x in S])
    assert np.array_equal(s, np.sign(brute))
    assert np.allclose(l, np.log(np.abs(brute)), atol=1e-4)


@pytest.mark.parametrize("n", [16, 34, 64])
def test_slogpf_generic_invariants(n):
    S = skew(randn((4, n, n)))
    s, l = g.slogpf_generic(S)
    s64, l64 = ref64.slogpf64(S)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, "oracle", S)
    # pf(S)^2 = det(S)
    sd, ld = ref64.slogdet64(S)
    assert np.all(sd == 1.0)
    assert np.allclose(2 * l64, ld, atol=1e-8 * n)
    # pf(B S B^T) = det(B) pf(S)
    Bm = (randn((4, n, n)) / np.sqrt(n) + np.eye(n)).astype(np.float64)
    T = (Bm @ S.astype(np.float64) @ np.swapaxes(Bm, 1, 2)).astype(np.float32)
    T = (0.5 * (T - np.swapaxes(T, 1, 2))).astype(np.float32)
    st, lt = g.slogpf_generic(T)
    sb, lb = ref64.slogdet64(Bm)
    assert np.array_equal(st, s64 * sb)
    assert np.allclose(lt, l64 + lb, atol=5e-3 * max(1, n / 32))


def test_slogpf_generic_direct_sum_closed_form():
    n = 12
    for _ in range(5):
        a = randn(n // 2)
        S = np.zeros((n, n), np.float32)
        for i, v in enumerate(a):
            S[2 * i, 2 * i + 1] = v
            S[2 * i + 1, 2 * i] = -v
        p = rng.permutation(n)
        Pm = np.eye(n, dtype=np.float32)[p]
        T = (Pm @ S @ Pm.T).astype(np.float32)
        inv = sum(1 for i, j in itertools.combinations(range(n), 2) if p[i] > p[j])
        s, l = g.slogpf_generic(T[None])
        assert s[0] == np.prod(np.sign(a)) * (-1.0) ** inv
        assert abs(l[0] - np.sum(np.log(np.abs(a.astype(np.float64))))) < 1e-5


def test_slogpf_generic_singular():
    S = skew(randn((2, 12, 12)))
    S[0, 5, :] = 0.0
    S[0, :, 5] = 0.0
    s, l = g.slogpf_generic(S)
    assert s[0] == 0 and np.isneginf(l[0]) and np.isfinite(l[1])


# --------------------------------------------------------------- gradients
@pytest.mark.parametrize("n", [5, 24])
def test_lu_parts_generic_inverse(n):
    A = randn((4, n, n)) + 2 * np.eye(n, dtype=np.float32)
    s, l, invT, lu, perm, zero = g.lu_parts_generic(A)
    ref = np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1)
    assert np.all(rel_fro(invT, ref) < 1e-4)
    # P A = L U with perm
    Lm = np.tril(lu, -1) + np.eye(n)
    Um = np.triu(lu)
    PA = np.take_along_axis(A, perm[:, :, None].astype(np.int64), axis=1)
    assert np.allclose(Lm @ Um, PA, atol=1e-4)
    # primal equals the plain forward bitwise
    s0, l0 = g.slogdet_generic(A)
    assert np.array_equal(s, s0) and np.array_equal(l, l0)


def test_lu_parts_generic_finite_differences():
    n = 7
    A = rng.standard_normal((1, n, n)) + 2 * np.eye(n)
    _, _, invT, _, _, _ = g.lu_parts_generic(A)
    E = rng.standard_normal((n, n))
    h = 1e-6
    lp = g.slogdet_generic(A + h * E)[1][0]
    lm = g.slogdet_generic(A - h * E)[1][0]
    assert abs((lp - lm) / (2 * h) - np.sum(invT[0] * E)) < 1e-6


def test_lu_parts_generic_singular_zero_gradient():
    A = randn((2, 8, 8))
    A[0, :, 3] = 0.0
    s, l, invT, _, _, zero = g.lu_parts_generic(A)
    assert np.all(invT[0] == 0) and np.all(np.isfinite(invT))
    assert zero[0].any() and not zero[1].any()


@pytest.mark.parametrize("n", [6, 20])
def test_pf_parts_generic_inverse(n):
    S = skew(randn((3, n, n)))
    s, l, G, pfv = g.pf_parts_generic(S, False)
    assert np.all(rel_fro(G, np.linalg.inv(S.astype(np.float64))) < 1e-4)
    s0, l0 = g.slogpf_generic(S)
    assert np.array_equal(s, s0) and np.array_equal(l, l0)


@pytest.mark.parametrize("case", ["regular", "one_zero", "two_zero"])
def test_pf_parts_generic_adjugate_brute_force(case):
    n = 8
    S = skew(randn((3, n, n)))
    if case == "one_zero":
        S[:, 2, :] = 0.0
        S[:, :, 2] = 0.0
    if case == "two_zero":
        # a null row paired with a regular one: rank n-2 with two exact zero pivots
        S[:, 0, :] = 0.0
        S[:, :, 0] = 0.0
        S[:, 1, :] = 0.0
        S[:, :, 1] = 0.0
        S[:, 1, 5] = 1.0
        S[:, 5, 1] = -1.0
    _, _, G, pfv = g.pf_parts_generic(S, True)
    grad = -0.5 * G  # d pf / dS
    ref = np.stack([ref64.pf_grad_brute(x) for x in S])
    scale = max(np.abs(ref).max(), 1e-12)
    assert np.all(np.isfinite(G))
    assert np.max(np.abs(grad - ref)) < 1e-4 * scale
    assert np.allclose(pfv, [ref64.pf_brute(x) for x in S], atol=1e-4 * max(1, np.abs(pfv).max()))


@pytest.mark.parametrize("rank_def", [0, 1, 2])
def test_det_gradT_brute_force(rank_def):
    n = 6
    A = randn((3, n, n)).astype(np.float32)
    for r in range(rank_def):
        A[:, :, r] = 0.0  # exact zero columns -> exact zero pivots
    d, G = g.det_parts(A)
    ref = np.stack([ref64.adjT_brute(x) for x in A])
    assert np.all(np.isfinite(G))
    assert np.max(np.abs(G - ref)) < 1e-4 * max(np.abs(ref).max(), 1e-12) + 1e-6
    assert np.allclose(d, np.linalg.det(A.astype(np.float64)), rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("kind", ["regular", "zero_col", "zero_col_row", "two_cols", "near"])
def test_adjT_svd_vs_cofactors(kind):
    """The SVD adjugate (float64 truth for the GPU tests at any n) against cofactors."""
    n = 7
    A = randn((4, n, n)).astype(np.float64)
    if kind == "zero_col":
        A[:, :, 2] = 0.0
    if kind == "zero_col_row":
        A[:, :, 0] = 0.0
        A[:, 1, :] = 0.0
    if kind == "two_cols":
        A[:, :, 0] = 0.0
        A[:, :, 3] = 0.0
    if kind == "near":
        A[:, -1, :] = np.einsum("bi,bij->bj", randn((4, n - 1)).astype(np.float64), A[:, :-1, :])
    for a in A:
        ref = ref64.adjT_brute(a)
        got = ref64.adjT_svd(a)
        assert np.max(np.abs(got - ref)) <= 1e-9 * max(np.abs(ref).max(), 1.0)
    # a transposed result (adj(A) instead of adj(A)^T) fails on a generic member
    a = A[0]
    if kind == "regular":
        assert np.max(np.abs(ref64.adjT_svd(a).T - ref64.adjT_brute(a))) > 1e-3


@pytest.mark.parametrize("n", [4, 6, 8])
def test_pf_grad64_vs_brute(n):
    S = skew(randn((2, n, n))).astype(np.float64)
    S[1, 1, :] = 0.0
    S[1, :, 1] = 0.0
    for x in S:
        ref = ref64.pf_grad_brute(x)
        assert np.max(np.abs(ref64.pf_grad64(x) - ref)) <= 1e-9 * max(np.abs(ref).max(), 1.0)
    # rows variant: S[1] has row / column 1 zero, so only those entries are nonzero
    ref = ref64.pf_grad_brute(S[1])
    assert np.max(np.abs(ref64.pf_grad64_rows(S[1], [1]) - ref)) <= 1e-9 * max(np.abs(ref).max(), 1.0)
    # regular: d pf / dS = pf S^-T / 2
    x = S[0]
    want = 0.5 * ref64.pf64(x) * np.linalg.inv(x).T
    assert np.max(np.abs(ref64.pf_grad64(x) - want)) <= 1e-8 * np.abs(want).max()


def test_polynomials():
    for n in range(0, 5):
        A = randn((4, n, n))
        assert np.allclose(g.det_poly(A), np.linalg.det(A.astype(np.float64)) if n else 1.0, rtol=1e-5)
    for n in (2, 4, 6):
        S = skew(randn((4, n, n)))
        assert np.allclose(g.pf_poly(S), [ref64.pf_brute(x) for x in S], rtol=1e-5)


def test_ref64_self_consistency():
    """The float64 Parlett-Reid against brute force and pf^2 = det."""
    for n in (4, 8, 10):
        S = skew(randn((3, n, n))).astype(np.float64)
        for x in S:
            assert math.isclose(ref64.pf64(x), ref64.pf_brute(x), rel_tol=1e-10)
            assert math.isclose(ref64.pf64(x) ** 2, np.linalg.det(x), rel_tol=1e-9)


# --------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught():
    """Mutants of the oracle (planted here, on the CPU) fail the pins above."""
    n = 9
    p = np.array([1, 0, 2, 3, 4, 5, 6, 7, 8])
    P = np.eye(n, dtype=np.float32)[p][None]

    def slog_no_swaps(lu, piv):  # drops the swap parity
        d = np.diagonal(lu, axis1=-2, axis2=-1)
        sign = np.where(np.sum(d < 0, -1) % 2, -1.0, 1.0).astype(lu.dtype)
        return sign, g.pairwise(np.log(np.abs(d)), np.add, 0)

    lu, piv, _ = g.lu_factor(P)
    assert g.slog_from_lu(lu, piv)[0][0] == -1.0
    assert slog_no_swaps(lu, piv)[0][0] != -1.0

    # Parlett-Reid with a flipped rank-2 update sign
    S = skew(randn((3, 8, 8)))
    brute = np.array([ref64.pf_brute(x) for x in S])

    def pr_flipped(S):
        A = np.array(S)
        B, n, _ = A.shape
        sign = np.ones(B, A.dtype)
        log = np.zeros(B, A.dtype)
        idx = np.arange(n)[None, :]
        for k in range(n // 2):
            c = 2 * k
            A, kp, _, d, tau, w = g._pr_step(A, c, idx)
            A = A - 2 * (tau[:, :, None] * w[:, None, :] - w[:, :, None] * tau[:, None, :])
            sign = np.where(kp != c + 1, -sign, sign) * np.sign(d)
            log = log + np.log(np.abs(d))
        return sign, log

    s, l = pr_flipped(S)
    assert not np.allclose(s * np.exp(l), brute, rtol=1e-3)
    s, l = g.slogpf_generic(S)
    assert np.allclose(s * np.exp(l), brute, rtol=1e-4)

    # a transposed inverse is caught by the float64 inverse check
    A = randn((2, 6, 6)) + 2 * np.eye(6, dtype=np.float32)
    _, _, invT, _, _, _ = g.lu_parts_generic(A)
    ref = np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1)
    assert relerr(np.swapaxes(invT, 1, 2), ref) > 1e-2


# --------------------------------------------------------------- complex kinds
def crandn(shape, dtype=np.complex64):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(dtype)


@pytest.mark.parametrize("dtype", [np.complex64, np.complex128])
def test_complex_oracle_slogdet_and_inverse(dtype):
    """Complex slogdet of the oracle (reference _slog_from_lu's complex branch,
    _fallback.py:36-55: sign = parity * prod(d / |d|)) against numpy's complex128 slogdet,
    with sign of the input dtype and logabs of its real dtype; the closed form of a
    permuted diagonal (sign = parity * prod of the phases, logabs = sum log|d_i|); A^-T
    without conjugation (lu_parts, _fallback.py:63-97) against numpy's inverse; and a zero
    column gives (0, -inf) and a zero gradient."""
    tol = 1e-4 if dtype == np.complex64 else 1e-11
    for n in (1, 4, 17, 40):
        A = crandn((5, n, n), dtype)
        s, l = g.slogdet_generic(A)
        s64, l64 = ref64.slogdet64(A)
        assert s.dtype == dtype and l.dtype == np.finfo(dtype).dtype
        assert np.max(np.abs(s - s64)) < tol * max(1, n / 8)
        assert np.max(np.abs(l - l64)) < tol * max(1, n / 8)
        _, _, invT, _, _, _ = g.lu_parts_generic(A)
        ref = np.linalg.inv(A.astype(np.complex128)).transpose(0, 2, 1)
        assert relerr(invT, ref) < 100 * tol
        assert relerr(invT, ref.conj()) > 0.1  # not the conjugate
    n = 7
    d = crandn((n,), np.complex128)
    p = rng.permutation(n)
    M = (np.eye(n)[p] * d[p][:, None]).astype(dtype)  # row i = d[p[i]] e_p[i]
    s, l = g.slogdet_generic(M[None])
    inv = sum(1 for i, j in itertools.combinations(range(n), 2) if p[i] > p[j])
    phase = np.prod(d / np.abs(d)) * (-1) ** inv
    assert abs(s[0] - phase) < tol and abs(l[0] - np.sum(np.log(np.abs(d)))) < tol * n
    A = crandn((2, 6, 6), dtype)
    A[0, :, 2] = 0
    s, l, invT, _, _, _ = g.lu_parts_generic(A)
    assert s[0] == 0 and l[0] == -np.inf and np.all(invT[0] == 0) and abs(abs(s[1]) - 1) < tol


@pytest.mark.parametrize("dtype", [np.complex64, np.complex128])
def test_complex_oracle_slogpf(dtype):
    """Complex slogpf of the oracle (reference _slogpf_generic, _fallback.py:266-300, with
    sign(d) = d / |d|) against the perfect-matching Pfaffian (n <= 8), pf^2 = det at larger
    n, the closed form pf(a_1 J + ... + a_k J) = prod a_i, and a zero row / column (0, -inf)."""
    tol = 1e-4 if dtype == np.complex64 else 1e-11
    for n in (2, 4, 8):
        S = skew(crandn((4, n, n), dtype))
        s, l = g.slogpf_generic(S)
        brute = np.array([ref64.pf_brute(x) for x in S])
        assert np.max(np.abs(s * np.exp(l) - brute)) < tol * np.max(np.abs(brute)) * n
    S = skew(crandn((3, 30, 30), dtype))
    s, l = g.slogpf_generic(S)
    sd, ld = ref64.slogdet64(S)
    assert np.max(np.abs(s * s - sd)) < 10 * tol and np.max(np.abs(2 * l - ld)) < 10 * tol * 30
    a = crandn((4,), np.complex128)
    D = np.zeros((8, 8), np.complex128)
    for i in range(4):
        D[2 * i, 2 * i + 1], D[2 * i + 1, 2 * i] = a[i], -a[i]
    s, l = g.slogpf_generic(D.astype(dtype)[None])
    assert abs(s[0] * np.exp(l[0]) - np.prod(a)) < tol * abs(np.prod(a)) * 8
    S = skew(crandn((1, 6, 6), dtype))
    S[0, 3, :] = 0
    S[0, :, 3] = 0
    s, l = g.slogpf_generic(S)
    assert s[0] == 0 and l[0] == -np.inf


def test_complex_planted_mistakes_are_caught():
    """A complex sign without the pivot phases (the real parity rule applied to complex
    pivots) and a conjugated inverse fail the complex pins."""
    A = crandn((3, 6, 6), np.complex128)
    lu, piv, _ = g.lu_factor(A)
    s, _ = g.slog_from_lu(lu, piv)
    s64, _ = ref64.slogdet64(A)
    assert np.max(np.abs(s - s64)) < 1e-10
    d = np.diagonal(lu, axis1=-2, axis2=-1)
    no_phase = np.where(np.sum(piv != np.arange(6), -1) % 2, -1.0, 1.0)
    assert np.max(np.abs(no_phase - s64)) > 0.1
    _, _, invT, _, _, _ = g.lu_parts_generic(A)
    ref = np.linalg.inv(A).transpose(0, 2, 1)
    assert relerr(invT.conj(), ref) > 0.1 and relerr(invT, ref) < 1e-10
    assert np.all(np.abs(d) > 0)


@pytest.mark.parametrize("case", ["regular", "rank n-1", "rank n-2"])
def test_complex_adjT_svd_vs_cofactors(case):
    """The complex SVD adjugate (the float64 / complex truth of the det gradient) against
    cofactors, the closed form det(A) A^-T for regular A, and 0 at rank n - 2; a
    conjugated continuation fails the check."""
    n = 6
    A = crandn((n, n), np.complex128)
    if case != "regular":
        A[:, 2] = 0.3 * A[:, 0] - 1j * A[:, 4]
    if case == "rank n-2":
        A[:, 3] = A[:, 1]
    S = ref64.adjT_svd(A)
    C = ref64.adjT_brute(A)
    assert np.max(np.abs(S - C)) < 1e-10 * max(1.0, np.max(np.abs(C)))
    if case == "regular":
        ref = np.linalg.det(A) * np.linalg.inv(A).T
        assert np.max(np.abs(C - ref)) < 1e-10 * np.max(np.abs(ref))
        assert np.max(np.abs(C.conj() - ref)) > 0.1 * np.max(np.abs(ref))
    elif case == "rank n-1":
        assert np.max(np.abs(C)) > 1e-3
    else:
        assert np.max(np.abs(C)) < 1e-10


@pytest.mark.parametrize("case", ["regular", "one_zero", "two_zero", "three_zero"])
def test_complex_pf_adjugate_vs_minors(case):
    """The complex Pfaffian adjugate of the oracle (reference _pf_parts_generic with the
    complex pivots' phases, _fallback.py:101-263) against minor Pfaffians by the
    perfect-matching expansion (the holomorphic d pf / dS) -- the truth of the complex pf
    gradient -- with a conjugated result failing it."""
    n = 8
    S = crandn((3, n, n), np.complex128)
    S = S - np.swapaxes(S, 1, 2)
    if case == "one_zero":
        S[:, 2, :] = 0.0
        S[:, :, 2] = 0.0
    if case == "two_zero":  # rows 0 and 2 null: two exact zero pivots, rank n - 2
        for r in (0, 2):
            S[:, r, :] = 0.0
            S[:, :, r] = 0.0
    if case == "three_zero":  # rank n - 4: the adjugate is zero
        for r in (0, 2, 4):
            S[:, r, :] = 0.0
            S[:, :, r] = 0.0
    _, _, G, pfv = g.pf_parts_generic(S, True)
    grad = -0.5 * G
    ref = np.stack([ref64.pf_grad_brute(x) for x in S])
    assert np.allclose(pfv, [ref64.pf_brute(x) for x in S], atol=1e-10 * max(1, np.abs(pfv).max()))
    if case == "three_zero":
        assert np.all(ref == 0) and np.max(np.abs(grad)) == 0
        return
    scale = np.abs(ref).max()
    assert scale > 0
    assert np.max(np.abs(grad - ref)) < 1e-10 * scale
    assert np.max(np.abs(grad.conj() - ref)) > 1e-3 * scale
    if case == "regular":
        want = 0.5 * pfv[:, None, None] * np.linalg.inv(S).transpose(0, 2, 1)
        assert np.max(np.abs(ref - want)) < 1e-10 * scale
