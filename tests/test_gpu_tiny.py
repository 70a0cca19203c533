"""GPU parity of the n <= 32 kernels (several matrices per wave, one lane per row):
batch tails that leave part of a workgroup empty, unaligned inputs (the scalar-load
path), exact singular cases and permutation parities, and the factor exports the
gradients consume (P A' = L U, P S' P^T = L D L^T)."""

import itertools

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs

pytestmark = pytest.mark.gpu


def _np(x):
    return x.detach().cpu().numpy()


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _unaligned(x, dev):
    """A contiguous device tensor equal to x whose data pointer is 4 bytes past a 16-byte
    boundary."""
    flat = torch.empty(x.size + 1, dtype=torch.float32, device=dev)
    v = flat[1:].view(x.shape)
    v.copy_(torch.from_numpy(np.ascontiguousarray(x)))
    assert v.data_ptr() % 16 == 4
    return v


def skew(A):
    return (A - np.swapaxes(A, -1, -2)).astype(np.float32)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 12, 16, 17, 24, 31, 32])
@pytest.mark.parametrize("B", [1, 5, 17, 33])
def test_slogdet_tiny_tails(dev, n, B):
    rng = np.random.default_rng(9000 + 100 * n + B)
    A = rng.standard_normal((B, n, n)).astype(np.float32)
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, f"tiny B={B}", A)
    su, lu = map(_np, fermix_amd.slogdet(_unaligned(A, dev)))
    assert np.array_equal(su, s) and np.array_equal(lu, l)  # same arithmetic either way


@pytest.mark.parametrize("n", [2, 4, 6, 12, 14, 16])
@pytest.mark.parametrize("B", [1, 5, 17])
def test_slogpf_tiny_tails(dev, n, B):
    rng = np.random.default_rng(9500 + 100 * n + B)
    A = rng.standard_normal((B, n, n)).astype(np.float32)
    S = skew(A)
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    s64, l64 = ref64.slogpf64(S)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, f"tiny pf B={B}", S)
    so, lo = g.slogpf_generic(S)
    assert np.array_equal(s, so)
    su, lu = map(_np, fermix_amd.slogpf(_unaligned(S, dev), skew_symmetrize=False))
    assert np.array_equal(su, s) and np.array_equal(lu, l)
    # skew_symmetrize on a: (a - a^T) / 2 = S / 2 exactly, so log|pf| drops by (n/2) log 2
    s2, l2 = map(_np, fermix_amd.slogpf(_t(A, dev)))
    assert np.array_equal(s2, s)
    assert np.all(np.abs(l2 - (l - 0.5 * n * np.log(2.0))) < 1e-5 * np.maximum(1, np.abs(l)) + 1e-6 * n)


def test_slogdet_tiny_exact_cases(dev):
    """Permutation matrices (sign = parity, logabs = 0 exactly), triangular matrices
    (logabs = sum log|diag|), exact zero pivots from a zero first, middle or last column
    or a zero last row, and the zero matrix."""
    n = 6
    perms = list(itertools.permutations(range(n)))[::37]
    P = np.stack([np.eye(n, dtype=np.float32)[list(p)] for p in perms])
    s, l = map(_np, fermix_amd.slogdet(_t(P, dev)))
    par = np.array([np.linalg.det(x) for x in P.astype(np.float64)])
    assert np.array_equal(s, np.sign(par).astype(np.float32)) and np.all(l == 0)
    rng = np.random.default_rng(9900)
    for n in (5, 16, 29):
        T = np.triu(rng.standard_normal((4, n, n))).astype(np.float32)
        s, l = map(_np, fermix_amd.slogdet(_t(T, dev)))
        d = np.diagonal(T, axis1=1, axis2=2).astype(np.float64)
        assert np.array_equal(s, np.prod(np.sign(d), axis=1).astype(np.float32))
        assert np.all(np.abs(l - np.sum(np.log(np.abs(d)), axis=1)) < 1e-5 * n)
        A = rng.standard_normal((5, n, n)).astype(np.float32)
        A[0, :, 0] = 0.0
        A[1, :, n // 2] = 0.0
        A[2, :, n - 1] = 0.0
        A[3, n - 1] = 0.0
        A[4] = 0.0
        s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
        assert np.all(s == 0) and np.all(np.isneginf(l))


def test_slogpf_tiny_exact_cases(dev):
    """pf(diag(a_i J)) = prod a_i; a symmetric permutation of it flips the sign by the
    permutation's parity; a zero row / column gives (0, -inf)."""
    rng = np.random.default_rng(9910)
    J = np.array([[0.0, 1.0], [-1.0, 0.0]])
    for n in (2, 8, 16):
        a = rng.uniform(0.5, 2.0, (6, n // 2)) * rng.choice([-1.0, 1.0], (6, n // 2))
        S = np.stack([np.kron(np.diag(x), J) for x in a]).astype(np.float32)
        perms = [rng.permutation(n) for _ in range(6)]
        Sp = np.stack([S[b][np.ix_(p, p)] for b, p in enumerate(perms)])
        s, l = map(_np, fermix_amd.slogpf(_t(Sp, dev), skew_symmetrize=False))
        parity = np.array([np.linalg.det(np.eye(n)[p]) for p in perms])
        want = parity * np.prod(a, axis=1)
        assert np.array_equal(s, np.sign(want).astype(np.float32))
        assert np.all(np.abs(l - np.log(np.abs(want))) < 1e-5 * n)
        Z = skew(rng.standard_normal((3, n, n)))
        Z[0, 0, :] = Z[0, :, 0] = 0.0
        Z[1, n - 1, :] = Z[1, :, n - 1] = 0.0
        Z[2] = 0.0
        s, l = map(_np, fermix_amd.slogpf(_t(Z, dev), skew_symmetrize=False))
        assert np.all(s == 0) and np.all(np.isneginf(l))


@pytest.mark.parametrize("n", [3, 9, 16, 20, 32])
def test_lu_tiny_factors_reconstruct(dev, n):
    rng = np.random.default_rng(9920 + n)
    B = 7
    A = rng.standard_normal((B, n, n)).astype(np.float32)
    A[0, :, n // 2] = 0.0
    At = _t(A, dev)
    s, l, _, lu, perm = _kernels.slogdet_parts(At, want_inv=False, want_lu=True)
    s0, l0 = fermix_amd.slogdet(At)
    assert torch.equal(s, s0) and torch.equal(l, l0)
    lu = _np(lu).astype(np.float64)
    perm = _np(perm)
    N = lu.shape[-1]
    Ap = np.zeros((B, N, N))
    Ap[:, :n, :n] = A
    Ap[:, n:, n:] = np.eye(N - n)
    L = np.tril(lu, -1) + np.eye(N)
    U = np.triu(lu)
    PA = np.take_along_axis(Ap, perm[:, :, None].astype(np.int64), axis=1)
    for b in range(B):
        assert sorted(perm[b]) == list(range(N))
        assert np.abs(L[b] @ U[b] - PA[b]).max() < 1e-4 * max(1.0, n / 16)
        assert np.all(np.abs(L[b]) <= 1.0 + 1e-6)


@pytest.mark.parametrize("n", [2, 6, 12, 16])
def test_pf_tiny_factors_reconstruct(dev, n):
    rng = np.random.default_rng(9930 + n)
    B = 5
    S = skew(rng.standard_normal((B, n, n)))
    St = _t(S, dev)
    s, l, gbuf, d, perm = _kernels.slogpf_factors(St, False)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert torch.equal(s, s0) and torch.equal(l, l0)
    gbuf, d, perm = _np(gbuf).astype(np.float64), _np(d).astype(np.float64), _np(perm)
    N = perm.shape[1]
    Sp = np.zeros((B, N, N))
    Sp[:, :n, :n] = S
    for t in range((N - n) // 2):
        Sp[:, n + 2 * t, n + 2 * t + 1] = 1.0
        Sp[:, n + 2 * t + 1, n + 2 * t] = -1.0
    for b in range(B):
        P = Sp[b][np.ix_(perm[b], perm[b])]
        L = np.eye(N)
        D = np.zeros((N, N))
        for s_ in range(N // 2):
            k, t = divmod(s_, 8)
            a, p = 2 * s_, 2 * s_ + 1
            D[a, p], D[p, a] = d[b, s_], -d[b, s_]
            rows = np.arange(p + 1, N)
            og = perm[b, rows]
            L[rows, a] = gbuf[b, k, og, 2 * t + 1] / d[b, s_]
            L[rows, p] = gbuf[b, k, og, 2 * t]
        assert np.abs(L @ D @ L.T - P).max() < 1e-4 * max(1.0, n / 16), (n, b)


@pytest.mark.parametrize("n", [1, 2, 3, 8, 16, 20, 31, 32])
@pytest.mark.parametrize("B", [1, 9, 33])
def test_slogdet_tiny_gradient(dev, n, B):
    """A^-T from the one-pass Gauss-Jordan kernel: against float64 and the oracle, the
    primal bit-identical to the forward, unaligned input giving the same bits."""
    rng = np.random.default_rng(9940 + 10 * n + B)
    A = (rng.standard_normal((B, n, n)) + 2 * np.eye(n)).astype(np.float32)
    s, l, invT, _, _ = _kernels.slogdet_parts(_t(A, dev))
    s0, l0 = fermix_amd.slogdet(_t(A, dev))
    assert torch.equal(s, s0) and torch.equal(l, l0), "parts primal != forward"
    su, lu_, invu, _, _ = _kernels.slogdet_parts(_unaligned(A, dev))
    assert torch.equal(su, s) and torch.equal(lu_, l) and torch.equal(invu, invT)
    ref = np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2)
    assert_grad(_np(invT), ref, A, f"tiny invT n={n} B={B}")
    _, _, invo, _, _, _ = g.lu_parts_generic(A)
    assert_grad(_np(invT), invo, A, f"tiny invT n={n} vs oracle")


def test_slogdet_tiny_gradient_singular(dev):
    """Exact zero pivots: zero gradient (zero_singular), or (zero_singular=False) the
    finite inverse of A~ = P^T L U~. A~ depends on which row takes the zero pivot (this
    library, like the reference's kernels, picks the lowest original row; LAPACK the
    lowest current position), so it is checked against this library's LU -> inverse path
    on the same pivots, and through the factorization-free property that A~ differs from
    A in one column: I - A A~^-1 has rank one."""
    rng = np.random.default_rng(9950)
    for n in (4, 13, 16, 27):
        A = rng.standard_normal((4, n, n)).astype(np.float32)
        A[0, :, 2] = 0.0
        A[2, n - 1, :] = 0.0
        At = _t(A, dev).requires_grad_()
        _, l = fermix_amd.slogdet(At)
        (gr,) = torch.autograd.grad(l[1] + l[3], At)
        gr = _np(gr)
        assert np.all(np.isfinite(gr)) and np.all(gr[0] == 0) and np.all(gr[2] == 0)
        ref = np.linalg.inv(A[[1, 3]].astype(np.float64)).swapaxes(-1, -2)
        assert_grad(gr[[1, 3]], ref, A[[1, 3]], f"tiny singular batch n={n}")
        _, _, inv2, _, _ = _kernels.slogdet_parts(_t(A, dev), zero_singular=False)
        inv2 = _np(inv2)
        # the general path (LU factors requested) runs the same pivots
        _, _, inv3, _, _ = _kernels.slogdet_parts(_t(A, dev), zero_singular=False, want_lu=True)
        inv3 = _np(inv3)
        assert np.all(np.isfinite(inv2))
        for b in (0, 2):
            assert np.max(np.abs(inv2[b] - inv3[b])) <= 1e-4 * max(1.0, np.abs(inv3[b]).max())
            D = np.eye(n) - A[b].astype(np.float64) @ inv2[b].T.astype(np.float64)
            sv = np.linalg.svd(D, compute_uv=False)
            assert sv[1] <= 1e-4 * (1.0 + sv[0]), (n, b, sv[:3])
