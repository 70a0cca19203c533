"""GPU parity of the forward kernels (slogdet / slogpf) against the CPU oracle, float64
truth and the golden vectors, plus size-independent properties at the BASELINE sizes
(B = 4096, n = 128). Mirrors the reference's forward tests
(tests/test_fermix.py:148-228, 442-456, 608-647)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import KAPPA_C, U32, assert_logabs, kappa, logabs_tol

pytestmark = pytest.mark.gpu

DET_NS = [1, 2, 3, 5, 8, 15, 16, 17, 31, 32, 40, 48, 63, 64, 65, 80, 96, 100, 112, 127, 128]
PF_NS = [2, 4, 6, 8, 10, 14, 16, 18, 32, 34, 48, 64, 66, 96, 100, 126, 128]


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def skew(A):
    return (A - np.swapaxes(A, -1, -2)).astype(np.float32)


@pytest.mark.parametrize("n", DET_NS)
def test_slogdet_vs_oracle_and_float64(dev, n):
    rng = np.random.default_rng(100 + n)
    A = rng.standard_normal((64, n, n)).astype(np.float32)
    print(f"slogdet n={n} B=64", flush=True)
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    s64, l64 = ref64.slogdet64(A)
    so, lo = g.slogdet_generic(A)
    assert s.dtype == np.float32 and l.dtype == np.float32
    assert np.array_equal(s, s64)
    assert np.array_equal(s, so)
    assert_logabs(l, l64, n, "vs float64", A)
    assert_logabs(l, lo, n, "vs oracle", A)


@pytest.mark.parametrize("n", [3, 8, 17, 40, 96, 128])
def test_slogdet_golden(dev, golden, n):
    A = golden[f"det_n{n}_a"]
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    assert np.array_equal(s, golden[f"det_n{n}_sign"])
    assert_logabs(l, golden[f"det_n{n}_logabs"], n, "golden", A)


def test_slogdet_singular_and_special(dev):
    n = 24
    rng = np.random.default_rng(5)
    A = rng.standard_normal((6, n, n)).astype(np.float32)
    A[0, :, 3] = 0.0  # zero column
    A[1, 5, :] = 0.0  # zero row
    A[2] = 0.0  # zero matrix
    A[3] = np.eye(n, dtype=np.float32)[rng.permutation(n)]  # permutation
    A[4] = -np.eye(n, dtype=np.float32)
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    for i in range(3):
        assert s[i] == 0 and np.isneginf(l[i])
    s64, l64 = ref64.slogdet64(A[3:])
    assert np.array_equal(s[3:], s64)
    assert l[3] == 0.0 and l[4] == 0.0 and s[4] == 1.0
    assert np.isfinite(l[5])


def test_slogdet_batch_dims_and_empty(dev):
    rng = np.random.default_rng(9)
    A = rng.standard_normal((2, 3, 7, 7)).astype(np.float32)
    s, l = fermix_amd.slogdet(_t(A, dev))
    assert s.shape == (2, 3) and l.shape == (2, 3)
    s2, l2 = fermix_amd.slogdet(_t(A.reshape(6, 7, 7), dev))
    assert torch.equal(s.reshape(6), s2) and torch.equal(l.reshape(6), l2)
    s0, l0 = fermix_amd.slogdet(torch.zeros((4, 0, 0), device=dev))
    assert torch.all(s0 == 1) and torch.all(l0 == 0)
    s0, l0 = fermix_amd.slogdet(torch.zeros((0, 5, 5), device=dev))
    assert s0.shape == (0,)


def test_slogdet_batch_invariance_c1(dev):
    """C1 size: B = 4096, n = 128. Every member is bit-identical to the same matrix in a
    batch of 1 (the kernels never depend on B), and matches float64 truth."""
    rng = np.random.default_rng(0)
    A = rng.standard_normal((4096, 128, 128)).astype(np.float32)
    At = _t(A, dev)
    s, l = map(_np, fermix_amd.slogdet(At))
    idx = [0, 1, 777, 2048, 4095]
    for i in idx:
        si, li = map(_np, fermix_amd.slogdet(At[i : i + 1]))
        assert si[0] == s[i] and li[0] == l[i]
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, 128, "C1 vs float64", A)
    so, lo = g.slogdet_generic(A[:512])
    assert np.array_equal(s[:512], so)
    assert_logabs(l[:512], lo, 128, "C1 vs oracle", A[:512])


def test_lu_factors_reconstruct(dev):
    """The factors export: P A' = L U in float64, primal bit-identical to the forward."""
    rng = np.random.default_rng(11)
    for n in (5, 16, 50, 128):
        A = rng.standard_normal((8, n, n)).astype(np.float32)
        A[0, :, 1] = 0.0
        At = _t(A, dev)
        s, l, _, lu, perm = _kernels.slogdet_parts(At, want_inv=False, want_lu=True)
        s0, l0 = fermix_amd.slogdet(At)
        assert torch.equal(s, s0) and torch.equal(l, l0)
        lu = _np(lu).astype(np.float64)
        perm = _np(perm)
        N = lu.shape[-1]
        Ap = np.zeros((8, N, N))
        Ap[:, :n, :n] = A
        Ap[:, n:, n:] = np.eye(N - n)
        L = np.tril(lu, -1) + np.eye(N)
        U = np.triu(lu)
        PA = np.take_along_axis(Ap, perm[:, :, None].astype(np.int64), axis=1)
        for b in range(8):
            assert sorted(perm[b]) == list(range(N))
            err = np.abs(L[b] @ U[b] - PA[b]).max()
            assert err < 1e-4 * max(1.0, n / 16), (n, b, err)
            assert np.all(np.abs(L[b]) <= 1.0 + 1e-6)  # partial pivoting bound


@pytest.mark.parametrize("n", PF_NS)
def test_slogpf_vs_oracle_and_float64(dev, n):
    rng = np.random.default_rng(300 + n)
    S = skew(rng.standard_normal((48, n, n)))
    print(f"slogpf n={n} B=48", flush=True)
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    s64, l64 = ref64.slogpf64(S)
    so, lo = g.slogpf_generic(S)
    assert np.array_equal(s, s64)
    assert np.array_equal(s, so)
    assert_logabs(l, l64, n, "vs float64", S)
    assert_logabs(l, lo, n, "vs oracle", S)
    if n <= 10:
        brute = np.array([ref64.pf_brute(x) for x in S])
        assert np.array_equal(s, np.sign(brute))


@pytest.mark.parametrize("n", [4, 6, 10, 34, 64, 128])
def test_slogpf_golden(dev, golden, n):
    S = golden[f"pf_n{n}_s"]
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    assert np.array_equal(s, golden[f"pf_n{n}_sign"])
    assert_logabs(l, golden[f"pf_n{n}_logabs"], n, "golden", S)


def test_slogpf_skew_symmetrize_and_odd(dev):
    rng = np.random.default_rng(21)
    A = rng.standard_normal((5, 20, 20)).astype(np.float32)
    s, l = map(_np, fermix_amd.slogpf(_t(A, dev)))
    S = ((A - np.swapaxes(A, 1, 2)) * np.float32(0.5)).astype(np.float32)
    s64, l64 = ref64.slogpf64(S)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, 20, "skew", S)
    so, lo = map(_np, fermix_amd.slogpf(_t(A[:, :7, :7], dev)))
    assert np.all(so == 0) and np.all(np.isneginf(lo))
    p = _np(fermix_amd.pf(_t(A[:, :7, :7], dev)))
    assert np.all(p == 0)


def test_slogpf_singular(dev):
    rng = np.random.default_rng(22)
    S = skew(rng.standard_normal((3, 18, 18)))
    S[0, 4, :] = 0.0
    S[0, :, 4] = 0.0
    S[1] = 0.0
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    assert s[0] == 0 and np.isneginf(l[0]) and s[1] == 0 and np.isneginf(l[1])
    assert np.isfinite(l[2])


def test_slogpf_c2_properties(dev):
    """C2 size: B = 4096, n = 128, S = A - A^T. (S - S^T)/2 = S exactly, so the
    skew-symmetrised call is bit-identical to the plain one; pf^2 = det checks every
    member against the slogdet kernel; a subset against float64 and the oracle."""
    rng = np.random.default_rng(1)
    A = rng.standard_normal((4096, 128, 128)).astype(np.float32)
    S = skew(A)
    St = _t(S, dev)
    s1, l1 = fermix_amd.slogpf(St, skew_symmetrize=False)
    s2, l2 = fermix_amd.slogpf(St, skew_symmetrize=True)
    assert torch.equal(s1, s2) and torch.equal(l1, l2)
    sd, ld = map(_np, fermix_amd.slogdet(St))
    l1 = _np(l1)
    assert np.all(sd == 1.0)
    err = np.abs(2 * l1.astype(np.float64) - ld)
    bad = err > 2 * logabs_tol(ld / 2, 128)
    print(f"pf^2 = det literal pass {int((~bad).sum())}/4096", flush=True)
    if bad.any():
        assert np.all(err[bad] <= 2 * KAPPA_C * U32 * kappa(S[bad]))
    s64, l64 = ref64.slogpf64(S[:256])
    assert np.array_equal(_np(s1)[:256], s64)
    assert_logabs(l1[:256], l64, 128, "C2 vs float64", S[:256])
    so, lo = g.slogpf_generic(S[:128])
    assert_logabs(l1[:128], lo, 128, "C2 vs oracle", S[:128])
    for i in (0, 4095):
        si, li = map(_np, fermix_amd.slogpf(St[i : i + 1], skew_symmetrize=False))
        assert si[0] == _np(s1)[i] and li[0] == l1[i]


def test_pf_factors_reconstruct(dev):
    """P S' P^T = L D L^T from the exported factors (float64 assembly)."""
    rng = np.random.default_rng(23)
    for n in (6, 16, 40, 128):
        S = skew(rng.standard_normal((4, n, n)))
        St = _t(S, dev)
        s, l, gbuf, d, perm = _kernels.slogpf_factors(St, False)
        s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
        assert torch.equal(s, s0) and torch.equal(l, l0)
        gbuf, d, perm = _np(gbuf).astype(np.float64), _np(d).astype(np.float64), _np(perm)
        N = perm.shape[1]
        Sp = np.zeros((4, N, N))
        Sp[:, :n, :n] = S
        for t in range((N - n) // 2):
            Sp[:, n + 2 * t, n + 2 * t + 1] = 1.0
            Sp[:, n + 2 * t + 1, n + 2 * t] = -1.0
        for b in range(4):
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
            err = np.abs(L @ D @ L.T - P).max()
            assert err < 1e-4 * max(1.0, n / 16), (n, b, err)
