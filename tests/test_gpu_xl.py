"""GPU parity beyond the C4 regime (the larger orders): the LU path for
1024 < n <= 4096 (panel factored in place in the work buffer) and the Parlett-Reid path
for 2048 < n <= 4096 (16-column blocks), forward and gradients, against float64 truth.

Pfaffian truth at these sizes comes from the closed form pf(B J B^T) = det(B) pf(J) =
det(B) (J = diag([[0, 1], [-1, 0]])), with det(B) from float64 LAPACK."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def _near_identity(rng, B, n):
    return np.eye(n) + 0.5 * rng.standard_normal((B, n, n)) / np.sqrt(n)


def _bjb(rng, B, n):
    """(S float32, sign, logabs, S float64) with S = X J X^T, X = I + N(0, 1/(4n))."""
    X = _near_identity(rng, B, n)
    J = np.kron(np.eye(n // 2), np.array([[0.0, 1.0], [-1.0, 0.0]]))
    S64 = X @ J @ X.swapaxes(-1, -2)
    S = S64.astype(np.float32)
    S = (0.5 * (S - S.swapaxes(-1, -2))).astype(np.float32)  # exactly skew in float32
    sgn, lab = np.linalg.slogdet(X)
    return S, sgn, lab, S.astype(np.float64)


@pytest.mark.parametrize("n", [1025, 1536, 2048, 3000, 4096])
def test_slogdet_xl(dev, n):
    B = 3 if n <= 2048 else 2
    rng = np.random.default_rng(8000 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    A[-1, :, n // 3] = 0.0  # exact zero pivot
    print(f"slogdet xl n={n} B={B}", flush=True)
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, "vs float64", A)
    if n <= 2048:
        so, lo = g.slogdet_generic(A)
        assert np.array_equal(s, so)
        assert_logabs(l, lo, n, "vs oracle", A)


@pytest.mark.parametrize("n", [1100, 2048, 4096])
def test_slogdet_grad_xl(dev, n):
    B = 2
    rng = np.random.default_rng(8100 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    print(f"slogdet grad xl n={n}", flush=True)
    s, l, invT, _, _ = _kernels.slogdet_parts(_t(A, dev))
    s0, l0 = fermix_amd.slogdet(_t(A, dev))
    assert torch.equal(s, s0) and torch.equal(l, l0), "parts primal != forward"
    ref = np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2)
    assert_grad(_np(invT), ref, A, f"n={n} vs float64")


def test_det_adjugate_xl(dev):
    """n = 2048: a regular member (adj(A) A = det I in float64) and a zero-column member
    (only that column of adj(A)^T is nonzero, against the float64 SVD adjugate)."""
    rng = np.random.default_rng(8200)
    n = 2048
    A = _near_identity(rng, 2, n).astype(np.float32)
    A[1, :, 700] = 0.0
    At = _t(A, dev).requires_grad_()
    d = fermix_amd.det(At)
    (gr,) = torch.autograd.grad(d.sum(), At)
    gr = _np(gr)
    assert np.all(np.isfinite(gr)) and _np(d)[1] == 0
    A64 = A.astype(np.float64)
    d64 = np.linalg.det(A64[0])
    assert np.abs(gr[0].astype(np.float64).T @ A64[0] - d64 * np.eye(n)).max() < 1e-4 * abs(d64)
    assert np.all(gr[1][:, :700] == 0) and np.all(gr[1][:, 701:] == 0)
    col = ref64.adjT_svd(A[1])[:, 700]
    assert np.max(np.abs(gr[1][:, 700] - col)) < 1e-4 * np.abs(col).max()


@pytest.mark.parametrize("n", [2050, 3000, 4096])
def test_slogpf_xl(dev, n):
    B = 2
    rng = np.random.default_rng(8300 + n)
    S, sgn, lab, _ = _bjb(rng, B, n)
    Sz = S.copy()
    Sz[1, n // 5, :] = 0.0
    Sz[1, :, n // 5] = 0.0
    print(f"slogpf xl n={n}", flush=True)
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    assert np.array_equal(s, sgn)
    assert_logabs(l, lab, n, "vs det(X)", S)
    # |pf|^2 = |det| against float64 LAPACK on the rounded matrix
    _, ld64 = np.linalg.slogdet(S.astype(np.float64))
    assert np.all(np.abs(2 * l - ld64) < 1e-5 * np.abs(ld64) + 2e-6 * n)
    sz, lz = map(_np, fermix_amd.slogpf(_t(Sz, dev), skew_symmetrize=False))
    assert sz[1] == 0 and np.isneginf(lz[1]) and sz[0] == sgn[0]


@pytest.mark.parametrize("n", [1000, 2176, 4096])
def test_slogpf_grad_xl(dev, n):
    """S^-1 (inverse mode) and pf S^-1 (adjugate mode) from the 64-column-block (n = 1000,
    padded to 1024) and 16-column-block factors."""
    B = 2
    rng = np.random.default_rng(8400 + n)
    S, sgn, lab, S64 = _bjb(rng, B, n)
    print(f"slogpf grad xl n={n}", flush=True)
    s, l, Sinv = _kernels.slogpf_parts(_t(S, dev), False)
    s0, l0 = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False)
    assert torch.equal(s, s0) and torch.equal(l, l0)
    inv64 = np.linalg.inv(S64)
    assert_grad(_np(Sinv), inv64, S, f"n={n} S^-1 vs float64")
    _, _, adj = _kernels.slogpf_parts(_t(S, dev), False, adjugate=True)
    pf = sgn * np.exp(lab)
    assert_grad(_np(adj), pf[:, None, None] * inv64, S, f"n={n} pf S^-1 vs float64")
