"""GPU parity of det's gradient d det / dA = adj(A)^T for the float64 and complex kinds
(fx_det_parts_f64 / _c64 / _c128): the exact adjugate from the same Gauss-Jordan run as
the value, continued to singular A (one and two zero pivots, rank n - 1 and n - 2), against
the float64 / complex128 SVD adjugate and det(A) A^-T -- the reference's det gradient tests
for every dtype (tests/test_fermix.py:428-520)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import ref64
from tests.tolerances import relerr

pytestmark = pytest.mark.gpu

KINDS = {"f64": (np.float64, 1e-11), "c64": (np.complex64, 2e-5), "c128": (np.complex128, 1e-11)}


def _np(x):
    return x.detach().cpu().numpy()


def _near_identity(rng, B, n, dt):
    """I + N(0, 1/(4n)) (complex: both parts): det = O(1) at any n."""
    X = rng.standard_normal((B, n, n))
    if np.dtype(dt).kind == "c":
        X = X + 1j * rng.standard_normal((B, n, n))
    return (np.eye(n) + 0.5 * X / np.sqrt(n)).astype(dt)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [1, 3, 16, 60, 100, 200])
def test_det_grad_regular_64_and_complex(dev, kind, n):
    """Regular A: adj(A)^T against det(A) A^-T in 64-bit; the primal bit-identical to the
    plain slogdet forward; torch's gradient of Re sum det is conj(adj(A)^T) (adj(A)^T for
    float64), matching torch.linalg.det's own autograd on the CPU."""
    dt, tol = KINDS[kind]
    rng = np.random.default_rng(9100 + n)
    A = _near_identity(rng, 4, n, dt)
    print(f"det grad {kind} n={n}", flush=True)
    At = torch.from_numpy(A).to(dev)
    sign, logabs, adjT = _kernels.det_parts(At)
    s0, l0 = fermix_amd.slogdet(At)
    assert torch.equal(sign, s0) and torch.equal(logabs, l0), "det primal != forward"
    W = A.astype(np.complex128 if kind != "f64" else np.float64)
    ref = np.linalg.det(W)[:, None, None] * np.linalg.inv(W).transpose(0, 2, 1)
    assert relerr(_np(adjT), ref) < tol * max(1.0, n / 16)
    X = At.clone().requires_grad_(True)
    d = fermix_amd.det(X)
    assert torch.equal(d, s0 * torch.exp(l0))
    (gr,) = torch.autograd.grad(d.real.sum() if d.is_complex() else d.sum(), X)
    Xc = torch.from_numpy(W).requires_grad_(True)
    dc = torch.linalg.det(Xc)
    (grc,) = torch.autograd.grad(dc.real.sum() if dc.is_complex() else dc.sum(), Xc)
    assert relerr(_np(gr), grc.numpy()) < tol * max(1.0, n / 16)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [3, 8, 40, 130])
def test_det_grad_singular_64_and_complex(dev, kind, n):
    """Zero column (one zero pivot), zero row (the zero pivot at the end), zero matrix, two
    zero columns (rank n - 2: adj = 0), zero column 0 plus zero row 1 (rank n - 1 with two
    zero pivots) and a regular member, against the SVD adjugate."""
    dt, tol = KINDS[kind]
    rng = np.random.default_rng(9200 + n)
    A = _near_identity(rng, 6, n, dt)
    A[0, :, 1] = 0
    A[1, 2 % n] = 0
    A[2] = 0
    A[3, :, 0] = 0
    A[3, :, 1 % n] = 0
    A[4, :, 0] = 0
    A[4, 1 % n] = 0
    print(f"det singular {kind} n={n}", flush=True)
    X = torch.from_numpy(A).to(dev).requires_grad_(True)
    d = fermix_amd.det(X)
    (gr,) = torch.autograd.grad(d.real.sum() if d.is_complex() else d.sum(), X)
    gr = _np(gr)
    if kind != "f64":
        gr = gr.conj()  # torch's conjugate-Wirtinger gradient -> adj(A)^T
    assert np.all(np.isfinite(gr)) and np.all(_np(d)[:5] == 0)
    ref = np.stack([ref64.adjT_svd(a) for a in A])
    assert np.all(gr[2] == 0) and np.all(gr[3] == 0)
    for k in (0, 1, 4, 5):
        assert np.abs(ref[k]).max() > 0
        err = relerr(gr[k], ref[k])
        print(f"  member {k}: relerr {err:.3g}", flush=True)
        assert err < tol * max(1.0, n / 16), (k, err)
