"""GPU parity above n = 4096 (the float32 blocked kernels up to n = 8192: LU panels of
8192 rows -- forced, the LU's default there being the field-generic kernels -- and
8-column Parlett-Reid blocks), forward and gradients, against float64 truth
formed on the GPU in float64 (slogdet by torch.linalg; the inverses through their float64
residuals M X - I, which bound the relative error of X as M^-1). The inputs are well
conditioned (I + N(0, 1/(4n)), and X J X^T for the Pfaffian, whose value is det(X) pf(J) =
det(X)), so the literal bars hold and the float32 results are compared member by member;
one member of the forward batch has an exact zero pivot."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels, _tune
from tests.tolerances import assert_logabs

pytestmark = pytest.mark.gpu


def _near_identity(dev, B, n, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    X = torch.randn((B, n, n), generator=g, dtype=torch.float64)
    return (torch.eye(n, dtype=torch.float64) + 0.5 * X / np.sqrt(n)).to(dev)


def _inv_residual(M, X):
    """||M X - I||_F / sqrt(n) per member, in float64 on the GPU: a bound on the relative
    2-norm error of X as M^-1 (X - M^-1 = M^-1 (M X - I))."""
    n = M.shape[-1]
    R = torch.matmul(M.to(torch.float64), X.to(torch.float64)) - torch.eye(n, dtype=torch.float64, device=M.device)
    return (torch.linalg.norm(R.flatten(1), dim=1) / np.sqrt(n)).cpu().numpy()


def _jmat(n, dev):
    J = torch.zeros((n, n), dtype=torch.float64, device=dev)
    idx = torch.arange(0, n, 2, device=dev)
    J[idx, idx + 1] = 1.0
    J[idx + 1, idx] = -1.0
    return J


@pytest.mark.parametrize("n,prec,family", [(4160, "bf16x3", None), (4160, "ieee", "blocked"), (8192, "bf16x3", None),
                                           (8192, "bf16x3", "blocked")])
def test_slogdet_xxl(dev, n, prec, family):
    """Above lu_generic_above_n (4096) the LU runs the field-generic kernels; family
    "blocked" keeps the float32 blocked LU (panels of up to 8192 rows) under test."""
    if family:
        with _tune.force_family(family):
            return test_slogdet_xxl(dev, n, prec, None)
    B = 2
    A64 = _near_identity(dev, B, n, 9600 + n)
    A64[1, :, n // 3] = 0.0  # exact zero pivot
    A = A64.to(torch.float32)
    print(f"slogdet xxl n={n} prec={prec} family={_tune.kernel_family(n)}", flush=True)
    s, l = fermix_amd.slogdet(A, prec=prec)
    s64, l64 = torch.linalg.slogdet(A.to(torch.float64))
    assert torch.equal(s.cpu().to(torch.float64), s64.cpu())
    assert_logabs(l.cpu().numpy(), l64.cpu().numpy(), n, f"n={n} {prec} vs float64")
    # the gradient: A^-T of the regular member, and the primal of the parts run
    sp, lp, invT, _, _ = _kernels.slogdet_parts(A[:1].contiguous(), x3=1 if prec == "bf16x3" else 0)
    assert torch.equal(sp, s[:1]) and torch.equal(lp, l[:1]), "parts primal != forward"
    err = _inv_residual(A[:1].transpose(1, 2), invT)
    print(f"  A^-T residual {err}", flush=True)
    assert np.all(err < 1e-5)


@pytest.mark.parametrize("n", [4160, 8192])
def test_slogpf_xxl(dev, n):
    """pf(X J X^T) = det(X): sign and logabs against float64 det(X) on the GPU; S^-1 and
    pf(S) S^-1 against the float64 inverse; a zero row / column gives pf = 0."""
    B = 1
    X = _near_identity(dev, B, n, 9700 + n)
    S64 = X @ _jmat(n, dev) @ X.transpose(1, 2)
    S = S64.to(torch.float32)
    S = (0.5 * (S - S.transpose(1, 2))).contiguous()  # exactly skew in float32
    sgn, lab = torch.linalg.slogdet(X)
    print(f"slogpf xxl n={n}", flush=True)
    s, l = fermix_amd.slogpf(S, skew_symmetrize=False)
    assert torch.equal(s.cpu().to(torch.float64), sgn.cpu())
    assert_logabs(l.cpu().numpy(), lab.cpu().numpy(), n, f"n={n} vs det(X)")
    sp, lp, Sinv = _kernels.slogpf_parts(S, False)
    assert torch.equal(sp, s) and torch.equal(lp, l)
    err = _inv_residual(S, Sinv)
    print(f"  S^-1 residual {err}", flush=True)
    assert np.all(err < 1e-5)
    # the adjugate over this factorisation's own pf (pf of the float32-rounded S, which
    # differs from det(X) by the rounding of S)
    _, _, adj = _kernels.slogpf_parts(S, False, adjugate=True)
    pf = (s.to(torch.float64) * torch.exp(l.to(torch.float64)))[:, None, None]
    err = _inv_residual(S, adj.to(torch.float64) / pf)
    print(f"  pf S^-1 / pf residual {err}", flush=True)
    assert np.all(err < 1e-5)
    del adj, Sinv
    Sz = S.clone()
    Sz[0, n // 5, :] = 0.0
    Sz[0, :, n // 5] = 0.0
    sz, lz = fermix_amd.slogpf(Sz, skew_symmetrize=False)
    assert sz.item() == 0 and torch.isneginf(lz).item()


def test_det_grad_xxl(dev):
    """n = 4160: det's gradient adj(A)^T for a regular member (A^T adj(A)^T / det = I, the
    float64 residual) and for a member with a zero column k (rank n - 1: only column k of
    adj(A)^T is nonzero, and v . adj(A)^T[:, k] = det(A with column k := v) for any v,
    checked with v = the column that was zeroed -- well conditioned for this near-identity
    A -- against float64 det on the GPU)."""
    n, k = 4160, 1234
    A64 = _near_identity(dev, 2, n, 9800)
    v = A64[1, :, k].clone()
    A64[1, :, k] = 0.0
    A = A64.to(torch.float32).requires_grad_()
    print(f"det grad xxl n={n}", flush=True)
    d = fermix_amd.det(A)
    (gr,) = torch.autograd.grad(d.sum(), A)
    assert torch.all(torch.isfinite(gr)) and d[1].item() == 0
    err = _inv_residual(A[:1].detach().transpose(1, 2), gr[:1].to(torch.float64) / d[0].item())
    print(f"  regular member residual {err}", flush=True)
    assert np.all(err < 1e-5)
    g1 = gr[1]
    assert torch.all(g1[:, :k] == 0) and torch.all(g1[:, k + 1 :] == 0)
    v = v.to(torch.float32).to(torch.float64)  # the column as A held it before zeroing
    Av = A[1].detach().to(torch.float64).clone()
    Av[:, k] = v
    want = torch.linalg.det(Av).item()
    got = torch.dot(v, g1[:, k].to(torch.float64)).item()
    print(f"  zero-column member: {got:.8g} vs {want:.8g}", flush=True)
    assert abs(got - want) < 1e-4 * abs(want)
