"""GPU parity of float32 above the float32 blocked kernels (8192 < n <= 16384: the
field-generic blocked kernels of the float64 path on float storage, products in fp64),
forward and gradients, against float64 truth formed on the GPU (torch.linalg slogdet /
inv in float64). Each batch holds a well-conditioned member (I + N(0, 1/(4n)); X J X^T
for the Pfaffian, whose value is det(X)) and an N(0, 1/n) one, held to the north-star
bars or, outside them, to KAPPA_C 2^-24 kappa with kappa from power iterations on the
matrix and its float64 inverse; n = 12288 adds an exact zero column / row."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from tests.tolerances import KAPPA_C, U32, logabs_tol

pytestmark = pytest.mark.gpu


def _members(dev, n, seed, skew=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    Z = torch.randn((2, n, n), generator=g, dtype=torch.float64).to(dev)
    M = Z / np.sqrt(n)
    M[0] = torch.eye(n, dtype=torch.float64, device=dev) + 0.5 * M[0]
    if skew:
        J = torch.zeros((n, n), dtype=torch.float64, device=dev)
        idx = torch.arange(0, n, 2, device=dev)
        J[idx, idx + 1] = 1.0
        J[idx + 1, idx] = -1.0
        X = M[0].clone()
        M[0] = X @ J @ X.T
        M[1] = (M[1] - M[1].T) / np.sqrt(2.0)
        return M, X
    return M, None


def _norm2(M, iters=40):
    """Largest singular value by power iteration on M^T M (float64, GPU)."""
    v = torch.ones(M.shape[-1], dtype=M.dtype, device=M.device)
    v /= torch.linalg.norm(v)
    s = 0.0
    for _ in range(iters):
        w = M.T @ (M @ v)
        s = torch.linalg.norm(w).item()
        v = w / s
    return float(np.sqrt(s))


def _check(err, lit, kap, what):
    """err within the literal bar, else within KAPPA_C 2^-24 kappa."""
    print(f"  {what}: err {err:.3g} literal {lit:.3g} kappa {kap:.3g} "
          f"err/(2^-24 kappa) {err / (U32 * kap):.3g}", flush=True)
    assert err <= lit or err <= KAPPA_C * U32 * kap, what


def _rel_fro(x, ref):
    return (torch.linalg.norm((x.to(torch.float64) - ref).flatten()) / torch.linalg.norm(ref.flatten())).item()


@pytest.mark.parametrize("n", [12288, 16384])
def test_slogdet_generic(dev, n):
    M, _ = _members(dev, n, 9800 + n)
    A = M.to(torch.float32)
    if n == 12288:
        Az = A[:1].clone()
        Az[0, :, n // 3] = 0.0
        A = torch.cat([A, Az])
    A = A.contiguous()
    A64 = A.to(torch.float64)
    print(f"slogdet generic n={n}", flush=True)
    s, l = fermix_amd.slogdet(A)
    s64, l64 = torch.linalg.slogdet(A64)
    assert torch.equal(s.cpu().to(torch.float64), s64.cpu())
    if n == 12288:
        assert s[2].item() == 0 and np.isneginf(l[2].item())
    inv64 = [torch.linalg.inv(A64[b]) for b in range(2)]
    kap = [_norm2(A64[b]) * _norm2(inv64[b]) for b in range(2)]
    for b in range(2):
        err = abs(l[b].item() - l64[b].item())
        _check(err, float(logabs_tol(l64[b].item(), n)), kap[b], f"logabs member {b}")
    # A^-T: the parts run's primal is the forward's; the autograd route returns it
    sp, lp, invT = _kernels.slogdet_parts(A)[:3]
    assert torch.equal(sp, s) and torch.equal(lp, l), "parts primal != forward"
    if n == 12288:
        assert torch.count_nonzero(invT[2]).item() == 0
    for b in range(2):
        _check(_rel_fro(invT[b], inv64[b].T), 1e-4, kap[b], f"A^-T member {b}")
    Ag = A.clone().requires_grad_()
    _, la = fermix_amd.slogdet(Ag)
    (gr,) = torch.autograd.grad(la[:2].sum(), Ag)
    assert torch.equal(gr[:2], invT[:2])
    del gr, Ag, invT
    # det's gradient of the well-conditioned member (logabs O(1)): det(A) A^-T
    Ad = A[:1].clone().requires_grad_()
    d = fermix_amd.det(Ad)
    (gd,) = torch.autograd.grad(d.sum(), Ad)
    ref = torch.exp(l64[0]) * s64[0] * inv64[0].T
    _check(_rel_fro(gd[0], ref), 1e-4, kap[0], "adj(A)^T member 0")


@pytest.mark.parametrize("n", [12288, 16384])
def test_slogpf_generic(dev, n):
    M, X = _members(dev, n, 9900 + n, skew=True)
    S = M.to(torch.float32)
    S = (0.5 * (S - S.transpose(1, 2))).contiguous()  # exactly skew in float32
    S64 = S.to(torch.float64)
    print(f"slogpf generic n={n}", flush=True)
    s, l = fermix_amd.slogpf(S, skew_symmetrize=False)
    sx, lx = torch.linalg.slogdet(X)  # pf(X J X^T) = det(X)
    _, ld = torch.linalg.slogdet(S64)  # log |pf| = log |det| / 2
    inv64 = [torch.linalg.inv(S64[b]) for b in range(2)]
    kap = [_norm2(S64[b]) * _norm2(inv64[b]) for b in range(2)]
    assert s[0].item() == sx.item() and abs(s[1].item()) == 1.0
    _check(abs(l[0].item() - lx.item()), float(logabs_tol(lx.item(), n)), kap[0], "log|pf| member 0 vs det X")
    _check(abs(l[1].item() - 0.5 * ld[1].item()), float(logabs_tol(0.5 * ld[1].item(), n)), kap[1],
           "log|pf| member 1 vs log|det| / 2")
    sp, lp, Sinv = _kernels.slogpf_parts(S, False)
    assert torch.equal(sp, s) and torch.equal(lp, l)
    for b in range(2):
        _check(_rel_fro(Sinv[b], inv64[b]), 1e-4, kap[b], f"S^-1 member {b}")
    Sg = S.clone().requires_grad_()
    _, la = fermix_amd.slogpf(Sg, skew_symmetrize=False)
    (gr,) = torch.autograd.grad(la.sum(), Sg)
    assert torch.equal(gr, -0.5 * Sinv)
    del gr, Sg, Sinv
    # pf's gradient of the X J X^T member: pf(S) S^-1 (the LU route; pf = det X = O(1))
    _, _, G = _kernels.slogpf_parts(S[:1].contiguous(), False, adjugate=True)
    ref = torch.exp(lx) * sx * inv64[0]
    _check(_rel_fro(G[0], ref), 1e-4, kap[0], "pf(S) S^-1 member 0")
    if n == 12288:
        # a zero row / column: pf = 0, S^-1 zero, the forward's bits for the other member
        Sz = S.clone()
        Sz[0, 5, :] = 0.0
        Sz[0, :, 5] = 0.0
        zs, zl, zg = _kernels.slogpf_parts(Sz, False)
        assert zs[0].item() == 0 and np.isneginf(zl[0].item())
        assert torch.count_nonzero(zg[0]).item() == 0
        assert torch.equal(zs[1], s[1]) and torch.equal(zl[1], l[1])
