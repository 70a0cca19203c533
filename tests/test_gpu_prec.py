"""GPU parity of both product modes of the blocked kernels: the split-bf16x3 mode
(prec="bf16x3", and "tf32x3", the reference's name for its fp32-accuracy three-pass mode,
src/fermix/_field.py:20-23, 173-190, which selects it on gfx950) and the IEEE fp32 MFMA
mode (prec="ieee"), each held to the same bars -- sign exact, logabs within the
north-star tolerance, gradients within 1e-4 relative Frobenius error of float64 truth (or
the conditioning bound). The C3 / C4 sizes run in both modes in tests/test_gpu_grad.py
(no less accurate on average than a float32 LAPACK inverse of the same members)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs, rel_fro

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


@pytest.mark.parametrize("prec", ["bf16x3", "ieee"])
@pytest.mark.parametrize("n", [129, 200, 256, 512, 1024])
def test_slogdet_forward_and_grad_by_mode(dev, n, prec):
    """Both product modes of the blocked LU (n > 128): sign exact and logabs against
    float64, A^-T against float64, the primal of the parts and autograd routes
    bit-identical to the forward of the same mode."""
    B = 8 if n <= 512 else 3
    x3 = 1 if prec == "bf16x3" else 0
    rng = np.random.default_rng(6100 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    A[1, :, n // 2] = 0.0  # exactly singular member
    print(f"{prec} slogdet n={n} B={B}", flush=True)
    At = _t(A, dev)
    s, l = map(_np, fermix_amd.slogdet(At, prec=prec))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, f"{prec} n={n} vs float64", A)
    # the parts route: primal bit-identical to the forward, A^-T against float64
    sp, lp, invT, _, _ = _kernels.slogdet_parts(At, x3=x3)
    assert np.array_equal(_np(sp), s) and np.array_equal(_np(lp), l)
    keep = np.arange(B) != 1
    assert np.all(_np(invT)[1] == 0)
    ref = np.linalg.inv(A[keep].astype(np.float64)).transpose(0, 2, 1)
    assert_grad(_np(invT)[keep], ref, A[keep], f"{prec} A^-T n={n} vs float64")
    # the autograd route (factors in the forward, the scaled inverse in the backward)
    Ag = At.clone().requires_grad_()
    _, la = fermix_amd.slogdet(Ag, prec=prec)
    assert np.array_equal(_np(la), l)
    (g,) = torch.autograd.grad(la[keep].sum(), Ag)
    assert torch.equal(g[keep], invT[keep])
    if prec == "bf16x3":
        # "tf32x3" selects the same mode
        s3, l3 = fermix_amd.slogdet(At, prec="tf32x3")
        assert torch.equal(s3, torch.from_numpy(s).to(dev)) and torch.equal(l3, torch.from_numpy(l).to(dev))
    else:
        # the modes differ in the trailing products only: same signs, logabs within the bar
        s1, l1 = map(_np, fermix_amd.slogdet(At, prec="bf16x3"))
        assert np.array_equal(s1, s)
        assert_logabs(l1, l, n, f"bf16x3 vs ieee n={n}", A)


@pytest.mark.parametrize("prec", ["bf16x3", "ieee"])
@pytest.mark.parametrize("n", [130, 256, 512, 1024])
def test_slogpf_grad_by_mode(dev, n, prec):
    B = 6 if n <= 512 else 3
    x3 = 1 if prec == "bf16x3" else 0
    rng = np.random.default_rng(6200 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    print(f"{prec} slogpf grad n={n} B={B}", flush=True)
    St = _t(S, dev)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    s, l, Sinv = _kernels.slogpf_parts(St, False, x3=x3)
    assert torch.equal(s, s0) and torch.equal(l, l0)  # the forward is the same in both modes
    _, ld64 = ref64.slogdet64(S)
    assert_logabs(_np(l), 0.5 * ld64, n, f"{prec} n={n} log|pf| vs log|det| / 2 float64", S)
    ref = np.linalg.inv(S.astype(np.float64))
    G = _np(Sinv)
    assert np.max(np.abs(G + G.transpose(0, 2, 1))) <= 1e-6 * np.abs(G).max()
    assert_grad(G, ref, S, f"{prec} S^-1 n={n} vs float64")
    Sg = St.clone().requires_grad_()
    _, la = fermix_amd.slogpf(Sg, skew_symmetrize=False, prec=prec)
    (g,) = torch.autograd.grad(la.sum(), Sg)
    assert torch.equal(g, -0.5 * Sinv)


@pytest.mark.parametrize("prec", ["bf16x3", "ieee"])
def test_det_pf_adjugates_by_mode(dev, prec):
    """The det / pf gradients (adjugates, exact for singular inputs) in each product mode
    against float64 cofactor-free references on regular members, finite on a member with
    one zero pivot."""
    n = 200
    rng = np.random.default_rng(6300)
    A = (rng.standard_normal((4, n, n)) / np.sqrt(n) + np.eye(n) * 0.5).astype(np.float32)
    A[2, :, 7] = 0.0
    At = _t(A, dev).requires_grad_()
    d = fermix_amd.det(At, prec=prec)
    (gd,) = torch.autograd.grad(d.sum(), At)
    A64 = A.astype(np.float64)
    for b in (0, 1, 3):
        ref = np.linalg.det(A64[b]) * np.linalg.inv(A64[b]).T
        assert rel_fro(_np(gd)[b:b + 1], ref[None])[0] < 1e-4, b
    # one zero column: the adjugate stays finite (its exact values are checked in the
    # default mode by tests/test_gpu_adjugate.py; the rank-1 branch's GEMMs are the same)
    assert np.all(np.isfinite(_np(gd)[2]))
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    St = _t(S, dev).requires_grad_()
    p = fermix_amd.pf(St, skew_symmetrize=False, prec=prec)
    (gp,) = torch.autograd.grad(p.sum(), St)
    S64 = S.astype(np.float64)
    for b in (0, 1, 3):
        _, lpf = ref64.slogpf64(S[b:b + 1])
        sgn = np.sign(_np(p)[b])
        pfv = sgn * np.exp(lpf[0])
        ref = -0.5 * pfv * np.linalg.inv(S64[b])
        assert rel_fro(_np(gp)[b:b + 1], ref[None])[0] < 1e-4, b
