"""GPU parity of the split-bf16x3 product mode (prec="bf16x3", and "tf32x3", the
reference's name for its fp32-accuracy three-pass mode, src/fermix/_field.py:20-23,
173-190, which selects it on gfx950): the same bars as the fp32 MFMA mode -- sign exact,
logabs within the north-star tolerance, gradients within 1e-4 relative Frobenius error
of float64 truth (or the conditioning bound), and at the C3 / C4 sizes no less accurate
on average than a float32 LAPACK inverse of the same members."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import ref64
from tests.tolerances import (assert_grad, assert_grad_vs_fp32, assert_logabs, lapack_inverse_f32,
                              rel_fro)

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


@pytest.mark.parametrize("n", [129, 200, 256, 512, 1024])
def test_bf16x3_slogdet_forward_and_grad(dev, n):
    B = 8 if n <= 512 else 3
    rng = np.random.default_rng(6100 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    A[1, :, n // 2] = 0.0  # exactly singular member
    print(f"bf16x3 slogdet n={n} B={B}", flush=True)
    At = _t(A, dev)
    s, l = map(_np, fermix_amd.slogdet(At, prec="bf16x3"))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, f"bf16x3 n={n} vs float64", A)
    # the parts route: primal bit-identical to the bf16x3 forward, A^-T against float64
    sp, lp, invT, _, _ = _kernels.slogdet_parts(At, x3=1)
    assert np.array_equal(_np(sp), s) and np.array_equal(_np(lp), l)
    keep = np.arange(B) != 1
    assert np.all(_np(invT)[1] == 0)
    ref = np.linalg.inv(A[keep].astype(np.float64)).transpose(0, 2, 1)
    assert_grad(_np(invT)[keep], ref, A[keep], f"bf16x3 A^-T n={n} vs float64")
    # the autograd route (factors in the forward, the scaled inverse in the backward)
    Ag = At.clone().requires_grad_()
    _, la = fermix_amd.slogdet(Ag, prec="bf16x3")
    assert np.array_equal(_np(la), l)
    (g,) = torch.autograd.grad(la[keep].sum(), Ag)
    assert torch.equal(g[keep], invT[keep])
    # "tf32x3" selects the same mode
    s3, l3 = fermix_amd.slogdet(At, prec="tf32x3")
    assert torch.equal(s3, torch.from_numpy(s).to(dev)) and torch.equal(l3, torch.from_numpy(l).to(dev))


@pytest.mark.parametrize("n", [130, 256, 512, 1024])
def test_bf16x3_slogpf_grad(dev, n):
    B = 6 if n <= 512 else 3
    rng = np.random.default_rng(6200 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    print(f"bf16x3 slogpf grad n={n} B={B}", flush=True)
    St = _t(S, dev)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    s, l, Sinv = _kernels.slogpf_parts(St, False, x3=1)
    assert torch.equal(s, s0) and torch.equal(l, l0)  # the forward is the same in both modes
    ref = np.linalg.inv(S.astype(np.float64))
    G = _np(Sinv)
    assert np.max(np.abs(G + G.transpose(0, 2, 1))) <= 1e-6 * np.abs(G).max()
    assert_grad(G, ref, S, f"bf16x3 S^-1 n={n} vs float64")
    Sg = St.clone().requires_grad_()
    _, la = fermix_amd.slogpf(Sg, skew_symmetrize=False, prec="bf16x3")
    (g,) = torch.autograd.grad(la.sum(), Sg)
    assert torch.equal(g, -0.5 * Sinv)


def test_bf16x3_det_pf_adjugates(dev):
    """The det / pf gradients (adjugates, exact for singular inputs) in the bf16x3 mode
    against float64 cofactor-free references on regular members and the rank-1 form on a
    member with one zero pivot."""
    n = 200
    rng = np.random.default_rng(6300)
    A = (rng.standard_normal((4, n, n)) / np.sqrt(n) + np.eye(n) * 0.5).astype(np.float32)
    A[2, :, 7] = 0.0
    At = _t(A, dev).requires_grad_()
    d = fermix_amd.det(At, prec="bf16x3")
    (gd,) = torch.autograd.grad(d.sum(), At)
    A64 = A.astype(np.float64)
    for b in (0, 1, 3):
        ref = np.linalg.det(A64[b]) * np.linalg.inv(A64[b]).T
        assert rel_fro(_np(gd)[b:b + 1], ref[None])[0] < 1e-4, b
    # one zero column: the adjugate stays finite (its exact values are checked in fp32
    # mode by tests/test_gpu_adjugate.py; the rank-1 branch's GEMMs are the same)
    assert np.all(np.isfinite(_np(gd)[2]))
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    St = _t(S, dev).requires_grad_()
    p = fermix_amd.pf(St, skew_symmetrize=False, prec="bf16x3")
    (gp,) = torch.autograd.grad(p.sum(), St)
    S64 = S.astype(np.float64)
    for b in (0, 1, 3):
        _, lpf = ref64.slogpf64(S[b:b + 1])
        sgn = np.sign(_np(p)[b])
        pfv = sgn * np.exp(lpf[0])
        ref = -0.5 * pfv * np.linalg.inv(S64[b])
        assert rel_fro(_np(gp)[b:b + 1], ref[None])[0] < 1e-4, b


def test_bf16x3_c3_properties(dev):
    """C3 size (B = 1024, n = 512, N(0, 1/n)) in the bf16x3 mode: the gradient on 18
    members against float64, and on average no less accurate than float32 LAPACK."""
    rng = np.random.default_rng(3)
    B, n = 1024, 512
    A = rng.standard_normal((B, n, n), dtype=np.float32) * np.float32(1 / np.sqrt(n))
    At = _t(A, dev)
    s, l, invT, _, _ = _kernels.slogdet_parts(At, x3=1)
    s0, l0 = fermix_amd.slogdet(At, prec="bf16x3")
    assert torch.equal(s, s0) and torch.equal(l, l0)
    assert bool(torch.isfinite(invT).all())
    idx = list(range(0, 1024, 64)) + [1, 1023]
    G = _np(invT[idx])
    ref = np.linalg.inv(A[idx].astype(np.float64)).transpose(0, 2, 1)
    assert_grad(G, ref, A[idx], "bf16x3 C3 subset vs float64")
    inv32 = lapack_inverse_f32(A[idx]).transpose(0, 2, 1)
    assert_grad_vs_fp32(G, ref, rel_fro(inv32, ref), "bf16x3 C3 subset vs fp32 LAPACK's error")
    s64, l64 = ref64.slogdet64(A[idx])
    assert np.array_equal(_np(s)[idx], s64)
    assert_logabs(_np(l)[idx], l64, n, "bf16x3 C3 subset logabs vs float64", A[idx])


def test_bf16x3_c4_properties(dev):
    """C4 size (B = 64, n = 2048, S = A - A^T) in the bf16x3 mode."""
    rng = np.random.default_rng(4)
    B, n = 64, 2048
    A = rng.standard_normal((B, n, n), dtype=np.float32) * np.float32(1 / np.sqrt(n))
    S = A - A.transpose(0, 2, 1)
    del A
    St = _t(S, dev)
    s, l, Sinv = _kernels.slogpf_parts(St, False, x3=1)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert torch.equal(s, s0) and torch.equal(l, l0)
    assert bool(torch.isfinite(Sinv).all())
    idx = [0, 1, 2, 31, 62, 63]
    G = _np(Sinv[idx])
    assert np.max(np.abs(G + G.transpose(0, 2, 1))) <= 1e-6 * np.abs(G).max()
    ref = np.linalg.inv(S[idx].astype(np.float64))
    assert_grad(G, ref, S[idx], "bf16x3 C4 subset vs float64")
    inv32 = lapack_inverse_f32(S[idx])
    assert_grad_vs_fp32(G, ref, rel_fro(inv32, ref), "bf16x3 C4 subset vs fp32 LAPACK's error")
