"""GPU parity of the float64 / complex64 / complex128 blocked kernels (lu64_impl.inc) at their
largest order, n = 8192 (B = 1, 256 panels of 32 columns, the tall ones on several
workgroups per matrix, lu64_panel_mwg_kernel): slogdet
against torch.linalg.slogdet in float64 / complex128 on the GPU; A^-T, S^-1 and the
Pfaffian adjugate pf(S) S^-1 through their float64 / complex128 residuals (M X - I, a
bound on the relative error of X as M^-1); pf(X J X^T) = det(X), which ties the
Parlett-Reid run to the LU of a different matrix. X = I + N(0, 1/(4n)) (both parts for
the complex kinds) is well conditioned, so the bars are those of the precision class:
float64 / complex128 logabs within 1e-12 n, residuals below 1e-11; complex64 the float32
bars (logabs 1e-5 max(1, |l|) + 1e-6 n, residuals below 1e-4)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels

pytestmark = pytest.mark.gpu

KINDS = {
    "f64": (torch.float64, torch.float64),
    "c64": (torch.complex64, torch.complex128),
    "c128": (torch.complex128, torch.complex128),
}


def _bars(kind, n, lref):
    if kind == "c64":
        return 1e-5 * max(1.0, abs(lref)) + 1e-6 * n, 1e-4
    return 1e-12 * n, 1e-11


def _residual(M, X, wide):
    """||M X - I||_F / sqrt(n) in the wide type on the GPU."""
    n = M.shape[-1]
    R = torch.matmul(M.to(wide), X.to(wide))
    R.diagonal(dim1=-2, dim2=-1).sub_(1.0)
    return (torch.linalg.norm(R.flatten(1), dim=1) / np.sqrt(n)).cpu().numpy()


@pytest.mark.parametrize("kind", list(KINDS))
def test_blocked_64bit_and_complex_n8192(dev, kind):
    n = 8192
    dt, wide = KINDS[kind]
    g = torch.Generator(device="cpu").manual_seed(9990)
    Z = torch.randn((1, n, n), generator=g, dtype=torch.float64)
    if wide.is_complex:
        Z = torch.complex(Z, torch.randn((1, n, n), generator=g, dtype=torch.float64))
    X = (torch.eye(n, dtype=wide) + 0.5 * Z.to(wide) / np.sqrt(n)).to(dev)
    del Z
    A = X.to(dt)
    print(f"blocked {kind} n={n}: slogdet", flush=True)
    s, l = fermix_amd.slogdet(A)
    sr, lr = torch.linalg.slogdet(A.to(wide))
    lbar, rbar = _bars(kind, n, lr.item())
    print(f"  sign {s.item()} vs {sr.item()}, logabs {l.item()} vs {lr.item()}", flush=True)
    assert abs(s.item() - sr.item()) < lbar
    assert abs(l.item() - lr.item()) < lbar
    print("  A^-T", flush=True)
    sp, lp, invT = _kernels.slogdet_parts(A)[:3]
    assert torch.equal(sp, s) and torch.equal(lp, l), "parts primal != forward"
    err = _residual(A.transpose(1, 2), invT, wide)
    print(f"  A^-T residual {err}", flush=True)
    assert np.all(err < rbar)
    del invT, sp, lp
    # pf(X J X^T) = det(X)
    J = torch.zeros((n, n), dtype=wide, device=dev)
    idx = torch.arange(0, n, 2, device=dev)
    J[idx, idx + 1] = 1.0
    J[idx + 1, idx] = -1.0
    S = X @ J @ X.transpose(1, 2)
    del J
    S = (0.5 * (S - S.transpose(1, 2))).to(dt).contiguous()
    sx, lx = torch.linalg.slogdet(X)
    print("  slogpf", flush=True)
    ps, pl = fermix_amd.slogpf(S, skew_symmetrize=False)
    print(f"  pf sign {ps.item()} vs {sx.item()}, logabs {pl.item()} vs {lx.item()}", flush=True)
    assert abs(ps.item() - sx.item()) < lbar
    assert abs(pl.item() - lx.item()) < lbar
    print("  S^-1", flush=True)
    qs, ql, Sinv = _kernels.slogpf_parts(S, False)
    assert torch.equal(qs, ps) and torch.equal(ql, pl)
    err = _residual(S, Sinv, wide)
    print(f"  S^-1 residual {err}", flush=True)
    assert np.all(err < rbar)
    del Sinv
    print("  pf(S) S^-1", flush=True)
    _, _, G = _kernels.slogpf_parts(S, False, adjugate=True)
    pfv = ps.to(wide) * torch.exp(pl.to(wide))
    err = _residual(S, G / pfv[:, None, None].to(G.dtype), wide)
    print(f"  adjugate residual {err}", flush=True)
    assert np.all(err < rbar)
