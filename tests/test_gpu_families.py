"""Cross-checks between the kernel families (several matrices per wave, one fused
workgroup per matrix, blocked with workspace), forced with the family override at the
same n -- the counterpart of the reference's table-override test (tests/test_fermix.py:
720-762): every family agrees with float64 and with the others, its differentiated
primal is bit-identical to its own forward, and det's gradient is the exact adjugate on
singular members whichever family factors them."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels, _tune
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def _families(n, op):
    out = []
    for f in ("tiny", "fused", "blocked"):
        with _tune.force_family(f):
            if _tune.kernel_family(n, op) != "unsupported":
                out.append(f)
    return out


@pytest.mark.parametrize("n", [5, 16, 24, 32, 48, 100, 128, 200])
def test_slogdet_families_agree(dev, n):
    rng = np.random.default_rng(7000 + n)
    B = 12
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n) + 0.5 * np.eye(n)).astype(np.float32)
    A[0, :, n // 2] = 0.0
    s64, l64 = ref64.slogdet64(A)
    inv64 = np.linalg.inv(A[1:].astype(np.float64)).swapaxes(-1, -2)
    fams = _families(n, "slogdet")
    assert "blocked" in fams and (len(fams) >= 2 or n > 128)
    res = {}
    for f in fams:
        with _tune.force_family(f):
            print(f"slogdet n={n} family={f}", flush=True)
            s, l = fermix_amd.slogdet(_t(A, dev))
            sp, lp, invT, _, _ = _kernels.slogdet_parts(_t(A, dev))
            assert torch.equal(s, sp) and torch.equal(l, lp), f"{f}: parts primal != forward"
            s, l, invT = _np(s), _np(l), _np(invT)
            assert np.array_equal(s, s64)
            assert_logabs(l, l64, n, f"{f} vs float64", A)
            assert np.all(invT[0] == 0)
            assert_grad(invT[1:], inv64, A[1:], f"{f} invT vs float64")
            res[f] = l
    for f in fams[1:]:
        assert_logabs(res[f], res[fams[0]], n, f"{f} vs {fams[0]}", A)


@pytest.mark.parametrize("n", [6, 16, 24, 64, 128, 160])
def test_slogpf_families_agree(dev, n):
    rng = np.random.default_rng(7100 + n)
    B = 8
    S = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (S - S.transpose(0, 2, 1)).astype(np.float32)
    S[0, 1, :] = 0.0
    S[0, :, 1] = 0.0
    s64, l64 = ref64.slogpf64(S)
    inv64 = np.linalg.inv(S[1:].astype(np.float64))
    fams = _families(n, "slogpf")
    assert "blocked" in fams and (len(fams) >= 2 or n > 128)
    for f in fams:
        with _tune.force_family(f):
            print(f"slogpf n={n} family={f}", flush=True)
            s, l = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False)
            sp, lp, Sinv = _kernels.slogpf_parts(_t(S, dev), False)
            assert torch.equal(s, sp) and torch.equal(l, lp), f"{f}: parts primal != forward"
            s, l, Sinv = _np(s), _np(l), _np(Sinv)
            assert np.array_equal(s, s64)
            assert_logabs(l, l64, n, f"{f} vs float64", S)
            assert np.all(Sinv[0] == 0)
            assert_grad(Sinv[1:], inv64, S[1:], f"{f} S^-1 vs float64")


@pytest.mark.parametrize("family", ["tiny", "fused", "blocked"])
def test_det_adjugate_any_family(dev, family):
    """n = 12 (tiny) / 40 (fused) / 40 forced blocked: zero column (rank n-1) and two zero
    columns (rank n-2) -- the exact adjugate against the float64 SVD adjugate."""
    n = 12 if family == "tiny" else 40
    rng = np.random.default_rng(7200 + n)
    A = (np.eye(n) + 0.5 * rng.standard_normal((4, n, n)) / np.sqrt(n)).astype(np.float32)
    A[0, :, 3] = 0.0
    A[1, :, 0] = 0.0
    A[1, :, 1] = 0.0
    with _tune.force_family(family):
        At = _t(A, dev).requires_grad_()
        d = fermix_amd.det(At)
        (g,) = torch.autograd.grad(d.sum(), At)
    g = _np(g)
    ref = np.stack([ref64.adjT_svd(a) for a in A])
    assert np.all(np.isfinite(g)) and np.all(g[1] == 0)
    assert np.max(np.abs(g - ref)) < 1e-4 * np.abs(ref).max()
    for k in (0, 2, 3):
        assert np.max(np.abs(g[k] - ref[k])) < 1e-4 * np.abs(ref[k]).max()


def test_unsupported_family_raises(dev):
    A = torch.zeros((2, 40, 40), device=dev)
    with _tune.force_family("tiny"):
        with pytest.raises(fermix_amd._lib.FermixLibraryError):
            fermix_amd.slogdet(A)
