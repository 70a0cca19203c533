"""GPU parity of the float64 entry points (fx_*_f64): slogdet / slogpf / det / pf values
against float64 truth (numpy's LAPACK slogdet, the float64 Parlett-Reid of the oracle,
the perfect-matching Pfaffian for n <= 8, closed forms), the gradients A^-T and S^-1 /
2 against numpy's float64 inverse, bit-identity of the differentiated primal, the
singular / odd-n conventions (0, -inf) with zero gradients, and autograd integration.
The reference runs the same API in float64 (src/fermix/api.py:24-31; its tests
tests/test_fermix.py:153-155, 192, 370, 442-456 use these float64 references)."""

import itertools

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import ref64
from tests.tolerances import assert_grad64, assert_logabs64

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def _skew(A):
    return (A - np.swapaxes(A, -1, -2)) * 0.5


# n spans the register-resident kernels (n <= 128: 16-column strips up to n = 64, 32-column
# strips from n = 65, no workspace) and, above, the blocked LU for the values (32-column
# panels, padded orders 160 .. 1024) with the Gauss-Jordan workspace kernel for A^-T
@pytest.mark.parametrize("n", [0, 1, 2, 3, 5, 16, 31, 61, 62, 64, 65, 87, 88, 128, 129, 200, 300, 520, 1024])
def test_f64_slogdet_and_inverse(dev, n):
    B = 8 if n <= 128 else (3 if n <= 300 else 2)
    rng = np.random.default_rng(7000 + n)
    A = rng.standard_normal((B, n, n)) / np.sqrt(max(n, 1))
    print(f"f64 slogdet n={n} B={B}", flush=True)
    s, l = fermix_amd.slogdet(_t(A, dev))
    assert s.dtype == torch.float64 and l.dtype == torch.float64
    s2, l2, invT, _, _ = _kernels.slogdet_parts(_t(A, dev))
    assert torch.equal(s, s2) and torch.equal(l, l2), "parts primal != forward"
    sr, lr = ref64.slogdet64(A)
    assert np.array_equal(_np(s), sr)
    assert_logabs64(_np(l), lr, n, "slogdet64", A)
    if n:
        assert_grad64(_np(invT), np.swapaxes(ref64.inv64(A), 1, 2), A, f"A^-T n={n}")


# above n = 128 the blocked Parlett-Reid (16 pair steps per panel, padded orders 160 .. 544)
@pytest.mark.parametrize("n", [0, 2, 4, 6, 8, 16, 30, 62, 64, 86, 88, 128, 130, 200, 256, 520])
def test_f64_slogpf_and_inverse(dev, n):
    B = 8 if n <= 128 else 3
    rng = np.random.default_rng(7100 + n)
    A = rng.standard_normal((B, n, n)) / np.sqrt(max(n, 1))
    S = _skew(A)
    print(f"f64 slogpf n={n} B={B}", flush=True)
    s, l = fermix_amd.slogpf(_t(A, dev))
    s2, l2, g = _kernels.slogpf_parts(_t(A, dev), True)
    assert torch.equal(s, s2) and torch.equal(l, l2), "parts primal != forward"
    # skew_symmetrize=False on the exactly skew S gives the same bits
    s3, l3 = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False)
    assert torch.equal(s, s3) and torch.equal(l, l3)
    sr, lr = ref64.slogpf64(S)
    assert np.array_equal(_np(s), sr)
    assert_logabs64(_np(l), lr, n, "slogpf64", S)
    if n <= 8:
        p = np.array([ref64.pf_brute(x) for x in S])
        assert np.allclose(_np(s) * np.exp(_np(l)), p, rtol=1e-12, atol=0)
    if n:
        assert_grad64(_np(g), ref64.inv64(S), S, f"S^-1 n={n}")
        # log|pf|^2 = log|det|
        _, ld = fermix_amd.slogdet(_t(S, dev))
        assert np.allclose(2 * _np(l), _np(ld), rtol=1e-11, atol=1e-11 * n)


def test_f64_closed_forms(dev):
    # permutation matrices: det = parity; triangular: det = product of the diagonal
    n = 6
    perms = list(itertools.permutations(range(n)))[::37]
    P = np.zeros((len(perms), n, n))
    par = np.empty(len(perms))
    for b, p in enumerate(perms):
        P[b, np.arange(n), p] = 1.0
        inv = sum(1 for i in range(n) for j in range(i + 1, n) if p[i] > p[j])
        par[b] = -1.0 if inv & 1 else 1.0
    s, l = fermix_amd.slogdet(_t(P, dev))
    assert np.array_equal(_np(s), par) and np.all(_np(l) == 0.0)
    rng = np.random.default_rng(7200)
    # column-dominant lower triangle (|d_j| >= 0.5 > every entry below it): partial
    # pivoting keeps the diagonal, the pivot rows are zero right of it, so u_jj = d_j
    # exactly (a random triangle would be exponentially ill-conditioned instead)
    d = rng.uniform(0.5, 2.0, (5, 40)) * rng.choice([-1.0, 1.0], (5, 40))
    T = np.clip(np.tril(0.1 * rng.standard_normal((5, 40, 40)), -1), -0.45, 0.45)
    T[:, np.arange(40), np.arange(40)] = d
    s, l = fermix_amd.slogdet(_t(T, dev))
    assert np.array_equal(_np(s), np.prod(np.sign(d), axis=1))
    assert np.allclose(_np(l), np.log(np.abs(d)).sum(axis=1), rtol=1e-14, atol=1e-13)
    # pf of a direct sum of a_i J blocks is prod a_i
    a = rng.standard_normal((4, 10))
    S = np.zeros((4, 20, 20))
    for i in range(10):
        S[:, 2 * i, 2 * i + 1] = a[:, i]
        S[:, 2 * i + 1, 2 * i] = -a[:, i]
    s, l = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False)
    assert np.array_equal(_np(s), np.prod(np.sign(a), axis=1))
    assert np.allclose(_np(l), np.log(np.abs(a)).sum(axis=1), rtol=1e-14, atol=1e-13)


@pytest.mark.parametrize("n", [12, 70, 150, 300])
def test_f64_singular_and_odd(dev, n):
    rng = np.random.default_rng(7300 + n)
    A = rng.standard_normal((4, n, n))
    A[0, :, 3] = 0.0
    A[2, 5, :] = 0.0
    At = _t(A, dev).requires_grad_()
    s, l = fermix_amd.slogdet(At)
    assert np.isneginf(_np(l)[0]) and np.isneginf(_np(l)[2]) and _np(s)[0] == 0
    (gr,) = torch.autograd.grad(l.sum(), At)
    gr = _np(gr)
    assert np.all(np.isfinite(gr)) and np.all(gr[0] == 0) and np.all(gr[2] == 0)
    assert_grad64(gr[[1, 3]], np.swapaxes(ref64.inv64(A[[1, 3]]), 1, 2), A[[1, 3]], "singular batch")
    # slogpf: a zero row / column of S gives an exact zero pivot
    S = _skew(A)
    S[1, 4, :] = 0.0
    S[1, :, 4] = 0.0
    St = _t(S, dev).requires_grad_()
    s, l = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert _np(s)[1] == 0 and np.isneginf(_np(l)[1])
    (gr,) = torch.autograd.grad(l.sum(), St)
    assert np.all(_np(gr)[1] == 0) and np.all(np.isfinite(_np(gr)))
    # odd n
    m = n | 1
    O = _t(rng.standard_normal((3, m, m)), dev)
    s, l = fermix_amd.slogpf(O)
    assert np.all(_np(s) == 0) and np.all(np.isneginf(_np(l)))
    s, l, g = _kernels.slogpf_parts(O, True)  # the kernel's own odd-n branch
    assert np.all(_np(s) == 0) and np.all(np.isneginf(_np(l))) and np.all(_np(g) == 0)


@pytest.mark.parametrize("n", [24, 100, 160])
def test_f64_autograd(dev, n):
    rng = np.random.default_rng(7400 + n)
    A = rng.standard_normal((3, n, n)) / np.sqrt(n)
    At = _t(A, dev).requires_grad_()
    s, l = fermix_amd.slogdet(At)
    s0, l0 = fermix_amd.slogdet(_t(A, dev))
    assert torch.equal(l.detach(), l0)
    (gr,) = torch.autograd.grad(l.sum(), At)
    assert_grad64(_np(gr), np.swapaxes(ref64.inv64(A), 1, 2), A, "slogdet autograd")
    (gp,) = torch.autograd.grad(fermix_amd.slogpf(At)[1].sum(), At)
    S = _skew(A)
    assert_grad64(_np(gp), 0.5 * np.swapaxes(ref64.inv64(S), 1, 2), S, "slogpf autograd")
    # forward mode and vmap
    dA = _t(rng.standard_normal(A.shape), dev)
    _, (_, dl) = torch.func.jvp(fermix_amd.slogdet, (_t(A, dev),), (dA,))
    ref = (np.swapaxes(ref64.inv64(A), 1, 2) * _np(dA)).sum(axis=(1, 2))
    assert np.allclose(_np(dl), ref, rtol=1e-9, atol=1e-9)
    sv, lv = torch.func.vmap(fermix_amd.slogdet)(_t(A, dev)[:, None])
    assert torch.equal(lv[:, 0], l0)
    # det / pf values in float64; det's gradient is the exact adjugate of the same run,
    # pf's the Pfaffian adjugate (tests/test_gpu_adjugate64.py and
    # tests/test_gpu_pf_adjugate64.py cover the singular cases)
    d = fermix_amd.det(_t(A, dev))
    assert np.allclose(_np(d), np.linalg.det(A), rtol=1e-10, atol=0)
    p = fermix_amd.pf(_t(A, dev))
    sr, lr = ref64.slogpf64(S)
    assert np.allclose(_np(p), sr * np.exp(lr), rtol=1e-10, atol=0)
    Ad = _t(A, dev).requires_grad_()
    dd = fermix_amd.det(Ad)
    assert torch.equal(dd.detach(), d)
    (gd,) = torch.autograd.grad(dd.sum(), Ad)
    assert_grad64(_np(gd), np.linalg.det(A)[:, None, None] * np.swapaxes(ref64.inv64(A), 1, 2), A,
                  "det autograd")
    Ap = _t(A, dev).requires_grad_()
    pp = fermix_amd.pf(Ap)
    assert torch.equal(pp.detach(), p)
    (gp,) = torch.autograd.grad(pp.sum(), Ap)
    pf_ref = sr * np.exp(lr)
    assert_grad64(_np(gp), 0.5 * pf_ref[:, None, None] * np.swapaxes(ref64.inv64(S), 1, 2), S, "pf autograd")


def _jmat(n):
    J = np.zeros((n, n))
    for i in range(0, n - 1, 2):
        J[i, i + 1], J[i + 1, i] = 1.0, -1.0
    return J


@pytest.mark.parametrize("n", [1030, 2048, 4096])
def test_f64_slogpf_blocked_large(dev, n):
    """The blocked Parlett-Reid at large n: pf(X J X^T) = det(X) (X = I + N(0, 1/(4n)), well
    conditioned) against float64 slogdet(X) on the GPU; a member with a zero row / column
    (pf = 0), odd n (pf = 0), and the same matrices with their order reversed (a symmetric
    permutation P S P^T, other pivots: pf changes by det P). n = 4096 runs unpadded."""
    B = 2 if n < 4096 else 1
    g = torch.Generator(device="cpu").manual_seed(9900 + n)
    X = torch.eye(n, dtype=torch.float64) + 0.5 * torch.randn((B, n, n), generator=g, dtype=torch.float64) / np.sqrt(n)
    X = X.to(dev)
    S = X @ torch.from_numpy(_jmat(n)).to(dev) @ X.transpose(1, 2)
    S = (0.5 * (S - S.transpose(1, 2))).contiguous()
    sgn, lab = torch.linalg.slogdet(X)
    print(f"f64 slogpf blocked n={n} B={B}", flush=True)
    s, l = fermix_amd.slogpf(S, skew_symmetrize=False)
    assert torch.equal(s.cpu(), sgn.cpu())
    err = np.abs(_np(l) - _np(lab))
    print(f"  logabs err {err}", flush=True)
    assert np.all(err < 1e-12 * n)
    # a symmetric permutation reverses the order: pf(P S P^T) = det(P) pf(S)
    perm = torch.arange(n - 1, -1, -1, device=dev)
    Sp = S[:, perm][:, :, perm].contiguous()
    sp, lp = fermix_amd.slogpf(Sp, skew_symmetrize=False)
    dP = (-1.0) ** ((n * (n - 1) // 2) % 2)
    assert torch.equal(sp.cpu(), dP * sgn.cpu())
    assert np.all(np.abs(_np(lp) - _np(lab)) < 1e-12 * n)
    if n < 4096:
        Sz = S.clone()
        Sz[0, n // 3, :] = 0.0
        Sz[0, :, n // 3] = 0.0
        sz, lz = fermix_amd.slogpf(Sz, skew_symmetrize=False)
        assert _np(sz)[0] == 0 and np.isneginf(_np(lz)[0])
        assert torch.equal(sz[1:], s[1:]) and torch.equal(lz[1:], l[1:])
        o = torch.randn((2, n - 1, n - 1), generator=g, dtype=torch.float64).to(dev)
        so, lo = fermix_amd.slogpf(o)
        assert np.all(_np(so) == 0) and np.all(np.isneginf(_np(lo)))


def test_f64_slogdet_blocked_large(dev):
    """n = 2050 (padded order 2080): the LU panels with their rows in memory (m > 1024) and
    then in registers, slogdet against torch's float64 slogdet on the GPU, A^-T through its
    float64 residual A^T A^-T - I, and the det adjugate det(A) A^-T of the same run."""
    n = 2050
    g = torch.Generator(device="cpu").manual_seed(9950)
    A = (torch.eye(n, dtype=torch.float64) + 0.5 * torch.randn((1, n, n), generator=g, dtype=torch.float64)
         / np.sqrt(n)).to(dev)
    print(f"f64 slogdet blocked n={n}", flush=True)
    s, l = fermix_amd.slogdet(A)
    sr, lr = torch.linalg.slogdet(A)
    assert torch.equal(s.cpu(), sr.cpu())
    assert abs(l.item() - lr.item()) < 1e-12 * n
    s2, l2, invT, _, _ = _kernels.slogdet_parts(A)
    assert torch.equal(s2, s) and torch.equal(l2, l)
    R = A[0].transpose(0, 1) @ invT[0] - torch.eye(n, dtype=torch.float64, device=dev)
    err = (torch.linalg.norm(R) / np.sqrt(n)).item()
    print(f"  A^-T residual {err:.3g}", flush=True)
    assert err < 1e-12
    Ad = A.clone().requires_grad_()
    d = fermix_amd.det(Ad)
    (gd,) = torch.autograd.grad(d.sum(), Ad)
    assert np.allclose(_np(gd), _np(d)[:, None, None] * _np(invT), rtol=1e-10, atol=0)
