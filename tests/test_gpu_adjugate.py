"""GPU parity of the det / pf gradients, which differentiate through the adjugates:
d det / dA = adj(A)^T and d pf / dS = -pf(S) S^-1 / 2 continued to singular S, against
float64 truth (cofactor / SVD adjugates, minor Pfaffians) and the CPU oracle, on
regular, exactly singular (one and two zero pivots, rank n-1 and n-2) and numerically
singular inputs (reference tests/test_fermix.py:428-559)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_grad, relerr

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def _near_identity(rng, B, n):
    """I + N(0, 1/(4n)): eigenvalues in the disc |z - 1| <= 1/2, so det = O(1) at any n."""
    return (np.eye(n) + 0.5 * rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)


def _skew(A):
    return (A - np.swapaxes(A, -1, -2)).astype(np.float32)


def _near_j(rng, B, n):
    """J = diag([[0, 1], [-1, 0]]) plus skew noise: pf = O(1) at any even n."""
    J = np.kron(np.eye(n // 2), np.array([[0.0, 1.0], [-1.0, 0.0]]))
    return (J + 0.25 * _skew(rng.standard_normal((B, n, n)) / np.sqrt(n))).astype(np.float32)


def _det_grad(A, dev):
    At = _t(A, dev).requires_grad_()
    d = fermix_amd.det(At)
    (gr,) = torch.autograd.grad(d.sum(), At)
    return _np(d), _np(gr)


def _pf_grad(S, dev):
    St = _t(S, dev).requires_grad_()
    p = fermix_amd.pf(St, skew_symmetrize=False)
    (gr,) = torch.autograd.grad(p.sum(), St)
    return _np(p), _np(gr)


# ------------------------------------------------------------------------ det


@pytest.mark.parametrize("n", [1, 2, 5, 64, 128, 129, 256, 512])
def test_det_grad_regular(dev, n):
    B = 6 if n <= 256 else 3
    rng = np.random.default_rng(6100 + n)
    A = _near_identity(rng, B, n)
    print(f"det regular n={n} B={B}", flush=True)
    sign, logabs, adjT = _kernels.det_parts(_t(A, dev))
    s0, l0 = fermix_amd.slogdet(_t(A, dev))
    assert torch.equal(sign, s0) and torch.equal(logabs, l0), "det primal != forward"
    d, gr = _det_grad(A, dev)
    assert np.array_equal(d, _np(s0 * torch.exp(l0)))
    assert np.array_equal(gr, _np(adjT))
    A64 = A.astype(np.float64)
    ref = np.linalg.det(A64)[:, None, None] * np.linalg.inv(A64).swapaxes(-1, -2)
    assert_grad(gr, ref, A, f"det n={n} vs float64")
    if n <= 256:
        _, Go = g.det_parts(A)
        assert_grad(gr, Go, A, f"det n={n} vs oracle")


@pytest.mark.parametrize("n", [3, 8, 40, 130, 300])
def test_det_grad_singular(dev, n):
    """Zero column (a zero pivot in the middle), zero row (a zero pivot at the end), zero
    matrix, two zero columns (rank n-2), zero column 0 plus zero row 1 (rank n-1 with two
    zero pivots) and a regular member, against the float64 SVD adjugate."""
    B = 6
    rng = np.random.default_rng(6200 + n)
    A = _near_identity(rng, B, n)
    A[0, :, 1] = 0.0
    A[1, 2 % n] = 0.0
    A[2] = 0.0
    A[3, :, 0] = 0.0
    A[3, :, 1 % n] = 0.0
    A[4, :, 0] = 0.0
    A[4, 1 % n] = 0.0
    print(f"det singular n={n}", flush=True)
    d, gr = _det_grad(A, dev)
    assert np.all(np.isfinite(gr))
    assert np.all(d[:5] == 0)
    ref = np.stack([ref64.adjT_svd(a) for a in A])
    scale = max(np.abs(ref).max(), 1e-30)
    assert np.max(np.abs(gr - ref)) < 1e-4 * scale
    assert np.all(gr[2] == 0) and np.all(gr[3] == 0)
    for k in (0, 1, 4, 5):  # rank n-1 members (and the regular one): nonzero, correct
        assert np.abs(ref[k]).max() > 0
        err = relerr(gr[k], ref[k])
        print(f"  member {k}: relerr {err:.3g}", flush=True)
        assert err < 1e-4, (k, err)
    # the oracle follows the same formula on its own LU
    if n <= 130:
        _, Go = g.det_parts(A)
        for k in range(B):
            assert np.max(np.abs(gr[k] - Go[k])) <= 1e-4 * max(np.abs(ref[k]).max(), 1e-30) + 1e-30


@pytest.mark.parametrize("n", [8, 24, 200])
def test_det_grad_near_singular(dev, n):
    """Numerically rank n-1 inputs (the last row a combination of the others, rounded to
    float32): a round-off pivot and no exact zero, where d det / dA is still the
    adjugate to working precision only if det and A^-T come from the same pivots."""
    B = 4
    rng = np.random.default_rng(6300 + n)
    A = rng.standard_normal((B, n, n)) * (1.0 if n <= 24 else 1.0 / np.sqrt(n))
    if n > 24:
        A += np.eye(n)
    c = rng.standard_normal((B, n - 1)) / np.sqrt(n)
    A[:, -1, :] = np.einsum("bi,bij->bj", c, A[:, :-1, :])
    A = A.astype(np.float32)
    _, gr = _det_grad(A, dev)
    ref = np.stack([ref64.adjT_svd(a) for a in A])
    for k in range(B):
        err = relerr(gr[k], ref[k])
        print(f"det near-singular n={n} member {k}: relerr {err:.3g}", flush=True)
        assert err < 1e-4, (k, err)


def test_det_jvp_vmap_and_bit_identity(dev):
    rng = np.random.default_rng(6400)
    n = 36
    A = _near_identity(rng, 6, n).reshape(3, 2, n, n)
    At = _t(A, dev)
    d0 = fermix_amd.det(At)
    dA = _t(rng.standard_normal(A.shape).astype(np.float32), dev)
    dp, dd = torch.func.jvp(lambda x: fermix_amd.det(x), (At,), (dA,))
    assert torch.equal(dp, d0)  # primal bit-identical to the plain forward
    A64 = A.astype(np.float64)
    adjT = np.linalg.det(A64)[..., None, None] * np.linalg.inv(A64).swapaxes(-1, -2)
    want = np.einsum("...ij,...ij->...", adjT, _np(dA).astype(np.float64))
    assert np.max(np.abs(_np(dd) - want)) < 1e-4 * max(1.0, np.abs(want).max())
    vd = torch.func.vmap(lambda x: fermix_amd.det(x))(At)
    assert torch.equal(vd, d0)
    gv = torch.func.vmap(torch.func.grad(lambda x: fermix_amd.det(x)))(At.reshape(6, n, n))
    assert_grad(_np(gv), adjT.reshape(6, n, n), A.reshape(6, n, n), "det vmap(grad)")


def test_det_adjugate_identity_large(dev):
    """n = 1024 (the largest LU size): adj(A) A = det(A) I in float64 for a regular and a
    zero-column member; the singular member's adjugate has rank one and A adj(A) = 0."""
    rng = np.random.default_rng(6500)
    n = 1024
    A = _near_identity(rng, 2, n)
    A[1, :, 17] = 0.0
    d, gr = _det_grad(A, dev)
    assert np.all(np.isfinite(gr)) and d[1] == 0
    A64 = A.astype(np.float64)
    G64 = gr.astype(np.float64)
    d64 = np.linalg.det(A64[0])
    res = G64[0].T @ A64[0] - d64 * np.eye(n)
    assert np.abs(res).max() < 1e-4 * abs(d64)
    adj1 = G64[1].T
    assert np.abs(adj1).max() > 0
    assert np.abs(adj1 @ A64[1]).max() < 1e-4 * np.abs(adj1).max() * np.abs(A64[1]).max() * np.sqrt(n)
    # only column 17 of adj(A)^T is nonzero for a zero column 17
    assert np.all(gr[1][:, :17] == 0) and np.all(gr[1][:, 18:] == 0)
    col = ref64.adjT_svd(A[1])[:, 17]
    assert np.max(np.abs(gr[1][:, 17] - col)) < 1e-4 * np.abs(col).max()


# ------------------------------------------------------------------------- pf


@pytest.mark.parametrize("n", [2, 6, 16, 64, 128, 130, 256, 512])
def test_pf_grad_regular(dev, n):
    B = 4 if n <= 256 else 2
    rng = np.random.default_rng(6600 + n)
    S = _near_j(rng, B, n)
    print(f"pf regular n={n} B={B}", flush=True)
    sign, logabs, adj = _kernels.slogpf_parts(_t(S, dev), False, adjugate=True)
    s0, l0 = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False)
    assert torch.equal(sign, s0) and torch.equal(logabs, l0), "pf primal != forward"
    p, gr = _pf_grad(S, dev)
    assert np.array_equal(p, _np(s0 * torch.exp(l0)))
    assert np.array_equal(gr, _np(-0.5 * adj))
    S64 = S.astype(np.float64)
    pf64 = np.array([ref64.pf64(x) for x in S64])
    ref = 0.5 * pf64[:, None, None] * np.linalg.inv(S64).swapaxes(-1, -2)
    assert_grad(gr, ref, S, f"pf n={n} vs float64")
    if n <= 130:
        _, _, Go, _ = g.pf_parts_generic(S, True)
        assert_grad(gr, -0.5 * Go, S, f"pf n={n} vs oracle")
    # skew_symmetrize=True: the gradient w.r.t. a through S = (a - a^T)/2 is the same G
    At = _t(S, dev).requires_grad_()
    (g2,) = torch.autograd.grad(fermix_amd.pf(At).sum(), At)
    assert np.array_equal(_np(g2), gr)


@pytest.mark.parametrize("n", [4, 8, 14, 130])
def test_pf_grad_singular(dev, n):
    """Zero row / column (rank n-2), zero matrix, two zero rows / columns (rank n-2 with
    two exact zero pivots: the lifted second evaluation) and a regular member, against
    float64 minor Pfaffians."""
    B = 4
    rng = np.random.default_rng(6700 + n)
    S = _skew(rng.standard_normal((B, n, n))) if n <= 14 else _near_j(rng, B, n)
    S[0, 3 % n, :] = 0.0
    S[0, :, 3 % n] = 0.0
    S[1] = 0.0
    S[2, 1, :] = 0.0
    S[2, :, 1] = 0.0
    S[2, 3 % n, :] = 0.0
    S[2, :, 3 % n] = 0.0
    print(f"pf singular n={n}", flush=True)
    p, gr = _pf_grad(S, dev)
    assert np.all(np.isfinite(gr))
    assert np.all(p[:3] == 0)
    if n <= 14:
        ref = np.stack([ref64.pf_grad64(x) for x in S])
    else:
        S64 = S.astype(np.float64)
        ref = np.stack([
            ref64.pf_grad64_rows(S64[0], [3]),
            np.zeros((n, n)),
            ref64.pf_grad64_rows(S64[2], [1, 3]),
            0.5 * ref64.pf64(S64[3]) * np.linalg.inv(S64[3]).T,
        ])
    scale = max(np.abs(ref).max(), 1e-30)
    assert np.max(np.abs(gr - ref)) < 1e-4 * scale
    assert np.all(gr[1] == 0) and np.abs(ref[0]).max() > 0
    if n > 4:  # n = 4 with rows 1 and 3 zeroed has pf' = 0 everywhere but (1, 3)
        assert np.abs(ref[2]).max() > 0
    for k in (0, 2, 3):
        if np.abs(ref[k]).max() > 0:
            err = relerr(gr[k], ref[k])
            print(f"  member {k}: relerr {err:.3g}", flush=True)
            assert err < 1e-4, (k, err)
    if n <= 130:
        _, _, Go, _ = g.pf_parts_generic(S, True)
        assert np.max(np.abs(gr - (-0.5 * Go))) < 1e-4 * scale


def _skew_rank_deficient(rng, B, n):
    """Numerically rank n-2 skew batch S = Q D Q^T rounded to float32, Q orthogonal, D =
    diag(sig_k J) with sig_k in [0.5, 1.5] and the last sig 0, with its exact Pfaffian
    adjugate pf(S) S^-1 = det(Q) Q diag(prod_{l != k} sig_l J^-1) Q^T -- only the last
    block survives: det(Q) prod_{l < h} sig_l Q_h J^-1 Q_h^T, Q_h the last two columns."""
    h = n // 2
    J = np.array([[0.0, 1.0], [-1.0, 0.0]])
    S = np.empty((B, n, n), np.float32)
    adj = np.empty((B, n, n))
    for b in range(B):
        Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
        sig = rng.uniform(0.5, 1.5, h)
        sig[-1] = 0.0
        D = np.kron(np.diag(sig), J)
        x = (Q @ D @ Q.T).astype(np.float32)
        S[b] = 0.5 * (x - x.T)
        Qh = Q[:, -2:]
        adj[b] = np.linalg.det(Q) * np.prod(sig[:-1]) * (Qh @ (-J) @ Qh.T)
    return S, adj


@pytest.mark.parametrize("n", [8, 24, 160])
def test_pf_grad_near_singular(dev, n):
    """Numerically rank n-2 inputs (rounded to float32): the two smallest pivots are
    round-off noise and d pf / dS must still be the Pfaffian adjugate to working
    precision. n <= 24: X J X^T (X of n-2 columns) against minor Pfaffians; n = 160: a
    rank n-2 Q D Q^T against its closed-form adjugate."""
    B = 4
    rng = np.random.default_rng(6800 + n)
    if n <= 24:
        X = rng.standard_normal((B, n, n - 2))
        J = np.kron(np.eye((n - 2) // 2), np.array([[0.0, 1.0], [-1.0, 0.0]]))
        S = (X @ J @ X.swapaxes(-1, -2)).astype(np.float32)
        S = S - S.swapaxes(-1, -2)
        ref = np.stack([ref64.pf_grad64(x) for x in S])
    else:
        S, adj = _skew_rank_deficient(rng, B, n)
        ref = -0.5 * adj
    _, gr = _pf_grad(S, dev)
    for k in range(B):
        err = relerr(gr[k], ref[k])
        print(f"pf near-singular n={n} member {k}: relerr {err:.3g}", flush=True)
        assert err < 1e-4, (k, err)
        adjk = -2.0 * gr[k].astype(np.float64)
        res = S[k].astype(np.float64) @ adjk
        assert np.abs(res).max() < 1e-4 * np.abs(adjk).max() * np.abs(S[k]).max() * np.sqrt(n)


def test_pf_jvp_vmap_and_bit_identity(dev):
    rng = np.random.default_rng(6900)
    n = 40
    S = _near_j(rng, 6, n).reshape(3, 2, n, n)
    St = _t(S, dev)
    p0 = fermix_amd.pf(St, skew_symmetrize=False)
    dS = _t(_skew(rng.standard_normal(S.shape)), dev)
    pp, dp = torch.func.jvp(lambda x: fermix_amd.pf(x, skew_symmetrize=False), (St,), (dS,))
    assert torch.equal(pp, p0)
    S64 = S.astype(np.float64)
    pf64 = np.array([ref64.pf64(x) for x in S64.reshape(6, n, n)]).reshape(3, 2)
    G = 0.5 * pf64[..., None, None] * np.linalg.inv(S64).swapaxes(-1, -2)
    want = np.einsum("...ij,...ij->...", G, _np(dS).astype(np.float64))
    assert np.max(np.abs(_np(dp) - want)) < 1e-4 * max(1.0, np.abs(want).max())
    vp = torch.func.vmap(lambda x: fermix_amd.pf(x, skew_symmetrize=False))(St)
    assert torch.equal(vp, p0)
    gv = torch.func.vmap(torch.func.grad(lambda x: fermix_amd.pf(x, skew_symmetrize=False)))(St.reshape(6, n, n))
    assert_grad(_np(gv), G.reshape(6, n, n), S.reshape(6, n, n), "pf vmap(grad)")


def test_pf_adjugate_identity_large(dev):
    """n = 1024: S adj = pf I in float64 for a regular member; a member with rows /
    columns 5 and 9 zeroed (two exact zero pivots, the lifted evaluation on the large
    path) has its only nonzero entries at (5, 9) and (9, 5), equal to the minor Pfaffian."""
    rng = np.random.default_rng(7000)
    n = 1024
    S = _near_j(rng, 2, n)
    for r in (5, 9):
        S[1, r, :] = 0.0
        S[1, :, r] = 0.0
    p, gr = _pf_grad(S, dev)
    assert np.all(np.isfinite(gr)) and p[1] == 0
    S64 = S.astype(np.float64)
    adj0 = -2.0 * gr[0].astype(np.float64)
    pf0 = ref64.pf64(S64[0])
    assert np.abs(S64[0] @ adj0 - pf0 * np.eye(n)).max() < 1e-4 * abs(pf0)
    mask = np.ones((n, n), bool)
    mask[5, 9] = mask[9, 5] = False
    keep = [k for k in range(n) if k not in (5, 9)]
    want = 0.5 * (-1) ** (5 + 9 + 1) * ref64.pf64(S64[1][np.ix_(keep, keep)])
    # the two lifted evaluations cancel everywhere else up to round-off
    assert np.abs(gr[1][mask]).max() < 1e-4 * abs(want)
    assert abs(gr[1][5, 9] - want) < 1e-4 * abs(want)
    assert abs(gr[1][9, 5] + want) < 1e-4 * abs(want)
