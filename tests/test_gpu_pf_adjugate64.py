"""GPU parity of pf's gradient, the Pfaffian adjugate pf(S) S^-1, for the float64 and
complex kinds (fx_slogpf_parts_f64 / _c64 / _c128 with adjugate != 0): regular members
against pf(S) S^-1 in float64 / complex128, singular ones (one and two exact zero pivots,
rank n - 2; three, rank n - 4) against minor Pfaffians, and the autograd / jvp rules with
torch's conjugate convention -- the reference's pf gradient tests for every dtype
(tests/test_fermix.py:522-610)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import relerr

pytestmark = pytest.mark.gpu

KINDS = {"f64": (np.float64, 1e-10), "c64": (np.complex64, 5e-5), "c128": (np.complex128, 1e-10)}


def _np(x):
    return x.detach().cpu().numpy()


def _jmat(n):
    J = np.zeros((n, n))
    for i in range(0, n - 1, 2):
        J[i, i + 1], J[i + 1, i] = 1.0, -1.0
    return J


def _near_j(rng, B, n, dt):
    """X J X^T with X = I + N(0, 1/(4n)) (complex: both parts): pf = det(X) = O(1)."""
    X = rng.standard_normal((B, n, n))
    if np.dtype(dt).kind == "c":
        X = X + 1j * rng.standard_normal((B, n, n))
    X = np.eye(n) + 0.5 * X / np.sqrt(n)
    S = X @ _jmat(n) @ np.swapaxes(X, 1, 2)
    return (0.5 * (S - np.swapaxes(S, 1, 2))).astype(dt)


def _wide(x):
    return x.astype(np.complex128 if np.iscomplexobj(x) else np.float64)


def _pf_adj(S, dev):
    """(sign, logabs, pf(S) S^-1) through the C ABI's adjugate mode (input already skew)."""
    St = torch.from_numpy(S).to(dev)
    sign, logabs, G = _kernels.slogpf_parts(St, False, adjugate=True)
    return St, sign, logabs, _np(G)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [2, 4, 16, 30, 64, 100, 130, 256])
def test_pf_adjugate_regular(dev, kind, n):
    """pf(S) S^-1 against float64 / complex128; the primal bit-identical to the plain
    slogpf forward; the pf gradient (autograd, with skew_symmetrize on a skew input) is
    -pf(S) S^-1 / 2, conjugated for the complex kinds, and the jvp is sum(G * dS)."""
    dt, tol = KINDS[kind]
    rng = np.random.default_rng(9300 + n)
    S = _near_j(rng, 3, n, dt)
    print(f"pf adjugate {kind} n={n}", flush=True)
    St, sign, logabs, G = _pf_adj(S, dev)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert torch.equal(sign, s0) and torch.equal(logabs, l0), "pf primal != forward"
    W = _wide(S)
    pf_ref = np.array([ref64.pf64(x) for x in W])
    ref = pf_ref[:, None, None] * np.linalg.inv(W)
    err = relerr(G, ref)
    print(f"  relerr {err:.3g}", flush=True)
    assert err < tol * max(1.0, n / 16)
    X = St.clone().requires_grad_(True)
    p = fermix_amd.pf(X)
    assert torch.equal(p.detach(), s0 * torch.exp(l0))
    (gr,) = torch.autograd.grad(p.real.sum() if p.is_complex() else p.sum(), X)
    gr = _np(gr)
    if kind != "f64":
        gr = gr.conj()  # torch's conjugate-Wirtinger gradient -> d pf / dS
    assert relerr(gr, -0.5 * ref) < tol * max(1.0, n / 16)
    dS = _near_j(rng, 3, n, dt) - _near_j(rng, 3, n, dt)
    _, dp = torch.func.jvp(fermix_amd.pf, (St,), (torch.from_numpy(dS).to(dev),))
    want = (-0.5 * ref * _wide(dS)).sum(axis=(1, 2))
    assert np.max(np.abs(_np(dp) - want)) < tol * max(1.0, n / 16) * np.abs(want).max() * 10


def _zero_rows(S, b, rows):
    for r in rows:
        S[b, r % S.shape[1], :] = 0.0
        S[b, :, r % S.shape[1]] = 0.0


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [4, 8, 10, 40, 130])
def test_pf_adjugate_singular(dev, kind, n):
    """Members: one zero row / column (one exact zero pivot, rank n - 2), rows 0 and 2
    zero (two exact zero pivots, rank n - 2: the lifted evaluations), rows 0, 2 and 4
    zero (rank n - 4: zero adjugate; for n = 4 the zero matrix), and a regular member,
    against minor Pfaffians (all entries for n <= 10, the zeroed rows' entries, which are
    then the only nonzero ones, above) and the oracle's generic formula."""
    dt, tol = KINDS[kind]
    rng = np.random.default_rng(9400 + n)
    S = _near_j(rng, 4, n, dt)
    _zero_rows(S, 0, [3])
    _zero_rows(S, 1, [0, 2])
    _zero_rows(S, 2, [0, 2, 4] if n > 4 else [0, 1, 2, 3])
    print(f"pf adjugate singular {kind} n={n}", flush=True)
    St, sign, logabs, G = _pf_adj(S, dev)
    assert np.all(np.isfinite(G)) and np.all(_np(sign)[:3] == 0)
    W = _wide(S)
    grad = -0.5 * G
    if n <= 10:
        ref = [ref64.pf_grad64(x) for x in W[:3]]
    else:
        ref = [ref64.pf_grad64_rows(W[0], [3]), ref64.pf_grad64_rows(W[1], [0, 2]), np.zeros((n, n), W.dtype)]
    ref.append(0.5 * ref64.pf64(W[3]) * np.linalg.inv(W[3]).T)
    ref = np.stack(ref)
    assert np.all(grad[2] == 0), "rank n - 4: zero adjugate"
    for k in (0, 1, 3):
        assert np.abs(ref[k]).max() > 0
        err = relerr(grad[k], ref[k])
        print(f"  member {k}: relerr {err:.3g}", flush=True)
        assert err < tol * max(1.0, n / 16), (k, err)
    if n <= 40:
        _, _, Go, _ = g.pf_parts_generic(W, True)
        assert relerr(G, Go) < tol * max(1.0, n / 16)
    # autograd through pf: finite, equal to the adjugate (conjugated for complex)
    X = St.clone().requires_grad_(True)
    p = fermix_amd.pf(X)
    (gr,) = torch.autograd.grad(p.real.sum() if p.is_complex() else p.sum(), X)
    gr = _np(gr)
    if kind != "f64":
        gr = gr.conj()
    assert np.array_equal(gr, grad)


@pytest.mark.parametrize("kind", list(KINDS))
def test_pf_adjugate_odd_and_empty(dev, kind):
    """Odd n: pf = 0 and a zero gradient; n = 0: pf = 1 and an empty gradient."""
    dt, _ = KINDS[kind]
    rng = np.random.default_rng(9500)
    for n in (3, 7):
        A = rng.standard_normal((2, n, n)).astype(dt)
        X = torch.from_numpy(A).to(dev).requires_grad_(True)
        p = fermix_amd.pf(X)
        assert np.all(_np(p) == 0)
        (gr,) = torch.autograd.grad(p.real.sum() if p.is_complex() else p.sum(), X)
        assert np.all(_np(gr) == 0)
    X = torch.zeros((2, 0, 0), dtype=torch.from_numpy(np.zeros(1, dt)).dtype, device=dev).requires_grad_(True)
    p = fermix_amd.pf(X)
    assert np.all(_np(p) == 1)


def test_pf_adjugate_f64_blocked(dev):
    """float64 above the register kernels (n = 520): a regular member takes pf(S) S^-1 from
    the blocked LU solves scaled by the Parlett-Reid pf (against float64 numpy), a member
    with a zero row / column k takes the Parlett-Reid adjugate (rank n - 2: only row and
    column k nonzero; entries against minor Pfaffians, G[i][j] = (-1)^(i+j) pf(S without
    i, j) for i < j)."""
    n, k = 520, 77
    rng = np.random.default_rng(9600)
    S = _near_j(rng, 2, n, np.float64)
    _zero_rows(S, 1, [k])
    print(f"pf adjugate f64 blocked n={n}", flush=True)
    St, sign, logabs, G = _pf_adj(S, dev)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert torch.equal(sign, s0) and torch.equal(logabs, l0)
    assert _np(sign)[1] == 0 and np.all(np.isfinite(G))
    ref = ref64.pf64(S[0]) * np.linalg.inv(S[0])
    err = relerr(G[0], ref)
    print(f"  regular relerr {err:.3g}", flush=True)
    assert err < 1e-10 * n / 16
    G1 = G[1]
    off = G1.copy()
    off[k, :] = 0.0
    off[:, k] = 0.0
    assert np.abs(off).max() <= 1e-10 * np.abs(G1).max()
    assert np.allclose(G1, -G1.T, rtol=0, atol=1e-10 * np.abs(G1).max())
    for j in (0, 300, n - 1):
        i, jj = min(k, j), max(k, j)
        keep = [x for x in range(n) if x not in (i, jj)]
        want = (-1.0) ** (i + jj) * ref64.pf64(S[1][np.ix_(keep, keep)])
        got = G1[i, jj]
        print(f"  G[{i}][{jj}] {got:.10g} vs {want:.10g}", flush=True)
        assert abs(got - want) <= 1e-9 * abs(want)


def _rank_deficient_xjx(rng, n, dt):
    """S = X J X^T with X = I + N(0, 1/(4n)) (complex: both parts) projected to rank n - 2
    (its two smallest singular values set to zero): pf(S) = det(X) = 0 exactly, so the
    stored S is singular up to its rounding and its adjugate pf(S) S^-1 is the rank-2
    matrix of the (n - 2)-minor Pfaffians."""
    X = rng.standard_normal((n, n))
    if np.dtype(dt).kind == "c":
        X = X + 1j * rng.standard_normal((n, n))
    X = np.eye(n) + 0.5 * X / np.sqrt(n)
    U, sv, Vt = np.linalg.svd(X)
    sv[-2:] = 0.0
    X = (U * sv) @ Vt
    S = X @ _jmat(n) @ X.T
    return (0.5 * (S - S.T)).astype(dt)


@pytest.mark.parametrize("kind", list(KINDS))
@pytest.mark.parametrize("n", [130, 256])
def test_pf_adjugate_numerically_singular(dev, kind, n):
    """A numerically singular member (S = X J X^T, X of rank n - 2: pf(S) at round-off
    level) beside a regular one at the blocked sizes. pf(S) times an LU inverse of S would
    be off by O(1) there (the LU's two small pivots and the Parlett-Reid run's small pair
    pivot come from different factorisations); the member must take the pivot-replaced
    formula. Entries against minor Pfaffians, G[i][j] = (-1)^(i+j) pf(S without i, j) for
    i < j, at the largest entries and at random ones; S G = pf(S) I ~ 0 and G skew; the
    regular member against pf(S) S^-1 in float64 / complex128."""
    dt, tol = KINDS[kind]
    rng = np.random.default_rng(9700 + n)
    S = np.stack([_rank_deficient_xjx(rng, n, dt), _near_j(rng, 1, n, dt)[0]])
    print(f"pf adjugate numerically singular {kind} n={n}", flush=True)
    St, sign, logabs, G = _pf_adj(S, dev)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert torch.equal(sign, s0) and torch.equal(logabs, l0)
    assert np.all(np.isfinite(G))
    W = _wide(S)
    bar = tol * max(1.0, n / 16)
    # the regular member: the LU route
    ref = ref64.pf64(W[1]) * np.linalg.inv(W[1])
    err = relerr(G[1], ref)
    print(f"  regular relerr {err:.3g}", flush=True)
    assert err < bar
    G0 = _wide(G[0])
    scale = np.abs(G0).max()
    assert scale > 0
    assert np.abs(G0 + G0.T).max() <= bar * scale
    res = np.abs(W[0] @ G0).max() / (np.abs(W[0]).max() * scale * n)
    print(f"  |S G| / (|S| |G| n) {res:.3g}", flush=True)
    assert res < bar
    iu, ju = np.triu_indices(n, 1)
    order = np.argsort(-np.abs(G0[iu, ju]))
    picks = list(order[:6]) + list(rng.choice(order[6:], 6, replace=False))
    worst = 0.0
    for t in picks:
        i, j = int(iu[t]), int(ju[t])
        keep = [x for x in range(n) if x not in (i, j)]
        want = (-1.0) ** (i + j) * ref64.pf64(W[0][np.ix_(keep, keep)])
        worst = max(worst, abs(G0[i, j] - want) / scale)
    print(f"  minor Pfaffians: max |G - want| / max |G| {worst:.3g}", flush=True)
    assert worst < bar
