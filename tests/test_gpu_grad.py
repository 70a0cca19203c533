"""GPU parity of the gradients: slogdet (A^-T from the forward's own LU) against the CPU
oracle and float64 truth; torch autograd / forward mode / vmap integration and the
bit-identity of the differentiated primal (reference tests/test_fermix.py:309-326,
373-425, 442-456, 608-647)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_grad, assert_grad_vs_fp32, assert_logabs, lapack_inverse_f32, rel_fro

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


# The product mode (prec) changes the arithmetic only of the blocked kernels (n > 128):
# both the IEEE fp32 MFMA mode and the split-bf16x3 mode are held to the same bars there.
PRECS = {0: "ieee", 1: "bf16x3"}


def _with_modes(ns):
    return [(n, 1) for n in ns] + [(n, 0) for n in ns if n > 128]


@pytest.mark.parametrize("n,x3", _with_modes([1, 2, 5, 16, 17, 33, 48, 64, 100, 128, 129, 200, 256, 300, 320, 512]))
def test_slogdet_invT_vs_float64_and_oracle(dev, n, x3):
    B = 12 if n <= 256 else 4
    rng = np.random.default_rng(2000 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    print(f"invT n={n} B={B} prec={PRECS[x3]}", flush=True)
    s, l, invT, _, _ = _kernels.slogdet_parts(_t(A, dev), x3=x3)
    s0, l0 = fermix_amd.slogdet(_t(A, dev), prec=PRECS[x3])
    assert torch.equal(s, s0) and torch.equal(l, l0), "parts primal != forward"
    invT = _np(invT)
    ref = np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1)
    assert_grad(invT, ref, A, f"n={n} {PRECS[x3]} vs float64")
    _, _, invo, _, _, _ = g.lu_parts_generic(A)
    assert_grad(invT, invo, A, f"n={n} {PRECS[x3]} vs oracle")


@pytest.mark.parametrize("n", [12, 40, 150])
def test_slogdet_singular_gradient_zero(dev, n):
    rng = np.random.default_rng(3000 + n)
    A = rng.standard_normal((4, n, n)).astype(np.float32)
    A[0, :, 3] = 0.0
    A[2, 5, :] = 0.0
    At = _t(A, dev).requires_grad_()
    s, l = fermix_amd.slogdet(At)
    assert np.isneginf(_np(l)[0]) and np.isneginf(_np(l)[2])
    (gr,) = torch.autograd.grad(l[1] + l[3], At)
    gr = _np(gr)
    assert np.all(np.isfinite(gr))
    assert np.all(gr[0] == 0) and np.all(gr[2] == 0)
    ref = np.linalg.inv(A[1].astype(np.float64)).T
    assert_grad(gr[1:2], ref[None], A[1:2], "singular batch member 1")
    # zero_singular=False keeps the U~ inverse (finite) for the det gradient
    _, _, inv2, _, _ = _kernels.slogdet_parts(_t(A, dev), zero_singular=False)
    assert np.all(np.isfinite(_np(inv2)))


def test_autograd_jvp_vmap_and_bit_identity(dev):
    rng = np.random.default_rng(7)
    n = 48
    A = (rng.standard_normal((3, 2, n, n)) + 2 * np.eye(n)).astype(np.float32)
    At = _t(A, dev)
    s0, l0 = fermix_amd.slogdet(At)
    Ag = At.clone().requires_grad_()
    s1, l1 = fermix_amd.slogdet(Ag)
    assert torch.equal(s0, s1) and torch.equal(l0, l1)  # primal bit-identical
    w = torch.from_numpy(rng.standard_normal((3, 2)).astype(np.float32)).to(dev)
    (gr,) = torch.autograd.grad((l1 * w).sum(), Ag)
    ref = np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2) * _np(w)[:, :, None, None]
    assert np.max(np.abs(_np(gr) - ref)) < 1e-4 * np.abs(ref).max()
    # forward mode: d logabs = tr(A^-1 dA)
    dA = torch.from_numpy(rng.standard_normal(A.shape).astype(np.float32)).to(dev)
    (sp, lp), (ds, dl) = torch.func.jvp(lambda x: fermix_amd.slogdet(x), (At,), (dA,))
    assert torch.equal(lp, l0) and torch.all(ds == 0)
    want = np.einsum("...ij,...ij->...", np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2), _np(dA))
    assert np.max(np.abs(_np(dl) - want)) < 1e-3 * max(1.0, np.abs(want).max())
    # vmap over a leading dim == the batched call, bitwise
    vs, vl = torch.func.vmap(lambda x: fermix_amd.slogdet(x))(At)
    assert torch.equal(vs, s0) and torch.equal(vl, l0)
    # torch.func.grad of a vmapped per-sample function
    gfun = torch.func.vmap(torch.func.grad(lambda x: fermix_amd.slogdet(x)[1]))
    gv = gfun(At.reshape(6, n, n))
    ref1 = np.linalg.inv(A.reshape(6, n, n).astype(np.float64)).swapaxes(-1, -2)
    assert np.max(np.abs(_np(gv) - ref1)) < 1e-4 * np.abs(ref1).max()


def test_det_value_and_grad(dev):
    rng = np.random.default_rng(8)
    n = 20
    A = (rng.standard_normal((4, n, n)) / np.sqrt(n) + np.eye(n)).astype(np.float32)
    At = _t(A, dev).requires_grad_()
    d = fermix_amd.det(At)
    d64 = np.linalg.det(A.astype(np.float64))
    assert np.allclose(_np(d), d64, rtol=1e-4)
    (gr,) = torch.autograd.grad(d.sum(), At)
    ref = d64[:, None, None] * np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2)
    assert np.max(np.abs(_np(gr) - ref)) < 1e-4 * np.abs(ref).max()


@pytest.mark.parametrize("x3", [0, 1])
def test_c3_properties(dev, x3):
    """C3 size: B = 1024, n = 512, A iid N(0, 1/n), in both product modes. Primal
    bit-identical to the forward, gradient finite, 18 members against float64 truth, the
    oracle and float32 LAPACK (on average no less accurate than either), logabs and sign
    of the same members against float64."""
    rng = np.random.default_rng(3)
    B, n = 1024, 512
    A = (rng.standard_normal((B, n, n), dtype=np.float32) * np.float32(1 / np.sqrt(n)))
    At = _t(A, dev)
    what = f"C3 {PRECS[x3]}"
    s, l, invT, _, _ = _kernels.slogdet_parts(At, x3=x3)
    s0, l0 = fermix_amd.slogdet(At, prec=PRECS[x3])
    assert torch.equal(s, s0) and torch.equal(l, l0)
    assert bool(torch.isfinite(invT).all())
    idx = list(range(0, 1024, 64)) + [1, 1023]
    G = _np(invT[idx])
    ref = np.linalg.inv(A[idx].astype(np.float64)).transpose(0, 2, 1)
    assert_grad(G, ref, A[idx], f"{what} subset vs float64")
    # no worse than the fp32 references on the same members: the oracle (the reference's
    # generic path restated) and float32 LAPACK
    _, _, invo, _, _, _ = g.lu_parts_generic(A[idx])
    assert_grad_vs_fp32(G, ref, rel_fro(invo, ref), f"{what} subset vs the oracle's error")
    inv32 = lapack_inverse_f32(A[idx]).transpose(0, 2, 1)
    assert_grad_vs_fp32(G, ref, rel_fro(inv32, ref), f"{what} subset vs fp32 LAPACK's error")
    s64, l64 = ref64.slogdet64(A[idx])
    assert np.array_equal(_np(s)[idx], s64)
    assert_logabs(_np(l)[idx], l64, n, f"{what} subset logabs vs float64", A[idx])


@pytest.mark.parametrize("n,x3", _with_modes([2, 4, 6, 10, 16, 34, 64, 96, 128, 130, 256, 300, 512]))
def test_slogpf_grad_vs_float64_and_oracle(dev, n, x3):
    B = 8 if n <= 256 else 3
    rng = np.random.default_rng(5000 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    print(f"slogpf grad n={n} B={B} prec={PRECS[x3]}", flush=True)
    s, l, Sinv = _kernels.slogpf_parts(_t(S, dev), False, x3=x3)
    s0, l0 = fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False, prec=PRECS[x3])
    assert torch.equal(s, s0) and torch.equal(l, l0), "parts primal != forward"
    Sinv = _np(Sinv)
    ref = np.linalg.inv(S.astype(np.float64))
    assert_grad(Sinv, ref, S, f"n={n} {PRECS[x3]} vs float64")
    if n <= 256:
        _, _, So, _ = g.pf_parts_generic(S, False)
        assert_grad(Sinv, So, S, f"n={n} {PRECS[x3]} vs oracle")
    # the autograd route of the same mode: -S^-1 / 2 from the saved factors
    Sg = _t(S, dev).requires_grad_()
    _, la = fermix_amd.slogpf(Sg, skew_symmetrize=False, prec=PRECS[x3])
    (gr,) = torch.autograd.grad(la.sum(), Sg)
    assert torch.equal(gr, -0.5 * _t(Sinv, dev))


def test_slogpf_autograd_and_singular(dev):
    rng = np.random.default_rng(77)
    n = 40
    A = rng.standard_normal((4, n, n)).astype(np.float32)
    A[0, 7, :] = 0.0
    A[0, :, 7] = 0.0  # S = (A - A^T)/2 has row/column 7 exactly zero
    At = _t(A, dev).requires_grad_()
    s, l = fermix_amd.slogpf(At)
    s0, l0 = fermix_amd.slogpf(_t(A, dev))
    assert torch.equal(s, s0) and torch.equal(l, l0)
    assert np.isneginf(_np(l)[0])
    (gr,) = torch.autograd.grad(l[1:].sum(), At)
    gr = _np(gr)
    assert np.all(np.isfinite(gr)) and np.all(gr[0] == 0)
    S = 0.5 * (A.astype(np.float64) - A.astype(np.float64).transpose(0, 2, 1))
    ref = 0.5 * np.linalg.inv(S[1:]).transpose(0, 2, 1)  # d log|pf| / da = S^-T / 2
    assert np.max(np.abs(gr[1:] - ref)) < 1e-4 * np.abs(ref).max()
    # forward mode and vmap
    dA = torch.from_numpy(rng.standard_normal(A.shape).astype(np.float32)).to(dev)
    (_, lp), (_, dl) = torch.func.jvp(lambda x: fermix_amd.slogpf(x), (_t(A, dev),), (dA,))
    dS = 0.5 * (_np(dA) - _np(dA).transpose(0, 2, 1)).astype(np.float64)
    want = 0.5 * np.einsum("bij,bji->b", np.linalg.inv(S[1:]), dS[1:])
    assert np.max(np.abs(_np(dl)[1:] - want)) < 1e-3 * max(1.0, np.abs(want).max())
    vs, vl = torch.func.vmap(lambda x: fermix_amd.slogpf(x))(_t(A, dev)[None])
    assert torch.equal(vs[0], s0) and torch.equal(vl[0], l0)


@pytest.mark.parametrize("x3", [0, 1])
def test_c4_properties(dev, x3):
    """C4 size: B = 64, n = 2048, S = A - A^T, A iid N(0, 1/n), in both product modes.
    Primal bit-identical to the forward, gradient finite and skew, 6 members against
    float64 truth and float32 LAPACK (on average no less accurate), |pf|^2 = |det| of the
    same members against float64."""
    rng = np.random.default_rng(4)
    B, n = 64, 2048
    A = rng.standard_normal((B, n, n), dtype=np.float32) * np.float32(1 / np.sqrt(n))
    S = A - A.transpose(0, 2, 1)
    del A
    St = _t(S, dev)
    what = f"C4 {PRECS[x3]}"
    s, l, Sinv = _kernels.slogpf_parts(St, False, x3=x3)
    s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False, prec=PRECS[x3])
    assert torch.equal(s, s0) and torch.equal(l, l0)
    assert bool(torch.isfinite(Sinv).all())
    idx = [0, 1, 2, 31, 62, 63]
    G = _np(Sinv[idx])
    assert np.max(np.abs(G + G.transpose(0, 2, 1))) <= 1e-6 * np.abs(G).max()
    ref = np.linalg.inv(S[idx].astype(np.float64))
    assert_grad(G, ref, S[idx], f"{what} subset vs float64")
    inv32 = lapack_inverse_f32(S[idx])
    assert_grad_vs_fp32(G, ref, rel_fro(inv32, ref), f"{what} subset vs fp32 LAPACK's error")
    _, ld64 = ref64.slogdet64(S[idx])
    assert_logabs(_np(l)[idx], 0.5 * ld64, n, f"{what} subset log|pf| vs log|det| / 2 float64", S[idx])


@pytest.mark.parametrize("n", [40, 129, 200, 512])
def test_slogdet_inverse_from_factors(dev, n):
    """fx_slogdet_factors_f32 + fx_slogdet_inverse_f32 (scale = a cotangent) against the
    one-call parts route times the cotangent: the same LU, the same inverse, and the scale
    applied once either way, so bit-identical; the primal bit-identical to the forward."""
    B = 5
    rng = np.random.default_rng(9100 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    A[2, :, n // 3] = 0.0  # exactly singular member: zero gradient
    At = _t(A, dev)
    w = _t(rng.standard_normal(B).astype(np.float32), dev)
    print(f"inverse from factors n={n}", flush=True)
    s, l, lu, perm = _kernels.slogdet_factors(At)
    s0, l0 = fermix_amd.slogdet(At)
    assert torch.equal(s, s0) and torch.equal(l, l0)
    _, _, invT, _, _ = _kernels.slogdet_parts(At)
    g = _kernels.slogdet_inverse(lu, perm, s, n, scale=w)
    assert torch.equal(g, w[:, None, None] * invT)
    assert torch.all(g[2] == 0)
    # the autograd route (factors in the forward, the scaled inverse in the backward),
    # including a second backward of a retained graph (the first overwrote the LU)
    Ag = At.clone().requires_grad_()
    _, la = fermix_amd.slogdet(Ag)
    (g1,) = torch.autograd.grad((la * w).sum(), Ag, retain_graph=True)
    (g2,) = torch.autograd.grad((la * w).sum(), Ag)
    assert torch.equal(g1, g) and torch.equal(g2, g)


@pytest.mark.parametrize("n", [34, 130, 512, 1000])
def test_slogpf_inverse_from_factors(dev, n):
    """fx_slogpf_factors_f32 + fx_slogpf_inverse_f32 (scale = -cotangent / 2) against the
    parts route times the same scale (bit-identical), both modes; the autograd route."""
    B = 4
    rng = np.random.default_rng(9200 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    S[1, n // 5, :] = 0.0
    S[1, :, n // 5] = 0.0
    St = _t(S, dev)
    w = _t(rng.standard_normal(B).astype(np.float32), dev)
    print(f"pf inverse from factors n={n}", flush=True)
    s, l, gbuf, d, perm = _kernels.slogpf_factors(St, False)
    for adj in (False, True):
        _, _, G = _kernels.slogpf_parts(St, False, adjugate=adj)
        g = _kernels.slogpf_inverse(gbuf, d, perm, n, scale=-0.5 * w, adjugate=adj)
        assert torch.equal(g, (-0.5 * w)[:, None, None] * G), f"adjugate={adj}"
    Sg = St.clone().requires_grad_()
    _, la = fermix_amd.slogpf(Sg, skew_symmetrize=False)
    (g1,) = torch.autograd.grad((la * w).sum(), Sg)
    _, _, G = _kernels.slogpf_parts(St, False)
    assert torch.equal(g1, (-0.5 * w)[:, None, None] * G)
