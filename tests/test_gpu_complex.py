"""GPU parity of the complex64 / complex128 paths (csrc/cplx.hip) -- the reference's
complex kinds (src/fermix/_field.py:32-162; tests/test_fermix.py:321-372): values against
numpy's complex128 slogdet, the perfect-matching Pfaffian and the complex oracle;
derivatives with jnp.linalg's conventions (d logabs = Re t, d sign = i Im(t) sign,
t = tr(A^-1 dA)), checked against closed forms and against torch.linalg.slogdet's own
complex autograd on the CPU; singular and odd-n conventions."""

import numpy as np
import pytest
import torch

import fermix_amd
from oracle import generic as g
from oracle import ref64
from tests.tolerances import rel_fro, relerr

pytestmark = pytest.mark.gpu

DT = {"c64": (np.complex64, torch.complex64), "c128": (np.complex128, torch.complex128)}


def _np(x):
    return x.detach().cpu().numpy()


def _crandn(rng, shape, dtype):
    return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(dtype)


def _tols(kind, n):
    """(phase / logabs tolerance, gradient relative tolerance) by precision class: the
    float32 bars (logabs 1e-5 max(1, |l|) + 1e-6 n, gradients 1e-4) for complex64, the
    float64 ones for complex128."""
    if kind == "c64":
        return 1e-5 * max(1.0, n / 8), 1e-4 * max(1.0, n / 64)
    return 1e-11 * max(1.0, n / 8), 1e-10 * max(1.0, n / 64)


@pytest.mark.parametrize("kind", ["c64", "c128"])
@pytest.mark.parametrize("n", [1, 2, 5, 16, 33, 64, 90, 128, 200, 300])
def test_complex_slogdet_values_and_inverse(dev, kind, n):
    """Values against numpy's complex128 slogdet and the oracle (LAPACK cgetrf / zgetrf);
    A^-T (no conjugation) against numpy's inverse; sizes on both sides of the LDS limit."""
    npdt, tdt = DT[kind]
    rng = np.random.default_rng(8000 + n)
    B = 6 if n <= 128 else 3
    A = (_crandn(rng, (B, n, n), npdt) / np.sqrt(n)).astype(npdt)
    A[1] += 2 * np.eye(n, dtype=npdt)
    print(f"complex slogdet {kind} n={n}", flush=True)
    At = torch.from_numpy(A).to(dev)
    s, l = map(_np, fermix_amd.slogdet(At))
    assert s.dtype == npdt and l.dtype == np.finfo(npdt).dtype
    s64, l64 = ref64.slogdet64(A)
    tl, tg = _tols(kind, n)
    tl_l = tl * np.maximum(1.0, np.abs(l64))
    assert np.all(np.abs(l - l64) < tl_l), np.max(np.abs(l - l64))
    assert np.max(np.abs(s - s64)) < tl * max(1.0, np.max(np.abs(l64))), np.max(np.abs(s - s64))
    assert np.max(np.abs(np.abs(s) - 1)) < 10 * tl
    so, lo = g.slogdet_generic(A)
    assert np.max(np.abs(s - so)) < 2 * tl * max(1.0, np.max(np.abs(l64)))
    sp, lp, invT = map(_np, fermix_amd._kernels.slogdet_parts(At)[:3])
    assert np.array_equal(sp, s) and np.array_equal(lp, l)
    ref = np.linalg.inv(A.astype(np.complex128)).transpose(0, 2, 1)
    err = rel_fro(invT, ref)
    k = np.linalg.cond(A.astype(np.complex128))
    lim = np.maximum(tg, (2.0**-24 if kind == "c64" else 2.0**-53) * 8 * k)
    assert np.all(err <= lim), (err, lim)


@pytest.mark.parametrize("kind", ["c64", "c128"])
@pytest.mark.parametrize("n", [2, 4, 8, 16, 64, 96, 128, 256])
def test_complex_slogpf_values_and_inverse(dev, kind, n):
    """pf against the perfect-matching expansion (n <= 8) and the complex128 Parlett-Reid,
    pf^2 = det, S^-1 against numpy's inverse, skew_symmetrize on and off."""
    npdt, tdt = DT[kind]
    rng = np.random.default_rng(8100 + n)
    B = 4
    A = (_crandn(rng, (B, n, n), npdt) / np.sqrt(n)).astype(npdt)
    S = (A - A.transpose(0, 2, 1)).astype(npdt)
    print(f"complex slogpf {kind} n={n}", flush=True)
    St = torch.from_numpy(S).to(dev)
    s, l = map(_np, fermix_amd.slogpf(St, skew_symmetrize=False))
    tl, tg = _tols(kind, n)
    if n <= 8:
        brute = np.array([ref64.pf_brute(x) for x in S])
        assert np.max(np.abs(s * np.exp(l) - brute)) < 10 * tl * np.max(np.abs(brute))
    s64, l64 = ref64.slogpf64(S)
    scale = max(1.0, float(np.max(np.abs(l64))))
    assert np.max(np.abs(l - l64)) < tl * scale and np.max(np.abs(s - s64)) < tl * scale
    sd, ld = ref64.slogdet64(S)
    assert np.max(np.abs(s * s - sd)) < 4 * tl * scale and np.max(np.abs(2 * l - ld)) < 4 * tl * scale
    # skew_symmetrize=True on A gives pf((A - A^T) / 2) = pf(S) / 2^(n/2)
    s2, l2 = map(_np, fermix_amd.slogpf(torch.from_numpy(A).to(dev)))
    assert np.max(np.abs(l2 - (l - (n // 2) * np.log(2.0)))) < tl * scale
    assert np.max(np.abs(s2 - s)) < tl * scale
    _, _, G = map(_np, fermix_amd._kernels.slogpf_parts(St, False))
    ref = np.linalg.inv(S.astype(np.complex128))
    assert np.all(rel_fro(G, ref) <= np.maximum(tg, (2.0**-24 if kind == "c64" else 2.0**-53) * 8 *
                                               np.linalg.cond(S.astype(np.complex128))))


@pytest.mark.parametrize("kind", ["c64", "c128"])
def test_complex_gradients_match_torch_linalg(dev, kind):
    """Reverse mode: d logabs / dA = conj(A^-T) (torch's conjugate-Wirtinger form of the
    reference's A^-T), the sign's cotangent included, equal to torch.linalg.slogdet's own
    complex autograd on the CPU; forward mode: d logabs = Re t and d sign = i Im(t) sign
    (the reference's test_complex_conventions_match_jnp_linalg, tests/test_fermix.py:
    329-361); slogpf: the same with t = tr(S^-1 dS) / 2, S the skew-symmetrised input."""
    npdt, tdt = DT[kind]
    n = 24
    rng = np.random.default_rng(8200)
    A = (_crandn(rng, (3, n, n), npdt) / np.sqrt(n) + 2 * np.eye(n)).astype(npdt)
    dA = _crandn(rng, (3, n, n), npdt)
    tl, tg = _tols(kind, n)
    rt = 100 * tg
    X = torch.from_numpy(A).to(dev).requires_grad_(True)
    s, l = fermix_amd.slogdet(X)
    w = torch.tensor([0.3 - 0.7j, 1.1 + 0.2j, -0.5 + 0.4j], dtype=tdt)
    loss = l.sum() + (w.to(dev).conj() * s).real.sum()
    (g,) = torch.autograd.grad(loss, X)
    Xc = torch.from_numpy(A.astype(np.complex128)).requires_grad_(True)
    sc, lc = torch.linalg.slogdet(Xc)
    (gc,) = torch.autograd.grad(lc.sum() + (w.to(torch.complex128).conj() * sc).real.sum(), Xc)
    assert relerr(_np(g), gc.numpy()) < rt
    Y = torch.from_numpy(A).to(dev).requires_grad_(True)
    (g1,) = torch.autograd.grad(fermix_amd.slogdet(Y)[1].sum(), Y)
    inv = np.linalg.inv(A.astype(np.complex128))
    assert relerr(_np(g1), inv.transpose(0, 2, 1).conj()) < rt
    # forward mode
    import torch.autograd.forward_ad as fwAD

    with fwAD.dual_level():
        D = fwAD.make_dual(torch.from_numpy(A).to(dev), torch.from_numpy(dA).to(dev))
        s2, l2 = fermix_amd.slogdet(D)
        ds, dl = _np(fwAD.unpack_dual(s2).tangent), _np(fwAD.unpack_dual(l2).tangent)
        s2 = _np(fwAD.unpack_dual(s2).primal)
    t = np.einsum("bij,bji->b", inv, dA.astype(np.complex128))
    assert np.allclose(dl, t.real, rtol=rt, atol=rt)
    assert np.allclose(ds, 1j * t.imag * s2, rtol=rt, atol=rt)
    # slogpf: gradient w.r.t. the input a through S = (a - a^T) / 2
    Z = torch.from_numpy(A).to(dev).requires_grad_(True)
    (gp,) = torch.autograd.grad(fermix_amd.slogpf(Z)[1].sum(), Z)
    S = 0.5 * (A - A.transpose(0, 2, 1)).astype(np.complex128)
    Sinv = np.linalg.inv(S)
    assert relerr(_np(gp), 0.5 * Sinv.transpose(0, 2, 1).conj()) < rt
    with fwAD.dual_level():
        D = fwAD.make_dual(torch.from_numpy(A).to(dev), torch.from_numpy(dA).to(dev))
        s3, l3 = fermix_amd.slogpf(D)
        ds3, dl3 = _np(fwAD.unpack_dual(s3).tangent), _np(fwAD.unpack_dual(l3).tangent)
        s3 = _np(fwAD.unpack_dual(s3).primal)
    tp = 0.5 * np.einsum("bij,bji->b", Sinv, dA.astype(np.complex128))
    assert np.allclose(dl3, tp.real, rtol=rt, atol=rt)
    assert np.allclose(ds3, 1j * tp.imag * s3, rtol=rt, atol=rt)


@pytest.mark.parametrize("kind", ["c64", "c128"])
def test_complex_singular_odd_and_det_pf(dev, kind):
    """An exactly singular member gives (0, -inf) and a zero gradient; odd n gives
    (0, -inf) for slogpf and 0 for pf; det / pf values are sign * exp(logabs) of the same
    run; batch dims and vmap fold into the batch."""
    npdt, tdt = DT[kind]
    n = 20
    rng = np.random.default_rng(8300)
    A = (_crandn(rng, (4, n, n), npdt) / np.sqrt(n)).astype(npdt)
    A[2, :, 5] = 0
    X = torch.from_numpy(A).to(dev).requires_grad_(True)
    s, l = fermix_amd.slogdet(X)
    (gx,) = torch.autograd.grad(l.sum(), X)
    assert _np(s)[2] == 0 and _np(l)[2] == -np.inf
    assert np.all(_np(gx)[2] == 0) and np.all(np.isfinite(_np(gx)))
    S = (A - A.transpose(0, 2, 1)).astype(npdt)
    S[1, 3, :] = 0
    S[1, :, 3] = 0
    ps, pl = map(_np, fermix_amd.slogpf(torch.from_numpy(S).to(dev), skew_symmetrize=False))
    assert ps[1] == 0 and pl[1] == -np.inf
    odd = torch.from_numpy(_crandn(rng, (2, 7, 7), npdt)).to(dev)
    os_, ol = map(_np, fermix_amd.slogpf(odd))
    assert np.all(os_ == 0) and np.all(ol == -np.inf)
    assert np.all(_np(fermix_amd.pf(odd)) == 0)
    At = torch.from_numpy(A).to(dev)
    st, lt = fermix_amd.slogdet(At)
    assert torch.equal(fermix_amd.det(At), st * torch.exp(lt))
    d64 = np.linalg.det(A.astype(np.complex128))
    tl, _ = _tols(kind, n)
    assert np.allclose(_np(fermix_amd.det(At)), d64, rtol=100 * tl, atol=0)
    # batch dims and vmap
    A4 = At.reshape(2, 2, n, n)
    s4, l4 = fermix_amd.slogdet(A4)
    assert torch.equal(s4.reshape(-1), st) and torch.equal(l4.reshape(-1), lt)
    sv, lv = torch.func.vmap(fermix_amd.slogdet)(A4)
    assert torch.equal(sv.reshape(-1), st) and torch.equal(lv.reshape(-1), lt)


@pytest.mark.parametrize("kind", ["c64", "c128"])
def test_complex_blocked_large(dev, kind):
    """The blocked complex kernels at n = 1030 (padded order 1056, 1024-thread panels):
    slogdet of X = I + N(0, 1/(4n)) (both parts) against numpy's complex128 slogdet, A^-T
    through its residual X^T A^-T - I (complex128 on the CPU), and pf(X J X^T) = det(X)
    with its S^-1 residual; a zero row / column gives pf = 0 and leaves the other member's
    bits unchanged."""
    nd, td = DT[kind]
    n = 1030
    rng = np.random.default_rng(9800)
    X = (np.eye(n) + 0.5 * _crandn(rng, (2, n, n), np.complex128) / np.sqrt(n)).astype(nd)
    Xw = X.astype(np.complex128)
    tol, gtol = _tols(kind, n)
    print(f"complex blocked {kind} n={n}", flush=True)
    s, l = fermix_amd.slogdet(torch.from_numpy(X).to(dev))
    sr, lr = np.linalg.slogdet(Xw)
    assert np.all(np.abs(_np(s) - sr) < tol) and np.all(np.abs(_np(l) - lr) < tol * max(1.0, np.abs(lr).max()))
    from fermix_amd import _kernels
    _, _, invT = _kernels.slogdet_parts(torch.from_numpy(X).to(dev))[:3]
    res = np.swapaxes(Xw, 1, 2) @ _np(invT).astype(np.complex128) - np.eye(n)
    print(f"  A^-T residual {np.abs(res).max():.3g}", flush=True)
    assert np.abs(res).max() < gtol
    J = np.zeros((n, n))
    J[np.arange(0, n, 2), np.arange(1, n, 2)] = 1.0
    J[np.arange(1, n, 2), np.arange(0, n, 2)] = -1.0
    S = Xw @ J @ np.swapaxes(Xw, 1, 2)
    S = (0.5 * (S - np.swapaxes(S, 1, 2))).astype(nd)
    St = torch.from_numpy(S).to(dev)
    ps, pl = fermix_amd.slogpf(St, skew_symmetrize=False)
    assert np.all(np.abs(_np(ps) - sr) < 10 * tol) and np.all(np.abs(_np(pl) - lr) < 10 * tol * max(1.0, np.abs(lr).max()))
    _, _, Sinv = _kernels.slogpf_parts(St, False)
    res = S.astype(np.complex128) @ _np(Sinv).astype(np.complex128) - np.eye(n)
    print(f"  S^-1 residual {np.abs(res).max():.3g}", flush=True)
    assert np.abs(res).max() < 10 * gtol
    Sz = St.clone()
    Sz[0, 7, :] = 0
    Sz[0, :, 7] = 0
    zs, zl = fermix_amd.slogpf(Sz, skew_symmetrize=False)
    assert _np(zs)[0] == 0 and np.isneginf(_np(zl)[0])
    assert torch.equal(zs[1], ps[1]) and torch.equal(zl[1], pl[1])


@pytest.mark.parametrize("n", [48, 130, 512])
def test_complex64_product_modes(dev, n):
    """complex64's two product modes of the blocked kernels: prec="ieee" (four fp32 MFMA
    products per complex one) and the default fp32-accuracy mode (the products on the
    fp64 MFMA, operands widened), each against complex128 numpy on X = I + N(0, 1/(4n)):
    slogdet, A^-T through its residual, pf(X J X^T) = det X and S^-1 through its residual;
    the parts calls' primal is bit-identical to the forward of the same mode. At n = 48
    (one workgroup per matrix, no blocked products) the modes give the same bits."""
    from fermix_amd import _kernels
    from fermix_amd._tune import prec_flag

    rng = np.random.default_rng(9850 + n)
    X = (np.eye(n) + 0.5 * _crandn(rng, (3, n, n), np.complex128) / np.sqrt(n)).astype(np.complex64)
    Xw = X.astype(np.complex128)
    J = np.zeros((n, n))
    J[np.arange(0, n, 2), np.arange(1, n, 2)] = 1.0
    J[np.arange(1, n, 2), np.arange(0, n, 2)] = -1.0
    S = Xw @ J @ np.swapaxes(Xw, 1, 2)
    S = (0.5 * (S - np.swapaxes(S, 1, 2))).astype(np.complex64)
    Xt, St = torch.from_numpy(X).to(dev), torch.from_numpy(S).to(dev)
    sr, lr = np.linalg.slogdet(Xw)
    tol, gtol = _tols("c64", n)
    out = {}
    for prec in ("ieee", "bf16x3"):
        x3 = prec_flag(prec)
        print(f"complex64 n={n} prec={prec}", flush=True)
        s, l = fermix_amd.slogdet(Xt, prec=prec)
        assert np.all(np.abs(_np(s) - sr) < tol) and np.all(np.abs(_np(l) - lr) < tol * max(1.0, np.abs(lr).max()))
        sp, lp, invT = _kernels.slogdet_parts(Xt, x3=x3)[:3]
        assert torch.equal(sp, s) and torch.equal(lp, l)
        res = np.swapaxes(Xw, 1, 2) @ _np(invT).astype(np.complex128) - np.eye(n)
        print(f"  A^-T residual {np.abs(res).max():.3g}", flush=True)
        assert np.abs(res).max() < gtol
        ps, pl = fermix_amd.slogpf(St, skew_symmetrize=False, prec=prec)
        assert np.all(np.abs(_np(ps) - sr) < 10 * tol)
        assert np.all(np.abs(_np(pl) - lr) < 10 * tol * max(1.0, np.abs(lr).max()))
        qs, ql, Sinv = _kernels.slogpf_parts(St, False, x3=x3)
        assert torch.equal(qs, ps) and torch.equal(ql, pl)
        res = S.astype(np.complex128) @ _np(Sinv).astype(np.complex128) - np.eye(n)
        print(f"  S^-1 residual {np.abs(res).max():.3g}", flush=True)
        assert np.abs(res).max() < 10 * gtol
        out[prec] = (_np(l), _np(invT))
    if n <= 64:
        assert np.array_equal(out["ieee"][0], out["bf16x3"][0])
        assert np.array_equal(out["ieee"][1], out["bf16x3"][1])
