"""Differentiation rules on top of the HIP kernels -- the counterpart of the reference's
custom_jvp rules (src/fermix/_diff.py:101-333) as torch.autograd.Functions with
reverse mode (backward), forward mode (jvp) and a vmap rule (all leading dimensions
fold into the kernels' batch, so vmap(f)(x) runs exactly the arithmetic of f(x)).

* slogdet: d logabs = sum(A^-T * dA), d sign = 0 (_diff.py:101-126). With a gradient
  requested, the forward runs the factorisation alone (its (sign, logabs) bit-identical
  to the plain forward: same kernel arithmetic) and keeps the packed LU; the backward
  forms g_logabs * A^-T from it in one pass. For n <= 32 one parts call forms the primal
  and A^-T together (a single Gauss-Jordan pass).
* slogpf: d logabs = -1/2 sum(S^-1 * dS) (_diff.py:129-156), likewise from the forward's
  kept Parlett-Reid factors with the cotangent applied by the inverse.
* det: d det = sum(adj(A)^T * dA) (_diff.py:270-302), with adj(A)^T from the same LU
  as the primal -- det(factors) * A^-T, or its rank-1 continuation for exact zero
  pivots -- so the gradient is finite and exact for singular A.
* pf: d pf = sum(G * dS), G = -pf(S) S^-1 / 2 (_diff.py:305-333), with the Pfaffian
  adjugate pf(S) S^-1 from the forward's own Parlett-Reid factors (finite for singular
  S); G is skew, so it is also the gradient w.r.t. ``a`` through S = (a - a^T)/2.

float64 and complex inputs, and float32 where the field-generic kernels run (the LU above
fx_tune.lu_generic_above_n, everything above 8192; no packed factors are exported
there), take the parts route (A^-T / S^-1 formed with the
primal by the field-generic blocked kernels); for complex kinds the sign is differentiable too, with
the reference's conventions (see _log_tangents below). Their det derivative is the exact
adjugate of the same Gauss-Jordan run (fx_det_parts_f64 / _c64 / _c128); their pf
derivative is the Pfaffian adjugate of fx_slogpf_parts_f64 / _c64 / _c128 (adjugate
mode), with the primal from the plain forward's own kernel. For complex kinds the
backward applies torch's conjugate convention (cotangent times the conjugate of the
holomorphic derivative), the jvp the holomorphic derivative itself.
"""

import torch

from . import _kernels, _tune
from ._kernels import DEFAULT_X3

# ----------------------------------------------------------------- helpers


def _wants_grad(A):
    """Whether a derivative of this call can be requested: autograd tracking, a
    forward-mode dual, or a torch.func grad/jvp wrapper around the input."""
    if A.requires_grad:
        return True
    try:
        import torch.autograd.forward_ad as fwAD

        if fwAD.unpack_dual(A).tangent is not None:
            return True
    except Exception:  # pragma: no cover - no dual level active
        pass
    fx = getattr(torch._C, "_functorch", None)
    if fx is not None and fx.is_functorch_wrapped_tensor(A):
        return not fx.is_batchedtensor(A)
    return False


def _plain_reverse(A):
    """A plain autograd tensor (requires_grad, no forward-mode dual, no torch.func
    wrapper): its derivative can only come from a backward pass on real tensors, so
    the factors may be kept and the inverse formed in the backward."""
    if not A.requires_grad:
        return False
    try:
        import torch.autograd.forward_ad as fwAD

        if fwAD.unpack_dual(A).tangent is not None:
            return False
    except Exception:  # pragma: no cover - no dual level active
        pass
    fx = getattr(torch._C, "_functorch", None)
    return not (fx is not None and fx.is_functorch_wrapped_tensor(A))


def _fold(info, in_dims, A):
    """vmap rule helper: move the vmapped dim first and fold it into the batch."""
    d = in_dims[0]
    if d is None:
        return A, None
    A = A.movedim(d, 0)
    V, B = A.shape[0], A.shape[1]
    return A.reshape((V * B,) + tuple(A.shape[2:])).contiguous(), (V, B)


def _unfold(x, vb):
    if vb is None:
        return x
    return x.reshape(vb + tuple(x.shape[1:]))


# complex kinds (the reference's _log_tangents, src/fermix/_diff.py:92-98): with
# t = tr(A^-1 dA) (tr(S^-1 dS) / 2 for slogpf), d logabs = Re t and d sign = i Im(t) sign --
# jnp.linalg.slogdet's convention -- and for real kinds d sign = 0. In torch's reverse
# mode (the gradient of a real loss L is the conjugate Wirtinger one, dL = Re(conj(g) dz))
# a sign cotangent g_s and a logabs cotangent g_l give g_A = (g_l - i Im(conj(g_s) sign))
# conj(M), where t = sum(M * dA).


def _keep_sign(ctx, sign, M):
    """setup_context of the parts rules: M is the gradient matrix (sum(M * dA) = t); the
    sign is differentiable for complex kinds only."""
    if sign.is_complex():
        ctx.mark_non_differentiable(M)
    else:
        ctx.mark_non_differentiable(sign, M)
    ctx.set_materialize_grads(False)  # no zero fills for the unused outputs
    ctx.save_for_backward(sign, M)
    ctx.save_for_forward(sign, M)


def _log_cotangent(sign, g_sign, g_logabs):
    """The per-member factor k with g_A = k conj(M) (real kinds: g_logabs); None if no
    cotangent reaches the derivative."""
    if not sign.is_complex():
        return g_logabs
    k = None if g_logabs is None else g_logabs.to(sign.dtype)
    if g_sign is not None:
        ks = -1j * (g_sign.conj() * sign).imag
        k = ks if k is None else k + ks
    return k


def _apply_cotangent(k, M):
    return k[:, None, None] * (M.conj() if M.is_complex() else M)


def _log_tangents(sign, t):
    """(d sign, d logabs) from t: None and t for real kinds."""
    if not sign.is_complex():
        return None, t
    return 1j * t.imag * sign, t.real


# ----------------------------------------------------------------- slogdet


class _SlogdetFwd(torch.autograd.Function):
    """Forward only (no derivative requested)."""

    @staticmethod
    def forward(A, x3):
        return _kernels.slogdet(A, x3)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.mark_non_differentiable(*output)

    @staticmethod
    def vmap(info, in_dims, A, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        s, l = _SlogdetFwd.apply(A2, x3)
        if vb is None:
            return (s, l), (None, None)
        return (_unfold(s, vb), _unfold(l, vb)), (0, 0)


class _SlogdetParts(torch.autograd.Function):
    """(sign, logabs, invT) from one factorisation; d logabs = sum(invT * dA)."""

    @staticmethod
    def forward(A, x3):
        sign, logabs, invT, _, _ = _kernels.slogdet_parts(A, x3=x3)
        return sign, logabs, invT

    @staticmethod
    def setup_context(ctx, inputs, output):
        sign, logabs, invT = output
        _keep_sign(ctx, sign, invT)

    @staticmethod
    def backward(ctx, g_sign, g_logabs, g_invT):
        sign, invT = ctx.saved_tensors
        k = _log_cotangent(sign, g_sign, g_logabs)
        if k is None:
            return None, None
        return _apply_cotangent(k, invT), None

    @staticmethod
    def jvp(ctx, dA, _x3):
        sign, invT = ctx.saved_tensors
        ds, dlog = _log_tangents(sign, (invT * dA).sum(dim=(-1, -2)))
        return ds, dlog, None

    @staticmethod
    def vmap(info, in_dims, A, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        s, l, inv = _SlogdetParts.apply(A2, x3)
        if vb is None:
            return (s, l, inv), (None, None, None)
        return (_unfold(s, vb), _unfold(l, vb), _unfold(inv, vb)), (0, 0, 0)


class _SlogdetSplit(torch.autograd.Function):
    """(sign, logabs) with the factors (lu, perm) kept for the derivative: the backward
    forms g_logabs * A^-T in one pass from them (the cotangent is the inverse kernel's
    per-member scale, so no separate product over B n^2). Used for plain reverse mode;
    the jvp (real tensors only) forms A^-T from a copy of lu.
    The backward overwrites lu (the inverse's scratch); a second backward of the same
    graph refactors the saved input."""

    @staticmethod
    def forward(A, x3):
        return _kernels.slogdet_factors(A, x3)

    @staticmethod
    def setup_context(ctx, inputs, output):
        sign, logabs, lu, perm = output
        ctx.mark_non_differentiable(sign, lu, perm)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(inputs[0], sign, lu, perm)
        ctx.save_for_forward(sign, lu, perm)
        ctx.n = inputs[0].shape[-1]
        ctx.x3 = inputs[1]
        ctx.lu_used = False

    @staticmethod
    def backward(ctx, g_sign, g_logabs, g_lu, g_perm):
        A, sign, lu, perm = ctx.saved_tensors
        if g_logabs is None:
            return None, None
        if ctx.lu_used:  # retained graph, second backward: lu was overwritten
            sign, _, lu, perm = _kernels.slogdet_factors(A.detach(), ctx.x3)
        ctx.lu_used = True
        return _kernels.slogdet_inverse(lu, perm, sign, ctx.n, scale=g_logabs, x3=ctx.x3), None

    @staticmethod
    def jvp(ctx, dA, _x3):
        sign, lu, perm = ctx.saved_tensors
        invT = _kernels.slogdet_inverse(lu.clone(), perm, sign, ctx.n, x3=ctx.x3)
        dlog = (invT * dA).sum(dim=(-1, -2))
        return None, dlog, None, None

    @staticmethod
    def vmap(info, in_dims, A, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        out = _SlogdetSplit.apply(A2, x3)
        if vb is None:
            return out, (None,) * 4
        return tuple(_unfold(x, vb) for x in out), (0,) * 4


def slogdet(A, x3=DEFAULT_X3):
    """x3: the split-bf16x3 product mode of the blocked kernels (0: fp32 MFMA)."""
    if _wants_grad(A):
        # n <= 32: one Gauss-Jordan pass forms A^-T with the factors; forward mode and
        # torch.func transforms: the parts call (their rules run on wrapped tensors)
        if (A.dtype == torch.float32 and 32 < A.shape[-1] <= _tune.LARGE_MAX_N and _plain_reverse(A)
                and _tune.kernel_family(A.shape[-1], "slogdet") != "generic"):
            s, l, _, _ = _SlogdetSplit.apply(A, x3)
        else:
            s, l, _ = _SlogdetParts.apply(A, x3)
        return s, l
    return _SlogdetFwd.apply(A, x3)


# ----------------------------------------------------------------- slogpf


class _SlogpfFwd(torch.autograd.Function):
    @staticmethod
    def forward(A, skew, x3):
        return _kernels.slogpf(A, skew, x3=x3)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.mark_non_differentiable(*output)

    @staticmethod
    def vmap(info, in_dims, A, skew, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        s, l = _SlogpfFwd.apply(A2, skew, x3)
        if vb is None:
            return (s, l), (None, None)
        return (_unfold(s, vb), _unfold(l, vb)), (0, 0)


class _SlogpfParts(torch.autograd.Function):
    """(sign, logabs, Sinv); d logabs = -1/2 sum(Sinv * dS), which is also the
    derivative w.r.t. ``a`` through S = (a - a^T)/2 (Sinv is skew)."""

    @staticmethod
    def forward(A, skew, x3):
        return _kernels.slogpf_parts(A, skew, x3=x3)

    @staticmethod
    def setup_context(ctx, inputs, output):
        sign, logabs, Sinv = output
        _keep_sign(ctx, sign, Sinv)

    @staticmethod
    def backward(ctx, g_sign, g_logabs, g_sinv):
        sign, Sinv = ctx.saved_tensors
        k = _log_cotangent(sign, g_sign, g_logabs)
        if k is None:
            return None, None, None
        return _apply_cotangent(-0.5 * k, Sinv), None, None

    @staticmethod
    def jvp(ctx, dA, _skew, _x3):
        sign, Sinv = ctx.saved_tensors
        ds, dlog = _log_tangents(sign, -0.5 * (Sinv * dA).sum(dim=(-1, -2)))
        return ds, dlog, None

    @staticmethod
    def vmap(info, in_dims, A, skew, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        s, l, inv = _SlogpfParts.apply(A2, skew, x3)
        if vb is None:
            return (s, l, inv), (None, None, None)
        return (_unfold(s, vb), _unfold(l, vb), _unfold(inv, vb)), (0, 0, 0)


class _SlogpfSplit(torch.autograd.Function):
    """(sign, logabs) with the Parlett-Reid factors kept for the derivative: the backward
    forms (-g_logabs / 2) S^-1 in one pass from them (the scale applied in the inverse's
    final gather). Used for plain reverse mode; the jvp (real tensors only) forms S^-1.
    The factors are only read."""

    @staticmethod
    def forward(A, skew, x3):
        return _kernels.slogpf_factors(A, skew)

    @staticmethod
    def setup_context(ctx, inputs, output):
        sign, logabs, gbuf, d, perm = output
        ctx.mark_non_differentiable(sign, gbuf, d, perm)
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(gbuf, d, perm)
        ctx.save_for_forward(gbuf, d, perm)
        ctx.n = inputs[0].shape[-1]
        ctx.x3 = inputs[2]

    @staticmethod
    def backward(ctx, g_sign, g_logabs, g_gbuf, g_d, g_perm):
        gbuf, d, perm = ctx.saved_tensors
        if g_logabs is None:
            return None, None, None
        return _kernels.slogpf_inverse(gbuf, d, perm, ctx.n, scale=-0.5 * g_logabs, x3=ctx.x3), None, None

    @staticmethod
    def jvp(ctx, dA, _skew, _x3):
        gbuf, d, perm = ctx.saved_tensors
        Sinv = _kernels.slogpf_inverse(gbuf, d, perm, ctx.n, x3=ctx.x3)
        dlog = -0.5 * (Sinv * dA).sum(dim=(-1, -2))
        return None, dlog, None, None, None

    @staticmethod
    def vmap(info, in_dims, A, skew, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        out = _SlogpfSplit.apply(A2, skew, x3)
        if vb is None:
            return out, (None,) * 5
        return tuple(_unfold(x, vb) for x in out), (0,) * 5


def slogpf(A, skew, x3=DEFAULT_X3):
    """x3: the split-bf16x3 product mode of the gradient's GEMMs (the forward's trailing
    update is memory-bound and runs in fp32 in both modes)."""
    if _wants_grad(A):
        n = A.shape[-1]
        if (A.dtype == torch.float32 and 0 < n <= _tune.LARGE_MAX_N and n % 2 == 0 and _plain_reverse(A)
                and _tune.kernel_family(n, "slogpf") != "generic"):
            s, l, _, _, _ = _SlogpfSplit.apply(A, skew, x3)
        else:
            s, l, _ = _SlogpfParts.apply(A, skew, x3)
        return s, l
    return _SlogpfFwd.apply(A, skew, x3)


# ----------------------------------------------------------------- det / pf


class _DetParts(torch.autograd.Function):
    """(det, adjT) from one factorisation; d det = sum(adjT * dA)."""

    @staticmethod
    def forward(A, x3):
        sign, logabs, adjT = _kernels.det_parts(A, x3)
        return sign * torch.exp(logabs), adjT

    @staticmethod
    def setup_context(ctx, inputs, output):
        _, adjT = output
        ctx.mark_non_differentiable(adjT)
        ctx.set_materialize_grads(False)  # no zero fills for the unused outputs
        ctx.save_for_backward(adjT)
        ctx.save_for_forward(adjT)

    @staticmethod
    def backward(ctx, g_det, g_adj):
        (adjT,) = ctx.saved_tensors
        if g_det is None:
            return None, None
        # det is holomorphic: with dL = Re(conj(g) d det), the conjugate-Wirtinger
        # gradient is g conj(adj(A)^T) (adj(A)^T itself for real kinds)
        return _apply_cotangent(g_det, adjT), None

    @staticmethod
    def jvp(ctx, dA, _x3):
        (adjT,) = ctx.saved_tensors
        return (adjT * dA).sum(dim=(-1, -2)), None

    @staticmethod
    def vmap(info, in_dims, A, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        d, adj = _DetParts.apply(A2, x3)
        if vb is None:
            return (d, adj), (None, None)
        return (_unfold(d, vb), _unfold(adj, vb)), (0, 0)


def det(A, x3=DEFAULT_X3):
    if _wants_grad(A):
        d, _ = _DetParts.apply(A, x3)
        return d
    s, l = _SlogdetFwd.apply(A, x3)
    return s * torch.exp(l)


class _PfParts(torch.autograd.Function):
    """(pf, G) with G = -pf(S) S^-1 / 2 from one Parlett-Reid run; d pf = sum(G * dS)."""

    @staticmethod
    def forward(A, skew, x3):
        sign, logabs, adj = _kernels.slogpf_parts(A, skew, adjugate=True, x3=x3)
        return sign * torch.exp(logabs), -0.5 * adj

    @staticmethod
    def setup_context(ctx, inputs, output):
        _, G = output
        ctx.mark_non_differentiable(G)
        ctx.set_materialize_grads(False)  # no zero fills for the unused outputs
        ctx.save_for_backward(G)
        ctx.save_for_forward(G)

    @staticmethod
    def backward(ctx, g_pf, g_G):
        (G,) = ctx.saved_tensors
        if g_pf is None:
            return None, None, None
        return _apply_cotangent(g_pf, G), None, None

    @staticmethod
    def jvp(ctx, dA, _skew, _x3):
        (G,) = ctx.saved_tensors
        return (G * dA).sum(dim=(-1, -2)), None

    @staticmethod
    def vmap(info, in_dims, A, skew, x3):
        A2, vb = _fold(info, in_dims[:1], A)
        p, G = _PfParts.apply(A2, skew, x3)
        if vb is None:
            return (p, G), (None, None)
        return (_unfold(p, vb), _unfold(G, vb)), (0, 0)


def pf(A, skew, x3=DEFAULT_X3):
    if _wants_grad(A):
        p, _ = _PfParts.apply(A, skew, x3)
        return p
    s, l = _SlogpfFwd.apply(A, skew, x3)
    return s * torch.exp(l)


# ------------------------------------------------------------------- odd n


class _OddConst(torch.autograd.Function):
    """Odd n: the reference's constant branch (api.py:122-123, 141-142) -- pf = 0, slogpf
    (0, -inf) -- as a function of the input with a zero derivative, so that reverse mode,
    forward mode and vmap see what the reference's constant differentiates to."""

    generate_vmap_rule = True

    @staticmethod
    def forward(A, what):
        B = A.shape[0]
        zero = torch.zeros(B, dtype=A.dtype, device=A.device)
        if what == "pf":
            return zero
        real = A.real.dtype if A.is_complex() else A.dtype
        return zero, torch.full((B,), -float("inf"), dtype=real, device=A.device)

    @staticmethod
    def setup_context(ctx, inputs, output):
        A, what = inputs
        ctx.what = what
        ctx.set_materialize_grads(False)
        ctx.meta = (A.shape, A.dtype, A.device)

    @staticmethod
    def backward(ctx, *grads):
        shape, dtype, device = ctx.meta
        return torch.zeros(shape, dtype=dtype, device=device), None

    @staticmethod
    def jvp(ctx, dA, _what):
        B = dA.shape[0]
        zero = torch.zeros(B, dtype=dA.dtype, device=dA.device)
        if ctx.what == "pf":
            return zero
        real = dA.real.dtype if dA.is_complex() else dA.dtype
        return zero, torch.zeros(B, dtype=real, device=dA.device)


def odd_pf(A):
    return _OddConst.apply(A, "pf")


def odd_slogpf(A):
    return _OddConst.apply(A, "slogpf")
