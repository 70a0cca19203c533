"""Public API of fermix_amd: ``slogdet``, ``slogpf``, ``det``, ``pf`` -- the interface of
ChenAo-Phys/fermix (src/fermix/api.py:148-227) on torch tensors, with the kernels
underneath replaced by hand-written HIP kernels for gfx950 (``libfermix_amd.so``).

Conventions kept from the reference:
* input (..., n, n); every leading dimension is a batch dimension (api.py:100-103);
* slogdet returns (sign, logabs) with sign exactly +-1 / 0 and logabs -inf for an
  exactly zero pivot, the jnp.linalg.slogdet convention (_fallback.py:6-9);
* slogpf skew-symmetrises its input as (a - a^T)/2 unless skew_symmetrize=False, and
  odd n gives (0, -inf) (api.py:122-125); pf of odd n is 0;
* unsupported dtype -> TypeError, bad shape / block / prec -> ValueError
  (api.py:24-31,92-97; _field.py:265-275);
* differentiable (torch.autograd, forward mode, torch.func.vmap / grad / jvp) with the
  reference's rules (_diff.py:101-333): d logabs = tr(A^-1 dA), d sign = 0; slogpf
  d logabs = tr(S^-1 dS)/2 (gradient w.r.t. ``a`` S^-T/2 through the
  skew-symmetrisation); exactly singular inputs get a zero (finite) slogdet / slogpf
  gradient; det and pf differentiate through the adjugates, d det = tr(adj(A) dA) and
  d pf = tr(pf(S) S^-1 dS)/2, finite and exact for singular inputs; the primal of a
  differentiated call is bit-identical to the plain forward.

dtypes: float32, float64, complex64 and complex128 (the reference's four kinds); for
complex inputs sign is a unit complex number (prod(d / |d|) times the parity) and
logabs real, and the derivatives follow jnp.linalg's convention (d logabs = Re t,
d sign = i Im(t) sign with t = tr(A^-1 dA)); torch's reverse mode then gives the
gradient of logabs as conj(A^-T).

Device handling: the product path is the HIP library on a ROCm GPU. A CPU tensor
raises ``FermixDeviceError`` (the reference's generic XLA fallback is not part of this
build) -- there is no silent CPU path.
"""

import torch

from . import _diff
from ._tune import FermixTuneWarning, block_flag, check_block, check_prec, note_ignored, prec_flag

_FLOAT_KINDS = (torch.float32, torch.float64, torch.complex64, torch.complex128)


class FermixFallbackWarning(UserWarning):
    """Kept for API compatibility with the reference (api.py:19-21). fermix_amd never
    falls back silently; see FermixDeviceError."""


class FermixDeviceError(RuntimeError):
    """The input is not on a ROCm GPU; fermix_amd runs only its HIP kernels."""


def _prep(a):
    if not isinstance(a, torch.Tensor):
        raise TypeError(f"fermix_amd expects a torch.Tensor, got {type(a).__name__}")
    if a.dtype not in _FLOAT_KINDS:
        raise TypeError(
            f"fermix supports float32, float64, complex64 and complex128, got {a.dtype}"
        )
    if a.dim() < 2 or a.shape[-1] != a.shape[-2]:
        raise ValueError(f"expected (..., n, n), got {tuple(a.shape)}")
    return a


def _on_device(a):
    if not a.is_cuda:
        raise FermixDeviceError(
            "fermix_amd runs on a ROCm GPU only (the reference's generic CPU fallback is "
            "not part of this build); move the input to a 'cuda' device"
        )


def _flat(a):
    batch = a.shape[:-2]
    n = a.shape[-1]
    B = 1
    for d in batch:
        B *= int(d)
    return a.reshape((B, n, n)).contiguous(), batch, n


def _lu_opts(a, prec, unroll_steps, block):
    """The C ABI's prec word of a slogdet / det call: the product mode and, for float32,
    the LU block option."""
    x3 = prec_flag(check_prec(prec, a.dtype))
    check_block(block)
    note_ignored("unroll_steps", unroll_steps)
    return x3 | (block_flag(block) if a.dtype == torch.float32 else 0)


def slogdet(a, *, prec=None, unroll_steps=None, block=None):
    """Sign and log|det| of a batch of matrices ``a`` (..., n, n) (reference
    ``slogdet``, api.py:148-174). prec: "bf16x3" (the float32 / complex64 default: three-way
    bf16 split, six bf16 MFMA products, fp32 accumulation, fp32 accuracy), "tf32x3" (the
    reference's name for its default fp32-accuracy three-pass mode; on gfx950, which has
    no TF32 type, it selects "bf16x3") or "ieee" (fp32 MFMA products; the only mode, and
    the default, of float64 / complex128). The mode applies to the blocked kernels
    (n > 128): the trailing updates and the inverse's GEMMs. block: the outer LU block of the blocked kernels
    (float32): None (the tuning table: block pairs above N = 256), 64 (single 64-column
    blocks, K = 64 trailing updates) or 128 (blocks in pairs, K = 128 updates); 32 runs
    64 with a FermixTuneWarning. unroll_steps: accepted, without effect on gfx950 (the
    panels are always unrolled), with a FermixTuneWarning when given."""
    a = _prep(a)
    x3 = _lu_opts(a, prec, unroll_steps, block)
    _on_device(a)
    A, batch, n = _flat(a)
    sign, logabs = _diff.slogdet(A, x3)
    return sign.reshape(batch), logabs.reshape(batch)


def slogpf(a, *, prec=None, skew_symmetrize=True, upd_warps=None):
    """Sign and log|pf| of a batch of skew-symmetric matrices (reference ``slogpf``,
    api.py:177-193): S = (a - a^T)/2 unless skew_symmetrize=False (then ``a`` must be
    exactly skew); odd n gives (0, -inf). prec as for slogdet; it applies to the
    gradient's GEMMs (the forward's trailing update is memory-bound and runs in fp32).
    upd_warps: accepted, without effect on gfx950 (the trailing update's shape is fixed;
    its blocking follows the tuning table, fermix_amd._tune), with a FermixTuneWarning
    when given."""
    a = _prep(a)
    x3 = prec_flag(check_prec(prec, a.dtype))
    note_ignored("upd_warps", upd_warps)
    _on_device(a)
    A, batch, n = _flat(a)
    if n % 2 == 1:
        sign, logabs = _diff.odd_slogpf(A)
        return sign.reshape(batch), logabs.reshape(batch)
    sign, logabs = _diff.slogpf(A, bool(skew_symmetrize), x3)
    return sign.reshape(batch), logabs.reshape(batch)


def det(a, *, prec=None, unroll_steps=None, block=None):
    """Determinant of a batch of matrices (reference ``det``, api.py:196-212):
    sign * exp(logabs) of the same factorisation. Options as for slogdet."""
    a = _prep(a)
    x3 = _lu_opts(a, prec, unroll_steps, block)
    _on_device(a)
    A, batch, n = _flat(a)
    return _diff.det(A, x3).reshape(batch)


def pf(a, *, prec=None, skew_symmetrize=True, upd_warps=None):
    """Pfaffian of a batch of skew-symmetric matrices (reference ``pf``, api.py:215-227);
    odd n gives 0. Options as for slogpf."""
    a = _prep(a)
    x3 = prec_flag(check_prec(prec, a.dtype))
    note_ignored("upd_warps", upd_warps)
    _on_device(a)
    A, batch, n = _flat(a)
    if n % 2 == 1:
        return _diff.odd_pf(A).reshape(batch)
    return _diff.pf(A, bool(skew_symmetrize), x3).reshape(batch)


__all__ = [
    "slogdet",
    "slogpf",
    "det",
    "pf",
    "FermixFallbackWarning",
    "FermixDeviceError",
    "FermixTuneWarning",
]
