"""Torch plumbing around the C ABI: allocate outputs / workspace on the input's device,
pass raw pointers and the current HIP stream. Inputs are (B, n, n) contiguous float32
tensors (float64 for the f64 entry points) on a ROCm device; no numerics happen here."""

import torch

from ._lib import FX_PREC_BF16X3, FX_PREC_IEEE, FX_PREC_MASK, check, lib
from ._tune import DEFAULT_PREC, prec_flag

# the C ABI's prec word of the library's default product mode (the public API's default
# for float32); the float64 and complex entry points take no prec
DEFAULT_X3 = prec_flag(DEFAULT_PREC)


def _stream(t):
    return ctypes_ptr(torch.cuda.current_stream(t.device).cuda_stream)


def ctypes_ptr(x):
    return int(x) if x else None


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _workspace(nbytes, device):
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


_CPLX = {torch.complex64: "c64", torch.complex128: "c128"}


def _check_input(A, f64_ok=False):
    """Returns True for a float64 input (the f64 entry points), False for float32."""
    if not A.is_cuda:
        raise RuntimeError("fermix_amd kernels need a tensor on a ROCm GPU")
    ok = (torch.float32, torch.float64) if f64_ok else (torch.float32,)
    if A.dtype not in ok or A.dim() != 3 or not A.is_contiguous():
        raise RuntimeError(f"internal: expected a contiguous (B, n, n) tensor of {ok}")
    return A.dtype == torch.float64


def _real_dtype(dt):
    return torch.float32 if dt == torch.complex64 else torch.float64


def _cplx_input(A):
    """The kind suffix ("c64" / "c128") of a complex input, else None."""
    k = _CPLX.get(A.dtype)
    if k is None:
        return None
    if not A.is_cuda:
        raise RuntimeError("fermix_amd kernels need a tensor on a ROCm GPU")
    if A.dim() != 3 or not A.is_contiguous():
        raise RuntimeError("internal: expected a contiguous (B, n, n) complex tensor")
    return k


def _cplx_prec(x3):
    """complex64's prec argument: the fp32-accuracy mode (products on the fp64 MFMA) for a
    bf16x3 word, fp32 MFMA products for an IEEE one."""
    return FX_PREC_BF16X3 if int(x3) & FX_PREC_MASK else FX_PREC_IEEE


def _cplx_call(A, name, skew=None, want_out=False, adjugate=False, x3=DEFAULT_X3):
    """complex64 / complex128: (sign, logabs[, out]) from fx_<name>_<kind>; sign complex
    (B,), logabs real (B,), out (B, n, n) complex (A^-T for slogdet_parts, S^-1 for
    slogpf_parts). complex64 passes its prec (from the C ABI's prec word x3)."""
    k = _cplx_input(A)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=_real_dtype(A.dtype), device=dev)
    out = torch.empty_like(A) if want_out else None
    L = lib()
    fn = f"fx_{name}_{k}"
    ws, wsb = _workspace(getattr(L, fn + "_workspace")(B, n), dev)
    args = [_ptr(A), B, n]
    if skew is not None:
        args.append(int(bool(skew)))
    if name == "slogpf_parts":
        args.append(int(bool(adjugate)))
    args += [_ptr(sign), _ptr(logabs)]
    if name.endswith("_parts"):
        args.append(_ptr(out))
    if k == "c64":
        args.append(_cplx_prec(x3))
    args += [_ptr(ws), wsb, _stream(A)]
    check(getattr(L, fn)(*args), fn)
    return (sign, logabs, out) if name.endswith("_parts") else (sign, logabs)


def _aligned(A):
    """A itself when its data is 16-byte aligned (the C ABI's contract), else an aligned
    copy: a view into a batch at an odd member offset of an odd-n batch is not."""
    return A if A.data_ptr() % 16 == 0 else A.clone()


def _no_f64(A, what):
    if A.dtype != torch.float32:
        raise NotImplementedError(
            f"fermix_amd: {what} is implemented for float32 only (float64 / complex64 / "
            "complex128 have the values and every derivative, formed by their own kernels)"
        )


def lu_padded_size(n):
    return int(lib().fx_lu_padded_size(n))


def pf_padded_size(n):
    return int(lib().fx_pf_padded_size(n))


def slogdet(A, x3=DEFAULT_X3):
    """(sign, logabs) of each (n, n) matrix of A (B, n, n); x3: the C ABI's prec word
    (FX_PREC_BF16X3 products, FX_LU_BLOCK_* options; float32 only)."""
    if A.is_complex():
        return _cplx_call(A, "slogdet", x3=x3)
    f64 = _check_input(A, f64_ok=True)
    A = _aligned(A)
    B, n, _ = A.shape
    sign = torch.empty(B, dtype=A.dtype, device=A.device)
    logabs = torch.empty(B, dtype=A.dtype, device=A.device)
    L = lib()
    if f64:
        ws, wsb = _workspace(L.fx_slogdet_f64_workspace(B, n), A.device)
        st = L.fx_slogdet_f64(_ptr(A), B, n, _ptr(sign), _ptr(logabs), _ptr(ws), wsb, _stream(A))
        check(st, "fx_slogdet_f64")
        return sign, logabs
    ws, wsb = _workspace(L.fx_slogdet_f32_workspace(B, n), A.device)
    st = L.fx_slogdet_f32(_ptr(A), B, n, _ptr(sign), _ptr(logabs), int(x3), _ptr(ws), wsb, _stream(A))
    check(st, "fx_slogdet_f32")
    return sign, logabs


def slogdet_parts(A, zero_singular=True, want_inv=True, want_lu=False, x3=DEFAULT_X3):
    """(sign, logabs, invT, lu, perm) with the optional outputs None when not asked for;
    lu / perm are padded to N = lu_padded_size(n). float64 and complex: invT only (zero
    for exactly singular members), no packed factors."""
    if A.is_complex():
        if want_lu or not zero_singular:
            _no_f64(A, "the packed LU / unguarded inverse")
        sign, logabs, invT = _cplx_call(A, "slogdet_parts", want_out=want_inv, x3=x3)
        return sign, logabs, invT, None, None
    f64 = _check_input(A, f64_ok=True)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=A.dtype, device=dev)
    invT = torch.empty_like(A) if want_inv else None
    if f64:
        if want_lu or not zero_singular:
            _no_f64(A, "the packed LU / unguarded inverse")
        L = lib()
        ws, wsb = _workspace(L.fx_slogdet_parts_f64_workspace(B, n), dev)
        st = L.fx_slogdet_parts_f64(
            _ptr(A), B, n, _ptr(sign), _ptr(logabs), _ptr(invT), _ptr(ws), wsb, _stream(A)
        )
        check(st, "fx_slogdet_parts_f64")
        return sign, logabs, invT, None, None
    lu = perm = None
    if want_lu and n > 0:
        N = lu_padded_size(n)
        lu = torch.empty((B, N, N), dtype=A.dtype, device=dev)
        perm = torch.empty((B, N), dtype=torch.int32, device=dev)
    L = lib()
    ws, wsb = _workspace(L.fx_slogdet_parts_f32_workspace(B, n), dev)
    st = L.fx_slogdet_parts_f32(
        _ptr(A), B, n, int(bool(zero_singular)), _ptr(sign), _ptr(logabs), _ptr(invT),
        _ptr(lu), _ptr(perm), int(x3), _ptr(ws), wsb, _stream(A),
    )
    check(st, "fx_slogdet_parts_f32")
    return sign, logabs, invT, lu, perm


def slogdet_factors(A, x3=DEFAULT_X3):
    """(sign, logabs, lu (B, N, N), perm (B, N)): the packed LU of fx_slogdet_parts_f32
    alone, N = lu_padded_size(n)."""
    _check_input(A)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    N = lu_padded_size(n) if n > 0 else 0
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=A.dtype, device=dev)
    lu = torch.empty((B, N, N), dtype=A.dtype, device=dev)
    perm = torch.empty((B, N), dtype=torch.int32, device=dev)
    L = lib()
    ws, wsb = _workspace(L.fx_slogdet_factors_f32_workspace(B, n), dev)
    st = L.fx_slogdet_factors_f32(
        _ptr(A), B, n, _ptr(sign), _ptr(logabs), _ptr(lu), _ptr(perm), int(x3), _ptr(ws), wsb, _stream(A)
    )
    check(st, "fx_slogdet_factors_f32")
    return sign, logabs, lu, perm


def slogdet_inverse(lu, perm, sign, n, scale=None, zero_singular=True, x3=DEFAULT_X3):
    """scale[b] * A^-T (B, n, n) from slogdet_factors' outputs; lu is overwritten."""
    B = sign.shape[0]
    dev = sign.device
    out = torch.empty((B, n, n), dtype=sign.dtype, device=dev)
    if scale is not None:
        scale = scale.to(dtype=sign.dtype).contiguous()
    L = lib()
    ws, wsb = _workspace(L.fx_slogdet_inverse_f32_workspace(B, n), dev)
    st = L.fx_slogdet_inverse_f32(
        _ptr(lu), _ptr(perm), _ptr(sign), _ptr(scale), B, n, int(bool(zero_singular)), _ptr(out),
        int(x3) & FX_PREC_MASK, _ptr(ws), wsb, _stream(sign),
    )
    check(st, "fx_slogdet_inverse_f32")
    return out


def det_parts(A, x3=DEFAULT_X3):
    """(sign, logabs, adjT) with adjT = adj(A)^T = d det / dA from one factorisation
    (holomorphic, no conjugation, for complex A)."""
    if A.dtype != torch.float32:
        k = {torch.float64: "f64", torch.complex64: "c64", torch.complex128: "c128"}[A.dtype]
        if not A.is_cuda:
            raise RuntimeError("fermix_amd kernels need a tensor on a ROCm GPU")
        A = _aligned(A.contiguous())
        B, n, _ = A.shape
        dev = A.device
        sign = torch.empty(B, dtype=A.dtype, device=dev)
        logabs = torch.empty(B, dtype=_real_dtype(A.dtype) if A.is_complex() else A.dtype, device=dev)
        adjT = torch.empty_like(A)
        L = lib()
        ws, wsb = _workspace(getattr(L, f"fx_det_parts_{k}_workspace")(B, n), dev)
        prec = [_cplx_prec(x3)] if k == "c64" else []
        st = getattr(L, f"fx_det_parts_{k}")(
            _ptr(A), B, n, _ptr(sign), _ptr(logabs), _ptr(adjT), *prec, _ptr(ws), wsb, _stream(A)
        )
        check(st, f"fx_det_parts_{k}")
        return sign, logabs, adjT
    _check_input(A)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=A.dtype, device=dev)
    adjT = torch.empty_like(A)
    L = lib()
    ws, wsb = _workspace(L.fx_det_parts_f32_workspace(B, n), dev)
    st = L.fx_det_parts_f32(
        _ptr(A), B, n, _ptr(sign), _ptr(logabs), _ptr(adjT), int(x3), _ptr(ws), wsb, _stream(A)
    )
    check(st, "fx_det_parts_f32")
    return sign, logabs, adjT


def slogpf(A, skew_symmetrize, x3=DEFAULT_X3):
    """(sign, logabs) of pf; x3 reaches only complex64 (the float32 forward's Parlett-Reid
    update has no product mode)."""
    if A.is_complex():
        return _cplx_call(A, "slogpf", skew=skew_symmetrize, x3=x3)
    f64 = _check_input(A, f64_ok=True)
    A = _aligned(A)
    B, n, _ = A.shape
    sign = torch.empty(B, dtype=A.dtype, device=A.device)
    logabs = torch.empty(B, dtype=A.dtype, device=A.device)
    L = lib()
    if f64:
        ws, wsb = _workspace(L.fx_slogpf_f64_workspace(B, n), A.device)
        st = L.fx_slogpf_f64(
            _ptr(A), B, n, int(bool(skew_symmetrize)), _ptr(sign), _ptr(logabs), _ptr(ws), wsb,
            _stream(A),
        )
        check(st, "fx_slogpf_f64")
        return sign, logabs
    ws, wsb = _workspace(L.fx_slogpf_f32_workspace(B, n), A.device)
    st = L.fx_slogpf_f32(
        _ptr(A), B, n, int(bool(skew_symmetrize)), _ptr(sign), _ptr(logabs), _ptr(ws), wsb,
        _stream(A),
    )
    check(st, "fx_slogpf_f32")
    return sign, logabs


def slogpf_factors(A, skew_symmetrize):
    """(sign, logabs, gbuf (B, N/PB, N, PB), d (B, N/2), perm (B, N))."""
    _check_input(A)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    L = lib()
    N = pf_padded_size(n)
    PB = int(L.fx_pf_block_columns(n))
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=A.dtype, device=dev)
    gbuf = torch.empty((B, N // PB, N, PB), dtype=A.dtype, device=dev)  # unspecified entries stay unset
    d = torch.empty((B, N // 2), dtype=A.dtype, device=dev)
    perm = torch.empty((B, N), dtype=torch.int32, device=dev)
    ws, wsb = _workspace(L.fx_slogpf_factors_f32_workspace(B, n), dev)
    st = L.fx_slogpf_factors_f32(
        _ptr(A), B, n, int(bool(skew_symmetrize)), _ptr(sign), _ptr(logabs), _ptr(gbuf),
        _ptr(d), _ptr(perm), _ptr(ws), wsb, _stream(A),
    )
    check(st, "fx_slogpf_factors_f32")
    return sign, logabs, gbuf, d, perm


def slogpf_inverse(gbuf, d, perm, n, scale=None, adjugate=False, x3=DEFAULT_X3):
    """scale[b] * S^-1 (or scale[b] * pf(S) S^-1) (B, n, n) from slogpf_factors' outputs,
    which are read only."""
    B = d.shape[0]
    dev = d.device
    out = torch.empty((B, n, n), dtype=d.dtype, device=dev)
    if scale is not None:
        scale = scale.to(dtype=d.dtype).contiguous()
    L = lib()
    ws, wsb = _workspace(L.fx_slogpf_inverse_f32_workspace(B, n), dev)
    st = L.fx_slogpf_inverse_f32(
        _ptr(gbuf), _ptr(d), _ptr(perm), _ptr(scale), B, n, int(bool(adjugate)), _ptr(out),
        int(x3), _ptr(ws), wsb, _stream(d),
    )
    check(st, "fx_slogpf_inverse_f32")
    return out


def slogpf_parts(A, skew_symmetrize, adjugate=False, x3=DEFAULT_X3):
    """(sign, logabs, G) of the (skew-symmetrised) batch from one Parlett-Reid run, G = S^-1
    or, with adjugate, pf(S) S^-1 (the Pfaffian adjugate)."""
    if A.is_complex():
        return _cplx_call(A, "slogpf_parts", skew=skew_symmetrize, want_out=True, adjugate=adjugate, x3=x3)
    f64 = _check_input(A, f64_ok=True)
    A = _aligned(A)
    B, n, _ = A.shape
    dev = A.device
    L = lib()
    sign = torch.empty(B, dtype=A.dtype, device=dev)
    logabs = torch.empty(B, dtype=A.dtype, device=dev)
    g = torch.empty_like(A)
    if f64:
        ws, wsb = _workspace(L.fx_slogpf_parts_f64_workspace(B, n), dev)
        st = L.fx_slogpf_parts_f64(
            _ptr(A), B, n, int(bool(skew_symmetrize)), int(bool(adjugate)), _ptr(sign), _ptr(logabs), _ptr(g),
            _ptr(ws), wsb, _stream(A),
        )
        check(st, "fx_slogpf_parts_f64")
        return sign, logabs, g
    ws, wsb = _workspace(L.fx_slogpf_parts_f32_workspace(B, n), dev)
    st = L.fx_slogpf_parts_f32(
        _ptr(A), B, n, int(bool(skew_symmetrize)), int(bool(adjugate)), _ptr(sign), _ptr(logabs), _ptr(g),
        int(x3), _ptr(ws), wsb, _stream(A),
    )
    check(st, "fx_slogpf_parts_f32")
    return sign, logabs, g
