"""ctypes binding of the in-tree HIP library ``libfermix_amd.so`` (C ABI declared in
``include/fermix.h``). The product path has no fallback: if the library is missing the
calls raise ``FermixLibraryError``."""

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfermix_amd.so")

FX_OK = 0

# the prec argument (include/fermix.h): the product mode and, for the float32 slogdet /
# det entry points, option bits
FX_PREC_IEEE = 0
FX_PREC_BF16X3 = 1
FX_PREC_MASK = 0x0F
FX_LU_BLOCK_64 = 0x100
FX_LU_BLOCK_128 = 0x200

# fields of struct fx_tune, in order (int32 each; 3 reserved int32 follow)
TUNE_FIELDS = (
    "fused_max_n",
    "lu_pair_above_n",
    "lu_direct_max_n",
    "pf_block64_min_n",
    "pf_block64_max_m",
    "gemm128_min_mn",
    "gemm128_min_k",
    "gemm128_tout",
    "gemm128_x3_min_mn",
    "gemm128_x3_min_k",
    "gemm128_x3_tout",
    "f64_reg_max_n",
    "f64_strip16_max_n",
    "pf_overlap_max_half",
    "pf_overlap_min_work",
    "lu_split_min_work",
    "lu_generic_above_n",
)


class FxTune(ctypes.Structure):
    """struct fx_tune of include/fermix.h."""

    _fields_ = [(f, ctypes.c_int32) for f in TUNE_FIELDS] + [("reserved", ctypes.c_int32 * 3)]


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every function declared in include/fermix.h
SIGNATURES = {
    "fx_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "fx_abi_version": (ctypes.c_int, []),
    "fx_lu_padded_size": (_i32, [_i32]),
    "fx_pf_padded_size": (_i32, [_i32]),
    "fx_tune_table": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(FxTune)]),
    "fx_tune_override": (ctypes.c_int, [ctypes.POINTER(FxTune)]),
    "fx_tune_active": (ctypes.c_int, [ctypes.POINTER(FxTune)]),
    "fx_slogdet_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _i32, _p, _sz, _p]),
    "fx_slogdet_parts_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_parts_f32": (
        ctypes.c_int,
        [_p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p, _sz, _p],
    ),
    "fx_slogdet_factors_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_factors_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p, _i32, _p, _sz, _p]),
    "fx_slogdet_inverse_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_inverse_f32": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _i32, _p, _i32, _p, _sz, _p]),
    "fx_slogdet_f32_noalloc": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p]),
    "fx_slogdet_f32_noalloc_batch": (_i64, [_i64, _i32]),
    "fx_det_parts_f32_workspace": (_sz, [_i64, _i32]),
    "fx_det_parts_f32": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _i32, _p, _sz, _p]),
    "fx_slogpf_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_f32": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, _sz, _p]),
    "fx_pf_block_columns": (_i32, [_i32]),
    "fx_slogpf_factors_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_factors_f32": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "fx_slogpf_inverse_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_inverse_f32": (ctypes.c_int, [_p, _p, _p, _p, _i64, _i32, _i32, _p, _i32, _p, _sz, _p]),
    "fx_slogpf_parts_f32_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_parts_f32": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _p, _p, _i32, _p, _sz, _p]),
    "fx_slogdet_f64_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_f64": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _sz, _p]),
    "fx_slogdet_parts_f64_workspace": (_sz, [_i64, _i32]),
    "fx_slogdet_parts_f64": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p, _p, _sz, _p]),
    "fx_slogpf_f64_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_f64": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p, _p, _sz, _p]),
    "fx_slogpf_parts_f64_workspace": (_sz, [_i64, _i32]),
    "fx_slogpf_parts_f64": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _sz, _p]),
}
# complex64 / complex128: the float64 signatures with interleaved (re, im) buffers;
# complex64's take the prec word before the workspace (PREC_ARG[_k]: the extra argument)
PREC_ARG = {"c64": [_i32], "c128": []}
for _k in ("c64", "c128"):
    _q = PREC_ARG[_k]
    SIGNATURES.update({
        f"fx_slogdet_{_k}_workspace": (_sz, [_i64, _i32]),
        f"fx_slogdet_{_k}": (ctypes.c_int, [_p, _i64, _i32, _p, _p] + _q + [_p, _sz, _p]),
        f"fx_slogdet_parts_{_k}_workspace": (_sz, [_i64, _i32]),
        f"fx_slogdet_parts_{_k}": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p] + _q + [_p, _sz, _p]),
        f"fx_slogpf_{_k}_workspace": (_sz, [_i64, _i32]),
        f"fx_slogpf_{_k}": (ctypes.c_int, [_p, _i64, _i32, _i32, _p, _p] + _q + [_p, _sz, _p]),
        f"fx_slogpf_parts_{_k}_workspace": (_sz, [_i64, _i32]),
        f"fx_slogpf_parts_{_k}": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _p, _p] + _q + [_p, _sz, _p]),
    })
# det's gradient (the exact adjugate) for the 64-bit and complex kinds
for _k in ("f64", "c64", "c128"):
    SIGNATURES.update({
        f"fx_det_parts_{_k}_workspace": (_sz, [_i64, _i32]),
        f"fx_det_parts_{_k}": (ctypes.c_int, [_p, _i64, _i32, _p, _p, _p] + PREC_ARG.get(_k, []) + [_p, _sz, _p]),
    })


class FermixLibraryError(RuntimeError):
    """The HIP library is missing, fails to load, or a call returned an error status."""


_lib = None


def lib():
    """The loaded library (loaded once). Raises FermixLibraryError if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FermixLibraryError(
                f"{LIB_PATH} is missing: build it with `python -m fermix_amd.build` "
                "(fermix_amd has no non-HIP fallback)"
            )
        try:
            h = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - environment specific
            raise FermixLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _lib = h
    return _lib


def check(status, what):
    if status != FX_OK:
        msg = lib().fx_status_string(status).decode()
        raise FermixLibraryError(f"{what}: {msg} (status {status})")
