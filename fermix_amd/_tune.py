"""Option validation and the gfx950 launch table -- the counterpart of the reference's
``Tune`` / ``TUNES`` / ``OVERRIDE`` (src/fermix/_common.py:17-378) and
``Field.check_prec`` (src/fermix/_field.py:262-275).

The reference keys its table by NVIDIA architecture and tunes Triton warps and tiles;
on gfx950 the choices are which kernel family runs for a given n (always chosen from n
alone, never from the batch size, so batched and vmapped calls run the same
arithmetic). The table lives in the C library's dispatch (``fermix_amd/csrc/api.hip``);
this module mirrors it for introspection and tests.
"""

import contextlib
import os

import torch

# prec values accepted by the public API (the reference's PREC, src/fermix/_field.py:20-23):
#  * "ieee": fp32 MFMA products;
#  * "bf16x3": each fp32 operand split into three bf16 parts and six bf16 MFMA products,
#    fp32 accumulation (fp32-level accuracy, several times the MFMA rate of fp32);
#  * "tf32x3": the reference's name for its three-pass fp32-accuracy mode on tensor cores;
#    gfx950 has no TF32 type, so it selects the gfx950 counterpart, "bf16x3".
# The mode applies to the blocked kernels' trailing LU updates and to the inverse /
# adjugate GEMMs (include/fermix.h, FX_PREC_*); the default is "ieee".
PREC = ("ieee", "tf32x3", "bf16x3")
DEFAULT_PREC = "ieee"


def check_prec(prec, dtype=None):
    """The mode a `prec` argument selects ("ieee" or "bf16x3"). The reduced-precision
    modes are float32-only (the reference rejects "tf32x3" for 64-bit types,
    src/fermix/_field.py:265-275)."""
    if prec is None:
        return DEFAULT_PREC
    if prec not in PREC:
        raise ValueError(f"prec must be one of {PREC}, got {prec!r}")
    if prec != "ieee" and dtype is not None and dtype != torch.float32:
        raise ValueError(
            f"prec={prec!r} applies to float32 / complex64 only; float64 and "
            "complex128 run in IEEE fp64 (prec='ieee')"
        )
    return "ieee" if prec == "ieee" else "bf16x3"


def prec_flag(mode):
    """The C ABI's prec value of a mode returned by check_prec."""
    return 1 if mode == "bf16x3" else 0


def check_block(block):
    """The reference's outer LU block choice (api.py:92-97): None, 32, 64 or 128."""
    if block is not None and block not in (32, 64, 128):
        raise ValueError(f"block must be None, 32, 64 or 128, got {block!r}")
    return block


# n ranges -> kernel family (mirrors fx_slogdet_f32 / fx_slogpf_f32 dispatch)
TINY_MAX_N = {"slogdet": 32, "slogpf": 16}  # several matrices per wave, one lane per row
SMALL_MAX_N = 128  # fused one-workgroup-per-matrix kernels, matrix resident in LDS
LARGE_MAX_N = 4096  # blocked kernels; larger n is unsupported

# The library's family override (read by every C entry point; the counterpart of the
# reference's OVERRIDE hook, src/fermix/_common.py:363-378, which its tests use to force
# a dispatch path, tests/test_fermix.py:720-762).
ENV = "FERMIX_AMD_KERNELS"
FAMILIES = {"tiny": "tiny-wave", "fused": "fused-lds", "blocked": "blocked"}


def kernel_family(n, op="slogdet"):
    """Name of the kernel family the library runs for order n ("slogdet" / "slogpf", the
    same for their gradients), honouring an active override."""
    forced = os.environ.get(ENV, "")
    if forced in FAMILIES:
        if n > LARGE_MAX_N:
            return "unsupported"
        ok = {
            "tiny": n <= TINY_MAX_N[op],
            "fused": TINY_MAX_N[op] < n <= SMALL_MAX_N,
            "blocked": True,
        }[forced]
        return FAMILIES[forced] if ok else "unsupported"
    if n <= TINY_MAX_N[op]:
        return "tiny-wave"
    if n <= SMALL_MAX_N:
        return "fused-lds"
    if n <= LARGE_MAX_N:
        return "blocked"
    return "unsupported"


@contextlib.contextmanager
def override(family):
    """Force a kernel family ("tiny", "fused" or "blocked") for the calls made inside the
    block (a size the family does not cover then raises FermixLibraryError). Sets the
    library's environment variable for the process and restores it on exit."""
    if family not in FAMILIES:
        raise ValueError(f"family must be one of {sorted(FAMILIES)}, got {family!r}")
    old = os.environ.get(ENV)
    os.environ[ENV] = family
    try:
        yield
    finally:
        if old is None:
            os.environ.pop(ENV, None)
        else:
            os.environ[ENV] = old
