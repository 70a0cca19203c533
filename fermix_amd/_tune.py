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

# prec values accepted by the public API. "ieee": fp32 MFMA / FMA updates (the only
# arithmetic of this build). "tf32x3" is accepted for drop-in compatibility with the
# reference's float32 default: it exists there to reach fp32-level accuracy on tensor
# cores; gfx950 has no TF32 type, and its IEEE fp32 MFMA path is that accuracy.
PREC = ("ieee", "tf32x3")


def check_prec(prec, dtype=None):
    """"tf32x3" is accepted for float32 only (the reference rejects it for 64-bit types,
    src/fermix/_field.py:265-275)."""
    if prec is None:
        return "ieee"
    if prec not in PREC:
        raise ValueError(f"prec must be 'tf32x3' or 'ieee', got {prec!r}")
    if prec == "tf32x3" and dtype is not None and dtype != torch.float32:
        raise ValueError(
            "prec='tf32x3' applies to float32 / complex64 only; float64 and "
            "complex128 run in IEEE fp64 (prec='ieee')"
        )
    return "ieee"


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
