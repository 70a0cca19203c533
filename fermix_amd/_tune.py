"""Option validation and the gfx950 launch table -- the counterpart of the reference's
``Tune`` / ``TUNES`` / ``OVERRIDE`` (src/fermix/_common.py:17-378) and
``Field.check_prec`` (src/fermix/_field.py:262-275).

The reference keys its table by NVIDIA architecture and tunes Triton warps and tiles;
on gfx950 the choices are which kernel family runs for a given n (always chosen from n
alone, never from the batch size, so batched and vmapped calls run the same
arithmetic). The table lives in the C library's dispatch (``fermix_amd/csrc/api.hip``);
this module mirrors it for introspection and tests.
"""

# prec values accepted by the public API. "ieee": fp32 MFMA / FMA updates (the only
# arithmetic of this build). "tf32x3" is accepted for drop-in compatibility with the
# reference's float32 default: it exists there to reach fp32-level accuracy on tensor
# cores; gfx950 has no TF32 type, and its IEEE fp32 MFMA path is that accuracy.
PREC = ("ieee", "tf32x3")


def check_prec(prec):
    if prec is None:
        return "ieee"
    if prec not in PREC:
        raise ValueError(f"prec must be 'tf32x3' or 'ieee', got {prec!r}")
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


def kernel_family(n, op="slogdet"):
    """Name of the kernel family the library runs for order n ("slogdet" / "slogpf", the
    same for their gradients)."""
    if n <= TINY_MAX_N[op]:
        return "tiny-wave"
    if n <= SMALL_MAX_N:
        return "fused-lds"
    if n <= LARGE_MAX_N:
        return "blocked"
    return "unsupported"
