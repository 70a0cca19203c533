"""Option validation and the gfx950 tuning table -- the counterpart of the reference's
``Tune`` / ``TUNES[arch][kind]`` / ``OVERRIDE`` / ``_tune`` (src/fermix/_common.py:17-378)
and ``Field.check_prec`` (src/fermix/_field.py:262-275).

The reference's table holds Triton tiles and warps per NVIDIA architecture and dtype
kind. The gfx950 table holds the size thresholds of the C library's own dispatch
decisions (``struct fx_tune`` in include/fermix.h): which kernel family runs an order n,
whether the blocked LU goes in block pairs, when the Parlett-Reid blocks are 64 columns
wide, when the GEMMs take 128 x 128 tiles, and the float64 kernels' register limits.
Every choice is made from n alone, never from the batch size, so batched and vmapped
calls run the same arithmetic. The C library holds the table (``fx_tune_table``) and
reads the values in effect on every call; ``TUNES`` below states the same values and a
CPU test checks that the two agree. ``override`` replaces the table for the calls made
inside it (the reference's ``OVERRIDE`` hook, used by its tests and tuning sweeps).
"""

import contextlib
import dataclasses
import os
import warnings

import torch

# prec values accepted by the public API (the reference's PREC, src/fermix/_field.py:20-23):
#  * "ieee": fp32 MFMA products;
#  * "bf16x3": each fp32 operand split into three bf16 parts and six bf16 MFMA products,
#    fp32 accumulation (fp32-level accuracy, several times the MFMA rate of fp32);
#  * "tf32x3": the reference's name for its three-pass fp32-accuracy mode on tensor cores;
#    gfx950 has no TF32 type, so it selects the gfx950 counterpart, "bf16x3".
# The mode applies to the blocked kernels' trailing LU updates and to the inverse /
# adjugate GEMMs (include/fermix.h, FX_PREC_*). The default is the three-pass mode for
# the 32-bit kinds and "ieee" for the 64-bit ones, as the reference's Field.default_prec
# (src/fermix/_field.py:262-263): on MI355X "bf16x3" is also the faster mode of the
# blocked gradients (128 x 128 GEMM tiles with the operands split once in LDS), with the
# same accuracy bar as "ieee" (tests/test_gpu_prec.py).
PREC = ("ieee", "tf32x3", "bf16x3")
DEFAULT_PREC = "bf16x3"


class FermixTuneWarning(UserWarning):
    """A tuning knob of the reference's API that has no counterpart (or only the nearest
    one) in the gfx950 kernels."""


def check_prec(prec, dtype=None):
    """The mode a `prec` argument selects ("ieee" or "bf16x3"). The reduced-precision
    modes apply to the 32-bit kinds only (the reference rejects "tf32x3" for float64 /
    complex128, src/fermix/_field.py:265-275). For complex64 the fp32-accuracy mode
    ("bf16x3" / "tf32x3", the default) forms the blocked kernels' products on the fp64
    MFMA with the operands widened, "ieee" as four fp32 MFMA products per complex one."""
    if prec is None:
        return "ieee" if dtype in (torch.float64, torch.complex128) else DEFAULT_PREC
    if prec not in PREC:
        raise ValueError(f"prec must be one of {PREC}, got {prec!r}")
    if prec != "ieee" and dtype is not None and dtype not in (torch.float32, torch.complex64):
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


# option bits of the C ABI's prec word (include/fermix.h: FX_LU_BLOCK_*)
FX_LU_BLOCK_64 = 0x100
FX_LU_BLOCK_128 = 0x200


def block_flag(block):
    """The FX_LU_BLOCK_* option of the reference's `block` (api.py:92-97, _common.py:31-41).
    The blocked LU is built from 64-column panels whose trailing updates run one block at a
    time (K = 64) or in pairs (one K = 128 update per pair, the role of the reference's
    128-column block): None -> the table, 64 -> single blocks, 128 -> pairs; 32 has no
    gfx950 kernel and runs single 64-column blocks, with a FermixTuneWarning. It applies to
    the blocked family (n above fused_max_n); the forward and the gradient of one call take
    the same option, so the differentiated primal stays bit-identical."""
    if block is None:
        return 0
    if block == 32:
        warnings.warn(
            "fermix_amd: block=32 has no gfx950 kernel (the LU panels are 64 columns wide); "
            "running single 64-column blocks (block=64)",
            FermixTuneWarning,
            stacklevel=3,
        )
        return FX_LU_BLOCK_64
    return FX_LU_BLOCK_64 if block == 64 else FX_LU_BLOCK_128


def note_ignored(name, value):
    """Warn (once per call site) that a reference knob has no effect on gfx950."""
    if value is None:
        return
    why = {
        "unroll_steps": "the gfx950 panels are always fully unrolled at compile time",
        "upd_warps": "the Parlett-Reid trailing update always runs 4 waves per 64 x 64 tile "
        "(tune the blocked kernels with fermix_amd._tune.override)",
    }[name]
    warnings.warn(f"fermix_amd: {name}={value!r} has no effect: {why}", FermixTuneWarning, stacklevel=3)


@dataclasses.dataclass(frozen=True)
class Tune:
    """The gfx950 launch thresholds (struct fx_tune, include/fermix.h); see the C header
    for each field's meaning and range. The values are those measured on MI355X
    (fermix_amd/csrc/tune.hip states the measurement behind each)."""

    # float32: n <= fused_max_n (beyond the several-matrices-per-wave sizes) runs one
    # workgroup per matrix in LDS, larger n the blocked kernels
    fused_max_n: int = 128
    # blocked LU: block pairs (one K = 128 update per pair) for padded N above this
    lu_pair_above_n: int = 256
    # blocked LU: the first block pair reads the input in place for n = N <= this
    lu_direct_max_n: int = 1024
    # blocked Parlett-Reid: 64-column blocks for N >= pf_block64_min_n (a multiple of 64)
    # once the trailing order is <= pf_block64_max_m
    pf_block64_min_n: int = 512
    pf_block64_max_m: int = 1024
    # GEMMs (fp32 MFMA): 128 x 128 tiles for M, N >= gemm128_min_mn and K >=
    # gemm128_min_k, also for the product with A^-T's transposed, row-permuted output
    # if gemm128_tout; the gemm128_x3_* fields are the same for prec="bf16x3"
    gemm128_min_mn: int = 1024
    gemm128_min_k: int = 512
    gemm128_tout: int = 0
    gemm128_x3_min_mn: int = 128
    gemm128_x3_min_k: int = 128
    gemm128_x3_tout: int = 1
    # float64: registers for n <= f64_reg_max_n, 16-column strips for n <= f64_strip16_max_n
    f64_reg_max_n: int = 128
    f64_strip16_max_n: int = 64
    # blocked float32 Parlett-Reid: two halves, one half's panels beside the other half's
    # update in each launch, for halves of at most pf_overlap_max_half matrices and
    # batch * N^2 >= pf_overlap_min_work * 2^20
    pf_overlap_max_half: int = 32
    pf_overlap_min_work: int = 256
    # blocked float32 LU (N <= 4096): two halves on two streams for batch * N^2 >=
    # lu_split_min_work * 2^20 (0: never)
    lu_split_min_work: int = 128
    # float32 LU: n above this runs the field-generic blocked kernels ("generic" family)
    lu_generic_above_n: int = 4096


# per-architecture tables (the library holds gfx950 code only)
TUNES = {"gfx950": Tune()}


def arch(device=None):
    """The gfx architecture name of a ROCm device ("gfx950"), without target features."""
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return props.gcnArchName.split(":")[0]


def table(arch_name="gfx950"):
    """The tuning table of an architecture."""
    if arch_name not in TUNES:
        raise ValueError(f"fermix_amd has kernels for {sorted(TUNES)} only, not {arch_name!r}")
    return TUNES[arch_name]


def _to_c(t):
    from ._lib import FxTune

    c = FxTune()
    for f in dataclasses.fields(Tune):
        setattr(c, f.name, int(getattr(t, f.name)))
    return c


def _from_c(c):
    return Tune(**{f.name: int(getattr(c, f.name)) for f in dataclasses.fields(Tune)})


def library_table(arch_name="gfx950"):
    """The table the C library holds for an architecture (fx_tune_table)."""
    from ._lib import FxTune, check, lib

    c = FxTune()
    check(lib().fx_tune_table(arch_name.encode(), c), f"fx_tune_table({arch_name!r})")
    return _from_c(c)


def active():
    """The values in effect in the library (the override if one is set, else the table)."""
    from ._lib import FxTune, check, lib

    c = FxTune()
    check(lib().fx_tune_active(c), "fx_tune_active")
    return _from_c(c)


def set_override(t):
    """Replace the library's table for every later call (None: back to the table); a
    value outside the compiled kernels' range raises FermixLibraryError and changes
    nothing."""
    from ._lib import check, lib

    check(lib().fx_tune_override(None if t is None else _to_c(t)), "fx_tune_override")


@contextlib.contextmanager
def override(t=None, **changes):
    """Run the calls inside the block with the table replaced: ``override(Tune(...))`` or
    ``override(lu_pair_above_n=0)`` (fields changed from the values in effect). The
    previous values come back on exit. Workspace sizes follow the values in effect."""
    old = active()
    new = dataclasses.replace(t if t is not None else old, **changes)
    set_override(new)
    try:
        yield new
    finally:
        set_override(None if old == table() else old)


# n ranges -> kernel family (mirrors fx_slogdet_f32 / fx_slogpf_f32 dispatch)
TINY_MAX_N = {"slogdet": 32, "slogpf": 16}  # several matrices per wave, one lane per row
SMALL_MAX_N = 128  # largest n the fused one-workgroup-per-matrix kernels are built for
LARGE_MAX_N = 8192  # blocked kernels (float32)
# float32 above LARGE_MAX_N: the field-generic blocked kernels of the float64 path on
# float storage (values and the gradients' parts runs, no packed factors); larger n is
# unsupported
GENERIC_MAX_N = 16384

# The library's family override (read by every C entry point; a test hook like the
# reference's OVERRIDE, src/fermix/_common.py:363-378, which its tests use to force a
# dispatch path, tests/test_fermix.py:720-762).
ENV = "FERMIX_AMD_KERNELS"
FAMILIES = {"tiny": "tiny-wave", "fused": "fused-lds", "blocked": "blocked", "generic": "generic"}


def _fused_max():
    try:
        return min(active().fused_max_n, SMALL_MAX_N)
    except Exception:  # library not built: the table's value
        return min(table().fused_max_n, SMALL_MAX_N)


def _lu_generic_above():
    try:
        return active().lu_generic_above_n
    except Exception:  # library not built: the table's value
        return table().lu_generic_above_n


def kernel_family(n, op="slogdet"):
    """Name of the kernel family the library runs for order n ("slogdet" / "slogpf", the
    same for their gradients), honouring the family override and the tuning values in
    effect."""
    forced = os.environ.get(ENV, "")
    if forced in FAMILIES:
        if n > LARGE_MAX_N:
            return "generic" if forced in ("blocked", "generic") and n <= GENERIC_MAX_N else "unsupported"
        ok = {
            "tiny": n <= TINY_MAX_N[op],
            "fused": TINY_MAX_N[op] < n <= SMALL_MAX_N,
            "blocked": True,
            "generic": n > SMALL_MAX_N,
        }[forced]
        return FAMILIES[forced] if ok else "unsupported"
    if n <= TINY_MAX_N[op]:
        return "tiny-wave"
    if n <= _fused_max():
        return "fused-lds"
    if op == "slogdet" and n > _lu_generic_above() and n <= GENERIC_MAX_N:
        return "generic"
    if n <= LARGE_MAX_N:
        return "blocked"
    if n <= GENERIC_MAX_N:
        return "generic"
    return "unsupported"


@contextlib.contextmanager
def force_family(family):
    """Force a kernel family ("tiny", "fused", "blocked" or "generic") for the calls made inside the
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
