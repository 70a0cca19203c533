"""CPU checks of the boundary: the HIP library is built, loads, and exports every
entry point include/fermix.h declares (no compute calls without a GPU); the Python API
raises the reference's error types (src/fermix/api.py:24-31,92-97; _field.py:265-275)."""

import ctypes
import dataclasses
import os
import re
import warnings

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _lib, _tune

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fermix.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("fx_slogdet_f32", "fx_slogdet_parts_f32", "fx_slogpf_f32", "fx_status_string"):
        assert s in syms


def test_library_loads_and_exports_every_symbol():
    assert os.path.exists(_lib.LIB_PATH), "build the library first (python -m fermix_amd.build)"
    h = ctypes.CDLL(_lib.LIB_PATH)
    for s in declared_symbols():
        assert hasattr(h, s), f"{s} declared in include/fermix.h but not exported"
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_host_only_calls():
    L = _lib.lib()
    assert L.fx_abi_version() == 203
    assert L.fx_status_string(0) == b"ok"
    assert L.fx_lu_padded_size(100) == 112
    assert L.fx_pf_padded_size(128) == 128
    # argument validation happens before any device work
    assert L.fx_slogdet_f32(None, -1, 4, None, None, 0, None, 0, None) == 1
    assert L.fx_slogdet_f32(None, 0, 4, None, None, 0, None, 0, None) == 0
    assert L.fx_det_parts_f32(None, -1, 4, None, None, None, 0, None, 0, None) == 1
    assert L.fx_det_parts_f32(None, 2, 4, None, None, None, 0, None, 0, None) == 1
    assert L.fx_det_parts_f32_workspace(4, 16385) == 0 and L.fx_det_parts_f32_workspace(4, 8192) > 0
    assert L.fx_det_parts_f32_workspace(4, 8193) > 0  # the generic blocked family above 8192
    assert L.fx_slogpf_parts_f32_workspace(1, 16384) > 0 and L.fx_slogpf_parts_f32_workspace(1, 16386) == 0
    # no packed factors above 8192
    assert L.fx_lu_padded_size(8193) == -1 and L.fx_pf_padded_size(8194) == -1
    assert L.fx_slogdet_factors_f32_workspace(1, 8193) == 0 and L.fx_slogpf_inverse_f32_workspace(1, 8194) == 0
    assert L.fx_det_parts_f32_workspace(4, 64) > L.fx_slogdet_parts_f32_workspace(4, 64)


def test_family_override_sizes():
    """The padded orders and workspaces follow the forced family (host-only queries)."""
    L = _lib.lib()
    assert L.fx_lu_padded_size(20) == 32 and L.fx_slogdet_f32_workspace(4, 20) == 0
    with _tune.force_family("blocked"):
        assert L.fx_lu_padded_size(20) == 64 and L.fx_pf_padded_size(20) == 32
        assert L.fx_slogdet_f32_workspace(4, 20) > 0 and L.fx_pf_block_columns(20) == 32
    # factor chunks: 32 columns for the blocked Parlett-Reid up to 2048, 16 above
    assert [L.fx_pf_block_columns(n) for n in (100, 200, 256, 500, 512, 1024, 1025, 2048, 2049)] == [16, 32, 32, 32, 32, 32, 32, 32, 16]
    with _tune.force_family("tiny"):
        assert L.fx_lu_padded_size(40) == -1 and L.fx_pf_padded_size(20) == -1
    with _tune.force_family("fused"):
        assert L.fx_lu_padded_size(20) == -1 and L.fx_lu_padded_size(100) == 112
    assert L.fx_lu_padded_size(20) == 32


def test_api_errors():
    A = torch.zeros((2, 4, 4), dtype=torch.float32)
    with pytest.raises(TypeError):
        fermix_amd.slogdet(torch.zeros((2, 4, 4), dtype=torch.int32))
    with pytest.raises(TypeError):
        fermix_amd.slogdet(np.zeros((4, 4), np.float32))
    with pytest.raises(ValueError):
        fermix_amd.slogdet(torch.zeros((2, 4, 3)))
    with pytest.raises(ValueError):
        fermix_amd.slogdet(torch.zeros((4,)))
    with pytest.raises(ValueError):
        fermix_amd.slogdet(A, block=48)
    with pytest.raises(ValueError):
        fermix_amd.det(A, prec="fast")
    with pytest.raises(fermix_amd.FermixDeviceError):
        fermix_amd.slogdet(A)
    with pytest.raises(fermix_amd.FermixDeviceError):
        fermix_amd.slogpf(A)
    # float64 and complex are supported dtypes (device check next); tf32x3 is for the
    # 32-bit kinds only (reference src/fermix/_field.py:265-275)
    with pytest.raises(fermix_amd.FermixDeviceError):
        fermix_amd.slogdet(A.double())
    with pytest.raises(ValueError):
        fermix_amd.slogdet(A.double(), prec="tf32x3")
    with pytest.raises(ValueError):
        fermix_amd.pf(A.double(), prec="tf32x3")
    for dt in (torch.complex64, torch.complex128):
        with pytest.raises(fermix_amd.FermixDeviceError):
            fermix_amd.slogpf(A.to(dt))
    with pytest.raises(fermix_amd.FermixDeviceError):
        fermix_amd.slogdet(A.to(torch.complex64), prec="tf32x3")
    with pytest.raises(ValueError):
        fermix_amd.slogdet(A.to(torch.complex128), prec="tf32x3")
    with pytest.raises(TypeError):
        fermix_amd.slogdet(A.to(torch.float16))


def test_tune_table():
    # default: the three-pass mode for the 32-bit kinds, "ieee" for the 64-bit ones
    # (reference Field.default_prec, src/fermix/_field.py:262-263)
    assert _tune.check_prec(None) == "bf16x3" and _tune.check_prec(None, torch.float32) == "bf16x3"
    assert _tune.check_prec(None, torch.complex64) == "bf16x3"
    assert _tune.check_prec(None, torch.float64) == "ieee" and _tune.check_prec(None, torch.complex128) == "ieee"
    assert _tune.check_prec("ieee") == "ieee"
    assert _tune.check_prec("tf32x3") == "bf16x3" and _tune.check_prec("bf16x3") == "bf16x3"
    assert _tune.prec_flag("bf16x3") == 1 and _tune.prec_flag("ieee") == 0
    with pytest.raises(ValueError):
        _tune.check_prec("bf16x3", torch.float64)
    with pytest.raises(ValueError):
        _tune.check_prec("fp16")
    assert _tune.kernel_family(128) == "fused-lds"
    assert _tune.kernel_family(32) == "tiny-wave" and _tune.kernel_family(32, "slogpf") == "fused-lds"
    assert _tune.kernel_family(8192, "slogpf") == "blocked" and _tune.kernel_family(8193) == "generic"
    # the LU's own blocked kernels stop at lu_generic_above_n (4096), the Parlett-Reid's at 8192
    assert _tune.kernel_family(4096) == "blocked" and _tune.kernel_family(4097) == "generic"
    assert _tune.kernel_family(4097, "slogpf") == "blocked"
    L = _lib.lib()
    assert L.fx_lu_padded_size(4096) == 4096 and L.fx_lu_padded_size(4097) == -1 and L.fx_pf_padded_size(4098) > 0
    with _tune.override(lu_generic_above_n=8192):
        assert _tune.kernel_family(4097) == "blocked" and L.fx_lu_padded_size(4097) > 0
    with _tune.force_family("blocked"):
        assert _tune.kernel_family(6000) == "blocked" and L.fx_lu_padded_size(6000) > 0
    with _tune.force_family("generic"):
        assert _tune.kernel_family(200) == "generic" and _tune.kernel_family(100) == "unsupported"
        assert L.fx_lu_padded_size(200) == -1 and L.fx_slogdet_f32_workspace(2, 200) > 0
    assert _tune.kernel_family(16384) == "generic" and _tune.kernel_family(16385) == "unsupported"


def test_misaligned_pointers_rejected():
    """The alignment contract of include/fermix.h: a matrix-shaped or workspace pointer
    that is not 16-byte aligned (here a fake address 4 bytes past a 16-byte boundary)
    returns FX_ERR_INVALID_ARGUMENT before any device work is enqueued, for every family
    and every float32 / float64 entry point."""
    L = _lib.lib()
    good, bad = 0x10000, 0x10004
    ws = 0x20000
    for n in (8, 100, 129, 512):
        assert L.fx_slogdet_f32(bad, 2, n, good, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_f32(good, 2, n, good, good, 0, bad, 1 << 40, None) == 1
        assert L.fx_slogdet_f32(good, 2, n, good + 2, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f32(good, 2, n, 1, good, good, bad, None, None, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f32(good, 2, n, 1, good, good, good, bad, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f32(good, 2, n, 1, good, good, good, good, bad, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_factors_f32(good, 2, n, good, good, bad, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_inverse_f32(bad, good, good, None, 2, n, 1, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_inverse_f32(good, good, good, None, 2, n, 1, good, 0, bad, 1 << 40, None) == 1
        assert L.fx_det_parts_f32(good, 2, n, good, good, bad, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_f32(bad, 2, n, 0, good, good, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_factors_f32(good, 2, n, 0, good, good, bad, good, good, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_inverse_f32(good, good, good, None, 2, n, 0, bad, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_parts_f32(bad, 2, n, 0, 0, good, good, good, 0, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_f64(bad, 2, n, good, good, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f64(good, 2, n, good, good, bad, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_f64(good, 2, n, 0, good + 4, good, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_parts_f64(good, 2, n, 0, 0, good, good, bad, ws, 1 << 40, None) == 1


def test_workspace_is_one_chunk():
    """Batches above 65528 members run in chunks of 65528 on the stream, so the workspace
    of any larger batch is that of one chunk (host-only queries)."""
    L = _lib.lib()
    C = 65528
    for fn, n in (
        (L.fx_slogdet_f32_workspace, 200),
        (L.fx_slogdet_parts_f32_workspace, 200),
        (L.fx_slogdet_parts_f32_workspace, 64),
        (L.fx_slogdet_factors_f32_workspace, 200),
        (L.fx_slogdet_inverse_f32_workspace, 64),
        (L.fx_det_parts_f32_workspace, 130),
        (L.fx_slogpf_f32_workspace, 200),
        (L.fx_slogpf_factors_f32_workspace, 200),
        (L.fx_slogpf_inverse_f32_workspace, 200),
        (L.fx_slogpf_parts_f32_workspace, 64),
    ):
        w = fn(C, n)
        assert w > 0 and fn(C + 1, n) == w and fn(10 * C, n) == w, (fn, n)
        assert fn(C - 8, n) < w, (fn, n)


def test_noalloc_host_checks():
    """fx_slogdet_f32_noalloc validates its arguments and rejects n whose one-matrix
    workspace exceeds the scratch array before any device work (host-only)."""
    L = _lib.lib()
    good = 0x10000
    assert L.fx_slogdet_f32_noalloc(None, -1, 300, None, None, None) == 1
    assert L.fx_slogdet_f32_noalloc(None, 0, 300, None, None, None) == 0
    assert L.fx_slogdet_f32_noalloc(None, 4, 300, None, None, None) == 1
    limit = 64 << 20
    assert L.fx_slogdet_f32_workspace(1, 4032) <= limit < L.fx_slogdet_f32_workspace(1, 4033)
    for n in (4033, 4096):
        assert L.fx_slogdet_f32_noalloc(good, 4, n, good, good, None) == 4
    assert L.fx_slogdet_f32_noalloc(good, 4, 5000, good, good, None) == 4
    # a misaligned matrix pointer is rejected before the first sub-batch is enqueued
    assert L.fx_slogdet_f32_noalloc(good + 4, 7, 2049, good, good, None) == 1


def test_noalloc_plan():
    """The sub-batch plan of fx_slogdet_f32_noalloc (host-only): every n the entry point
    accepts has a plan, each sub-batch's workspace fits the scratch array, and sub-batches
    of 8 or more are multiples of 8. (For odd n a sub-batch may start 4-byte aligned only,
    e.g. n = 2049 runs 3 + 3 + 1 members: the blocked LU reads such matrices with 4-byte
    loads; tests/test_zz_no_alloc.py checks that case on the GPU.)"""
    L = _lib.lib()
    limit = 64 << 20
    assert L.fx_slogdet_f32_noalloc_batch(7, 2049) == 3
    assert L.fx_slogdet_f32_noalloc_batch(5, 100) == 5  # no workspace at all
    assert L.fx_slogdet_f32_noalloc_batch(3, 4033) == 0
    for n in list(range(129, 1500, 38)) + list(range(1401, 4033, 89)) + [2049, 2050, 4031, 4032]:
        for batch in (1, 3, 7, 64, 1000):
            m = L.fx_slogdet_f32_noalloc_batch(batch, n)
            assert 1 <= m <= batch and L.fx_slogdet_f32_workspace(m, n) <= limit, (n, batch, m)
            if m < batch:
                assert m < 8 or m % 8 == 0, (n, batch, m)
                assert L.fx_slogdet_f32_workspace(m + 1, n) > limit or m >= 8, (n, batch, m)


def test_prec_argument_validated():
    """prec outside {FX_PREC_IEEE, FX_PREC_BF16X3} is rejected before any device work."""
    L = _lib.lib()
    good, ws = 0x10000, 0x20000
    for bad_prec in (-1, 2, 7):
        assert L.fx_slogdet_f32(good, 2, 300, good, good, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f32(good, 2, 300, 1, good, good, good, None, None, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_factors_f32(good, 2, 300, good, good, good, good, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_inverse_f32(good, good, good, None, 2, 300, 1, good, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_det_parts_f32(good, 2, 300, good, good, good, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_inverse_f32(good, good, good, None, 2, 300, 0, good, bad_prec, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_parts_f32(good, 2, 300, 0, 0, good, good, good, bad_prec, ws, 1 << 40, None) == 1


def test_lu_block_option_validated():
    """The FX_LU_BLOCK_* option bits are accepted by the LU factorisations only, and
    FX_LU_BLOCK_64 | FX_LU_BLOCK_128 together, or unknown bits, are rejected before any
    device work (batch 0 returns FX_OK once the arguments pass)."""
    L = _lib.lib()
    good, ws = 0x10000, 0x20000
    for opt in (_lib.FX_LU_BLOCK_64, _lib.FX_LU_BLOCK_128, _lib.FX_LU_BLOCK_128 | 1):
        assert L.fx_slogdet_f32(good, 0, 300, good, good, opt, ws, 1 << 40, None) == 0
        assert L.fx_slogdet_parts_f32(good, 0, 300, 1, good, good, good, None, None, opt, ws, 1 << 40, None) == 0
        assert L.fx_slogdet_factors_f32(good, 0, 300, good, good, good, good, opt, ws, 1 << 40, None) == 0
        assert L.fx_det_parts_f32(good, 0, 300, good, good, good, opt, ws, 1 << 40, None) == 0
        # the inverse and the Parlett-Reid entry points take no option bits
        assert L.fx_slogdet_inverse_f32(good, good, good, None, 2, 300, 1, good, opt, ws, 1 << 40, None) == 1
        assert L.fx_slogpf_parts_f32(good, 2, 300, 0, 0, good, good, good, opt, ws, 1 << 40, None) == 1
    for bad in (_lib.FX_LU_BLOCK_64 | _lib.FX_LU_BLOCK_128, 0x400, 0x10, _lib.FX_LU_BLOCK_64 | 2):
        assert L.fx_slogdet_f32(good, 0, 300, good, good, bad, ws, 1 << 40, None) == 1
        assert L.fx_slogdet_parts_f32(good, 0, 300, 1, good, good, good, None, None, bad, ws, 1 << 40, None) == 1
        assert L.fx_det_parts_f32(good, 0, 300, good, good, good, bad, ws, 1 << 40, None) == 1


def test_tuning_table_in_library():
    """The gfx950 table the C library holds is the one fermix_amd._tune states; other
    architecture names are refused; target features after ':' are ignored."""
    assert _tune.library_table("gfx950") == _tune.TUNES["gfx950"] == _tune.table()
    assert _tune.library_table("gfx950:sramecc+:xnack-") == _tune.TUNES["gfx950"]
    L = _lib.lib()
    t = _lib.FxTune()
    assert L.fx_tune_table(b"gfx942", t) == 4 and L.fx_tune_table(b"gfx9500", t) == 4
    assert _tune.active() == _tune.table()
    with pytest.raises(ValueError):
        _tune.table("gfx90a")


def test_tuning_override():
    """The override hook replaces the table for later calls (dispatch and workspace
    queries follow it), rejects values outside the compiled kernels' ranges without
    changing anything, and the context manager restores the table."""
    L = _lib.lib()
    base = _tune.table()
    # fused family up to 128 by the table; lowered, n = 100 goes to the blocked kernels
    assert L.fx_lu_padded_size(100) == 112 and L.fx_slogdet_f32_workspace(4, 100) == 0
    assert _tune.kernel_family(100) == "fused-lds"
    with _tune.override(fused_max_n=64) as t:
        assert t.fused_max_n == 64 and _tune.active() == t
        assert L.fx_lu_padded_size(100) == 128 and L.fx_slogdet_f32_workspace(4, 100) > 0
        assert L.fx_pf_padded_size(100) == 128 and L.fx_pf_block_columns(100) == 32
        assert _tune.kernel_family(100) == "blocked" and _tune.kernel_family(64) == "fused-lds"
    assert _tune.active() == base and L.fx_lu_padded_size(100) == 112
    # 64-column Parlett-Reid blocks need a G buffer twice as wide: the workspace follows
    w64 = L.fx_slogpf_f32_workspace(4, 1024)
    with _tune.override(pf_block64_max_m=0):
        w32 = L.fx_slogpf_f32_workspace(4, 1024)
    with _tune.override(pf_block64_min_n=2048):
        assert L.fx_slogpf_f32_workspace(4, 1024) == w32
    assert w32 < w64 == L.fx_slogpf_f32_workspace(4, 1024)
    # float64: the register kernels need no workspace; lowered, n = 100 takes the LDS /
    # workspace kernel (n * 2n doubles do not fit its LDS for the inverse)
    assert L.fx_slogdet_parts_f64_workspace(4, 100) == 0
    with _tune.override(f64_reg_max_n=64):
        assert L.fx_slogdet_parts_f64_workspace(4, 100) > 0
    for bad in (
        dict(fused_max_n=129),
        dict(fused_max_n=16),
        dict(lu_direct_max_n=2048),
        dict(pf_block64_max_m=2048),
        dict(pf_block64_min_n=64),
        dict(gemm128_min_mn=64),
        dict(f64_reg_max_n=256),
        dict(f64_strip16_max_n=128),
        dict(lu_pair_above_n=-1),
        dict(pf_overlap_max_half=-1),
        dict(lu_split_min_work=-1),
        dict(lu_generic_above_n=64),
        dict(lu_generic_above_n=8193),
    ):
        with pytest.raises(_lib.FermixLibraryError):
            _tune.set_override(dataclasses.replace(base, **bad))
        assert _tune.active() == base
    t = _lib.FxTune()
    assert L.fx_tune_active(t) == 0
    t.reserved[2] = 1
    assert L.fx_tune_override(t) == 1 and _tune.active() == base


def test_knob_warnings():
    """The reference's knobs without a gfx950 counterpart warn (FermixTuneWarning) instead
    of passing silently; block=32 maps to 64 with a warning; valid block values do not
    warn. (The device check comes after: CPU tensors still raise FermixDeviceError.)"""
    A = torch.zeros((2, 4, 4), dtype=torch.float32)
    with pytest.warns(fermix_amd.FermixTuneWarning, match="unroll_steps"):
        with pytest.raises(fermix_amd.FermixDeviceError):
            fermix_amd.slogdet(A, unroll_steps=True)
    with pytest.warns(fermix_amd.FermixTuneWarning, match="upd_warps"):
        with pytest.raises(fermix_amd.FermixDeviceError):
            fermix_amd.slogpf(A, upd_warps=8)
    with pytest.warns(fermix_amd.FermixTuneWarning, match="block=32"):
        assert _tune.block_flag(32) == _lib.FX_LU_BLOCK_64
    assert _tune.block_flag(None) == 0 and _tune.block_flag(128) == _lib.FX_LU_BLOCK_128
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        for blk in (None, 64, 128):
            with pytest.raises(fermix_amd.FermixDeviceError):
                fermix_amd.det(A, block=blk)


def test_complex_entry_points_host_checks():
    """The complex entry points validate alignment (16 bytes for matrices / workspace,
    the value size for sign / logabs), batch and n before any device work, and size
    their workspace (none while the matrix fits the LDS limit)."""
    L = _lib.lib()
    good, bad, ws = 0x10000, 0x10008, 0x20000
    for k, esz in (("c64", 4), ("c128", 8)):
        q = [_lib.FX_PREC_BF16X3] if k == "c64" else []  # complex64's prec argument
        f = getattr(L, f"fx_slogdet_{k}")
        assert f(bad, 2, 40, good, good, *q, ws, 1 << 40, None) == 1
        assert f(good, 2, 40, good + esz, good, *q, ws, 1 << 40, None) == 1  # sign: one complex value
        assert f(good, -1, 40, good, good, *q, ws, 1 << 40, None) == 1
        assert f(good, 0, 40, good, good, *q, ws, 1 << 40, None) == 0
        assert f(good, 2, 8193, good, good, *q, ws, 1 << 40, None) == 4
        if k == "c64":  # an unknown product mode
            assert f(good, 2, 40, good, good, 7, ws, 1 << 40, None) == 1
        assert getattr(L, f"fx_slogdet_parts_{k}")(good, 2, 40, good, good, bad, *q, ws, 1 << 40, None) == 1
        assert getattr(L, f"fx_slogpf_{k}")(bad, 2, 40, 0, good, good, *q, ws, 1 << 40, None) == 1
        assert getattr(L, f"fx_slogpf_parts_{k}")(good, 2, 40, 0, 0, good, good, bad, *q, ws, 1 << 40, None) == 1
        # the Pfaffian adjugate mode checks its workspace like the inverse mode
        assert getattr(L, f"fx_slogpf_parts_{k}")(good, 2, 300, 0, 1, good, good, good, *q, ws, 256, None) == 2
        assert getattr(L, f"fx_slogdet_{k}_workspace")(4, 40) == 0
        # n = 300 runs the blocked LU: one copy of padded order 320 plus its pivots and the
        # multi-workgroup panels' posts (G = 1 workgroup's worth per member at this order;
        # each buffer rounded up to 256 bytes); the inverse adds the solve's matrix and flags
        w = getattr(L, f"fx_slogdet_{k}_workspace")(4, 300)

        def al(x):
            return (x + 255) // 256 * 256

        fz = 2 * esz
        G = 1
        sync = 2 * al(4 * 4) + al(4 * 2 * G * 8) + al(4 * 2 * G * 4) + al(4 * 2 * G * 32 * fz) + al(4 * 2 * 32 * fz)
        assert w == al(4 * 320 * 320 * fz) + al(4 * 320 * 4) + al(4 * 320 * fz) + al(4 * 10 * 4) + sync
        assert getattr(L, f"fx_slogdet_parts_{k}_workspace")(4, 300) == w + al(4 * 320 * 320 * fz) + al(4 * 4)


def test_tune_struct_layout():
    """The ctypes mirror of struct fx_tune has the header's fields in the header's order
    and the same size (fx_tune_table writes the whole struct)."""
    hdr = open(os.path.join(os.path.dirname(__file__), "..", "include", "fermix.h")).read()
    body = re.search(r"typedef struct fx_tune \{(.*?)\} fx_tune;", hdr, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = re.findall(r"int32_t\s+(\w+)(?:\[(\d+)\])?;", body)
    names = [f for f, n in fields if not n]
    count = sum(int(n) if n else 1 for _, n in fields)
    assert tuple(names) == _lib.TUNE_FIELDS
    assert ctypes.sizeof(_lib.FxTune) == 4 * count
