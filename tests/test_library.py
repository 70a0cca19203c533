"""CPU checks of the boundary: the HIP library is built, loads, and exports every
entry point include/fermix.h declares (no compute calls without a GPU); the Python API
raises the reference's error types (src/fermix/api.py:24-31,92-97; _field.py:265-275)."""

import ctypes
import os
import re

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
    assert L.fx_abi_version() == 200
    assert L.fx_status_string(0) == b"ok"
    assert L.fx_lu_padded_size(100) == 112
    assert L.fx_pf_padded_size(128) == 128
    # argument validation happens before any device work
    assert L.fx_slogdet_f32(None, -1, 4, None, None, 0, None, 0, None) == 1
    assert L.fx_slogdet_f32(None, 0, 4, None, None, 0, None, 0, None) == 0
    assert L.fx_det_parts_f32(None, -1, 4, None, None, None, 0, None, 0, None) == 1
    assert L.fx_det_parts_f32(None, 2, 4, None, None, None, 0, None, 0, None) == 1
    assert L.fx_det_parts_f32_workspace(4, 5000) == 0 and L.fx_det_parts_f32_workspace(4, 4096) > 0
    assert L.fx_det_parts_f32_workspace(4, 64) > L.fx_slogdet_parts_f32_workspace(4, 64)


def test_family_override_sizes():
    """The padded orders and workspaces follow the forced family (host-only queries)."""
    L = _lib.lib()
    assert L.fx_lu_padded_size(20) == 32 and L.fx_slogdet_f32_workspace(4, 20) == 0
    with _tune.override("blocked"):
        assert L.fx_lu_padded_size(20) == 64 and L.fx_pf_padded_size(20) == 32
        assert L.fx_slogdet_f32_workspace(4, 20) > 0 and L.fx_pf_block_columns(20) == 32
    # factor chunks: 32 columns for the blocked Parlett-Reid up to 2048, 16 above
    assert [L.fx_pf_block_columns(n) for n in (100, 200, 256, 500, 512, 1024, 1025, 2048, 2049)] == [16, 32, 32, 32, 32, 32, 32, 32, 16]
    with _tune.override("tiny"):
        assert L.fx_lu_padded_size(40) == -1 and L.fx_pf_padded_size(20) == -1
    with _tune.override("fused"):
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
    # float64 is a supported dtype (device check next); tf32x3 is float32-only
    # (reference src/fermix/_field.py:265-275); complex is not built
    with pytest.raises(fermix_amd.FermixDeviceError):
        fermix_amd.slogdet(A.double())
    with pytest.raises(ValueError):
        fermix_amd.slogdet(A.double(), prec="tf32x3")
    with pytest.raises(ValueError):
        fermix_amd.pf(A.double(), prec="tf32x3")
    with pytest.raises(TypeError):
        fermix_amd.slogdet(A.to(torch.complex64))


def test_tune_table():
    assert _tune.check_prec(None) == "ieee"
    assert _tune.check_prec("ieee") == "ieee"
    assert _tune.check_prec("tf32x3") == "bf16x3" and _tune.check_prec("bf16x3") == "bf16x3"
    assert _tune.prec_flag("bf16x3") == 1 and _tune.prec_flag("ieee") == 0
    with pytest.raises(ValueError):
        _tune.check_prec("bf16x3", torch.float64)
    with pytest.raises(ValueError):
        _tune.check_prec("fp16")
    assert _tune.kernel_family(128) == "fused-lds"
    assert _tune.kernel_family(32) == "tiny-wave" and _tune.kernel_family(32, "slogpf") == "fused-lds"
    assert _tune.kernel_family(4096, "slogpf") == "blocked" and _tune.kernel_family(4097) == "unsupported"


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
