"""GPU checks of the tuning table's choices (fermix_amd._tune, struct fx_tune) and of the
per-call LU block option (the reference's `block`, src/fermix/api.py:92-97): every value
the table or an override can select runs kernels whose results meet the parity bars
against float64, choices documented as rounding-neutral are bit-identical to the table's,
and a differentiated call reproduces its own forward bit for bit under the same choice --
the counterpart of the reference's OVERRIDE-driven dispatch tests
(tests/test_fermix.py:720-762)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _tune
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs, assert_logabs64

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def _mats(n, B, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)


@pytest.mark.parametrize("n", [129, 192, 256, 320, 512])
@pytest.mark.parametrize("block", [64, 128])
def test_lu_block_option(dev, n, block):
    """block=64 (single blocks) and block=128 (pairs) at sizes where the table picks the
    other: values and A^-T against float64, and the differentiated primal bit-identical to
    the plain forward with the same block."""
    A = _mats(n, 6, 7000 + n)
    print(f"lu block={block} n={n}", flush=True)
    At = _t(A, dev)
    s, l = map(_np, fermix_amd.slogdet(At, block=block))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, f"block={block}", A)
    X = At.clone().requires_grad_(True)
    s2, l2 = fermix_amd.slogdet(X, block=block)
    assert np.array_equal(_np(s2), s) and np.array_equal(_np(l2), l)
    (g,) = torch.autograd.grad(l2.sum(), X)
    ref = np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1)
    assert_grad(_np(g), ref, A, f"block={block} grad")
    # det takes the same option: sign * exp(logabs) of the same factorisation
    st, lt = fermix_amd.slogdet(At, block=block)
    assert torch.equal(fermix_amd.det(At, block=block), st * torch.exp(lt))


def test_lu_block_changes_rounding_only(dev):
    """At n = 512 the table runs block pairs; block=128 is that choice (bit-identical),
    block=64 a different rounding of the same factorisation."""
    A = _t(_mats(512, 8, 7100), dev)
    s0, l0 = map(_np, fermix_amd.slogdet(A))
    s1, l1 = map(_np, fermix_amd.slogdet(A, block=128))
    s2, l2 = map(_np, fermix_amd.slogdet(A, block=64))
    assert np.array_equal(s0, s1) and np.array_equal(l0, l1)
    assert np.array_equal(s0, s2) and np.max(np.abs(l2 - l0)) < 1e-3


@pytest.mark.parametrize("n", [200, 512])
def test_lu_override_pairs_and_direct(dev, n):
    """Override: pairs from the smallest blocked size (lu_pair_above_n = 0) against float64;
    the input copy instead of the in-place first pair (lu_direct_max_n = 0) gives the same
    bits as the table."""
    A = _mats(n, 6, 7200 + n)
    At = _t(A, dev)
    s0, l0 = map(_np, fermix_amd.slogdet(At))
    print(f"lu override n={n}", flush=True)
    with _tune.override(lu_direct_max_n=0):
        s1, l1 = map(_np, fermix_amd.slogdet(At))
        _, _, inv1 = fermix_amd._kernels.slogdet_parts(At)[:3]
    _, _, inv0 = fermix_amd._kernels.slogdet_parts(At)[:3]
    assert np.array_equal(s0, s1) and np.array_equal(l0, l1)
    assert torch.equal(inv0, inv1)
    with _tune.override(lu_pair_above_n=0):
        s2, l2 = map(_np, fermix_amd.slogdet(At))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(s2, s64)
    assert_logabs(l2, l64, n, "pairs everywhere", A)


@pytest.mark.parametrize("n", [256, 512])
def test_gemm_tile_override_bit_identical(dev, n):
    """fp32 MFMA: 128 x 128 GEMM tiles (gemm128_min_mn / _k lowered and gemm128_tout set, so
    that every n <= 512 inverse GEMM, the A^-T product with its transposed output included,
    takes them) give the same bits as the 64 x 64 tiles of the table, for A^-T and S^-1."""
    A = _mats(n, 4, 7300 + n)
    At = _t(A, dev)
    S = _t(A - A.transpose(0, 2, 1), dev)
    ref_inv = fermix_amd._kernels.slogdet_parts(At, x3=0)[2]
    ref_sinv = fermix_amd._kernels.slogpf_parts(S, False, x3=0)[2]
    print(f"gemm128 override n={n}", flush=True)
    with _tune.override(gemm128_min_mn=128, gemm128_min_k=64, gemm128_tout=1):
        inv = fermix_amd._kernels.slogdet_parts(At, x3=0)[2]
        sinv = fermix_amd._kernels.slogpf_parts(S, False, x3=0)[2]
    assert torch.equal(inv, ref_inv)
    assert torch.equal(sinv, ref_sinv)
    # bf16x3: the table's 128 x 128 tiles (operands split once in LDS) against 64 x 64
    # tiles (split at every use): the same split values and products, the same bits
    ref3 = fermix_amd._kernels.slogdet_parts(At, x3=1)[2]
    ref3s = fermix_amd._kernels.slogpf_parts(S, False, x3=1)[2]
    with _tune.override(gemm128_x3_min_mn=1 << 20, gemm128_x3_tout=0):
        inv3 = fermix_amd._kernels.slogdet_parts(At, x3=1)[2]
        sinv3 = fermix_amd._kernels.slogpf_parts(S, False, x3=1)[2]
    assert torch.equal(inv3, ref3)
    assert torch.equal(sinv3, ref3s)


@pytest.mark.parametrize("n,override", [(1024, dict(pf_block64_max_m=0)), (256, dict(pf_block64_min_n=256)),
                                        (512, dict(pf_block64_max_m=256))])
def test_pf_block_width_override(dev, n, override):
    """Parlett-Reid with 32-column blocks only, with 64-column blocks at N = 256, and with
    the switch moved to m = 256: values against float64 and S^-1 against float64."""
    A = _mats(n, 3, 7400 + n)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    St = _t(S, dev)
    print(f"pf block override n={n} {override}", flush=True)
    with _tune.override(**override):
        s, l = map(_np, fermix_amd.slogpf(St, skew_symmetrize=False))
        X = St.clone().requires_grad_(True)
        s2, l2 = fermix_amd.slogpf(X, skew_symmetrize=False)
        (g,) = torch.autograd.grad(l2.sum(), X)
    s64, l64 = ref64.slogpf64(S)
    assert np.array_equal(s, s64)
    assert np.array_equal(_np(s2), s) and np.array_equal(_np(l2), l)
    assert_logabs(l, l64, n, f"pf {override}", S)
    # d logabs / dS = S^-T / 2 for skew_symmetrize=False
    ref = 0.5 * np.linalg.inv(S.astype(np.float64)).transpose(0, 2, 1)
    assert_grad(_np(g), ref, S, f"pf {override} grad")


@pytest.mark.parametrize("n", [80, 100, 128])
def test_fused_max_override(dev, n):
    """fused_max_n = 64 sends 64 < n <= 128 to the blocked kernels: slogdet / slogpf values
    and gradients against float64."""
    A = _mats(n, 8, 7500 + n)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    print(f"fused_max override n={n}", flush=True)
    with _tune.override(fused_max_n=64):
        assert _tune.kernel_family(n) == "blocked"
        X = _t(A, dev).requires_grad_(True)
        s, l = fermix_amd.slogdet(X)
        (g,) = torch.autograd.grad(l.sum(), X)
        ps, pl = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(_np(s), s64)
    assert_logabs(_np(l), l64, n, "blocked via override", A)
    assert_grad(_np(g), np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1), A, "blocked via override grad")
    ps64, pl64 = ref64.slogpf64(S)
    assert np.array_equal(ps, ps64)
    assert_logabs(pl, pl64, n, "pf blocked via override", S)


@pytest.mark.parametrize("n", [40, 100])
def test_f64_override(dev, n):
    """float64 through the LDS / workspace kernel (f64_reg_max_n lowered) and with
    32-column register strips (f64_strip16_max_n = 0): values and A^-T against numpy's
    float64, S^-1 against numpy's float64 inverse."""
    rng = np.random.default_rng(7600 + n)
    A = rng.standard_normal((4, n, n)) / np.sqrt(n)
    S = A - A.transpose(0, 2, 1)
    print(f"f64 override n={n}", flush=True)
    for ov in (dict(f64_reg_max_n=min(32, n - 1)), dict(f64_strip16_max_n=0)):
        with _tune.override(**ov):
            X = _t(A, dev).requires_grad_(True)
            s, l = fermix_amd.slogdet(X)
            (g,) = torch.autograd.grad(l.sum(), X)
            ps, pl = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
        s64, l64 = np.linalg.slogdet(A)
        assert np.array_equal(_np(s), s64), ov
        assert_logabs64(_np(l), l64, n, f"f64 {ov}", A)
        inv = np.linalg.inv(A).transpose(0, 2, 1)
        assert np.max(np.abs(_np(g) - inv)) / np.max(np.abs(inv)) < 1e-10, ov
        pl64 = 0.5 * np.linalg.slogdet(S)[1]
        assert np.all(np.abs(pl - pl64) < 1e-9 * np.maximum(1, np.abs(pl64))), ov


def _vals_and_grad(fn, A):
    X = A.clone().requires_grad_(True)
    s, l = fn(X)
    (g,) = torch.autograd.grad(l.sum(), X)
    return s.detach(), l.detach(), g


@pytest.mark.parametrize("n,B", [(300, 5), (640, 8), (1100, 3)])
def test_lu_split_halves_bit_identical(dev, n, B):
    """The LU's two batch halves on two streams (lu_split_min_work) give the unsplit bits:
    values and A^-T, odd batches (unequal halves) included; and meet the float64 bar."""
    A = _mats(n, B, 7400 + n)
    At = _t(A, dev)
    print(f"lu split n={n} B={B}", flush=True)
    with _tune.override(lu_split_min_work=0):
        ref = _vals_and_grad(fermix_amd.slogdet, At)
    with _tune.override(lu_split_min_work=1):
        out = _vals_and_grad(fermix_amd.slogdet, At)
    for a, b in zip(ref, out):
        assert torch.equal(a, b)
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(_np(out[0]), s64)
    assert_logabs(_np(out[1]), l64, n, "split", A)


@pytest.mark.parametrize("n,B", [(1100, 3), (2100, 3), (4200, 2)])
def test_pf_overlap_halves_bit_identical(dev, n, B):
    """The Parlett-Reid halves with one half's panels beside the other half's update in each
    launch (pf_overlap_*: 32-, 16- and 8-column blocks, N <= 2048 / 4096 / above) give the
    unsplit bits: values, and S^-1 through the gradient; odd batches (unequal halves)
    included; values against float64 (log|pf| = log|det| / 2)."""
    A = _mats(n, B, 7500 + n)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    St = _t(S, dev)
    print(f"pf overlap n={n} B={B}", flush=True)
    with _tune.override(pf_overlap_max_half=0):
        ref = _vals_and_grad(lambda X: fermix_amd.slogpf(X), St)
    with _tune.override(pf_overlap_max_half=1 << 20, pf_overlap_min_work=0):
        out = _vals_and_grad(lambda X: fermix_amd.slogpf(X), St)
    for a, b in zip(ref, out):
        assert torch.equal(a, b)
    _, l64 = ref64.slogdet64(S)
    assert_logabs(_np(out[1]), 0.5 * l64, n, "overlap", S)
