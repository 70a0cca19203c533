"""GPU parity of the blocked large-n paths (128 < n <= 1024) against the CPU oracle
and float64 truth: slogdet forward (and, below, the gradients)."""

import numpy as np
import pytest
import torch

import fermix_amd
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_logabs

pytestmark = pytest.mark.gpu


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


@pytest.mark.parametrize("n", [129, 160, 192, 200, 256, 300, 320, 384, 448, 512, 640, 1000, 1024])
def test_slogdet_large_vs_oracle(dev, n):
    B = 16 if n <= 512 else 6
    rng = np.random.default_rng(1000 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    if B > 3:
        A[1, :, n // 2] = 0.0
    print(f"slogdet large n={n} B={B}", flush=True)
    s, l = map(_np, fermix_amd.slogdet(_t(A, dev)))
    s64, l64 = ref64.slogdet64(A)
    so, lo = g.slogdet_generic(A)
    assert np.array_equal(s, s64)
    assert np.array_equal(s, so)
    assert_logabs(l, l64, n, "vs float64", A)
    assert_logabs(l, lo, n, "vs oracle", A)


@pytest.mark.parametrize("n", [130, 160, 256, 300, 512, 1000, 1024, 2048])
def test_slogpf_large_vs_oracle(dev, n):
    B = 8 if n <= 512 else 3
    rng = np.random.default_rng(4000 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    if B > 3:
        S[1, n // 3, :] = 0.0
        S[1, :, n // 3] = 0.0
    print(f"slogpf large n={n} B={B}", flush=True)
    s, l = map(_np, fermix_amd.slogpf(_t(S, dev), skew_symmetrize=False))
    s64, l64 = ref64.slogpf64(S)
    assert np.array_equal(s, s64)
    assert_logabs(l, l64, n, "vs float64", S)
    if n <= 512:
        so, lo = g.slogpf_generic(S)
        assert np.array_equal(s, so)
        assert_logabs(l, lo, n, "vs oracle", S)
    # pf^2 = det against the slogdet kernels where they exist
    if n <= 1024:
        sd, ld = map(_np, fermix_amd.slogdet(_t(S, dev)))
        fin = np.isfinite(l64)
        assert np.all(np.abs(2 * l[fin] - ld[fin]) < 1e-3 * np.maximum(1, np.abs(ld[fin])) + 1e-3)


@pytest.mark.parametrize("n", [192, 512, 1024, 1536])
def test_no_row_moves(dev, n):
    """Column-diagonally-dominant matrices: the diagonal entry is the largest of its column
    throughout the elimination, so no panel moves a row and every row-permutation step
    runs with an empty move list. slogdet and A^-T against float64."""
    from fermix_amd import _kernels
    from tests.tolerances import assert_grad

    B = 3
    rng = np.random.default_rng(6000 + n)
    A = (rng.standard_normal((B, n, n)) / n).astype(np.float32) + np.float32(4.0) * np.eye(n, dtype=np.float32)
    print(f"no row moves n={n}", flush=True)
    s, l, invT, _, _ = _kernels.slogdet_parts(_t(A, dev))
    s0, l0 = fermix_amd.slogdet(_t(A, dev))
    assert torch.equal(s, s0) and torch.equal(l, l0)
    s64, l64 = ref64.slogdet64(A)
    assert np.array_equal(_np(s), s64)
    assert_logabs(_np(l), l64, n, "vs float64", A)
    ref = np.linalg.inv(A.astype(np.float64)).swapaxes(-1, -2)
    assert_grad(_np(invT), ref, A, f"n={n} A^-T vs float64")


@pytest.mark.parametrize("n", [160, 512, 1056, 2080])
def test_slogpf_first_block_paths_agree(dev, n):
    """The blocked Parlett-Reid keeps the trailing matrix as its lower triangle in 4-row
    strips. With skew_symmetrize=False and n a multiple of 32 the first block reads the
    full-storage input in place of a copy (its update gathering the old entries through
    the permutation); with skew_symmetrize=True the input is first copied into the strip
    layout ((S - S^T) / 2 = S exactly for an exactly skew S, so both runs factor the same
    numbers). The two runs must agree bit for bit, in the forward and in the factors of
    the gradient route; n covers 32- and 64-column blocks and the 16-column blocks above
    2048."""
    from fermix_amd import _kernels

    B = 4 if n <= 1056 else 2
    rng = np.random.default_rng(9100 + n)
    A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
    S = (A - A.transpose(0, 2, 1)).astype(np.float32)
    S[0, 3, :] = 0.0  # an exactly singular member: (0, -inf) on both paths
    S[0, :, 3] = 0.0
    print(f"slogpf first-block paths n={n} B={B}", flush=True)
    St = _t(S, dev)
    s1, l1 = fermix_amd.slogpf(St, skew_symmetrize=False)
    s2, l2 = fermix_amd.slogpf(St, skew_symmetrize=True)
    assert torch.equal(s1, s2) and torch.equal(l1, l2)
    assert _np(s1)[0] == 0 and np.isneginf(_np(l1)[0])
    sp1, lp1, G1 = _kernels.slogpf_parts(St, False)
    sp2, lp2, G2 = _kernels.slogpf_parts(St, True)
    assert torch.equal(sp1, s1) and torch.equal(lp1, l1)
    assert torch.equal(sp2, s2) and torch.equal(lp2, l2)
    assert torch.equal(G1, G2)
    s64, l64 = ref64.slogpf64(S[1:])
    assert np.array_equal(_np(s1)[1:], s64)
    assert_logabs(_np(l1)[1:], l64, n, "vs float64", S[1:])
