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


@pytest.mark.parametrize("n", [129, 160, 192, 200, 256, 300, 384, 512, 640, 1000, 1024])
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
