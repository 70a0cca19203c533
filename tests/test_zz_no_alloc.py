"""GPU check of fx_slogdet_f32_noalloc through the C ABI: bit-identical to fx_slogdet_f32
(with a caller workspace) on two calls in a row, the second with a smaller input, so the
second runs on the scratch array as the first left it; then a batch that needs several
sub-batches of the scratch array, and an n <= 128 call (no workspace at all)."""

import numpy as np
import pytest
import torch

from fermix_amd import _lib

pytestmark = pytest.mark.gpu


def _call_pair(dev, A):
    L = _lib.lib()
    B, n, _ = A.shape
    stream = torch.cuda.current_stream(dev).cuda_stream or None
    s0 = torch.empty(B, device=dev)
    l0 = torch.empty(B, device=dev)
    nb = L.fx_slogdet_f32_workspace(B, n)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
    st = L.fx_slogdet_f32(A.data_ptr(), B, n, s0.data_ptr(), l0.data_ptr(), 0, ws.data_ptr() if nb else None, nb,
                          stream)
    assert st == 0, st
    s1 = torch.full((B,), 7.0, device=dev)
    l1 = torch.full((B,), 7.0, device=dev)
    st = L.fx_slogdet_f32_noalloc(A.data_ptr(), B, n, s1.data_ptr(), l1.data_ptr(), stream)
    assert st == 0, st
    torch.cuda.synchronize(dev)
    return s0, l0, s1, l1


# (7, 2049): 3 members per sub-batch, so the second and third sub-batches of this odd
# order start 4-byte aligned only
@pytest.mark.parametrize("first,second", [((96, 700), (40, 300)), ((24, 2048), (5, 129)), ((7, 2049), (3, 1501))])
def test_noalloc_matches_workspace_entry_point(dev, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for B, n in (first, second):
        print(f"noalloc slogdet B={B} n={n}", flush=True)
        A = torch.from_numpy((rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)).to(dev)
        A[B // 2, :, n // 3] = 0.0  # an exactly singular member
        s0, l0, s1, l1 = _call_pair(dev, A)
        assert torch.equal(s0, s1) and torch.equal(l0, l1), (B, n)
        assert float(s1[B // 2]) == 0.0 and float(l1[B // 2]) == float("-inf")
        assert bool(torch.all(s1[torch.arange(B, device=dev) != B // 2].abs() == 1))


def test_noalloc_small_n_and_limits(dev):
    rng = np.random.default_rng(5)
    A = torch.from_numpy(rng.standard_normal((64, 100, 100)).astype(np.float32)).to(dev)
    s0, l0, s1, l1 = _call_pair(dev, A)
    assert torch.equal(s0, s1) and torch.equal(l0, l1)
    L = _lib.lib()
    x = torch.empty(16, device=dev)
    assert L.fx_slogdet_f32_noalloc(x.data_ptr(), 1, 4096, x.data_ptr(), x.data_ptr(), None) == 4
