"""GPU checks of two rules of the C ABI's boundary (include/fermix.h):

* batches beyond one grid chunk (65528 members) run in consecutive chunks, and every
  member's result is the one it gets in a call of its own (the kernels are per matrix,
  so bit-identical), on both sides of each chunk edge;
* misaligned views (a batch sliced at an odd member offset of an odd-n batch) are copied
  to aligned memory by the Python layer and give the aligned call's results bitwise.
"""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from tests.tolerances import assert_grad

pytestmark = pytest.mark.gpu

CHUNK = 65528


def _edges(B):
    """Member indices around the chunk edges of a batch of B."""
    idx = [0, 1, CHUNK - 2, CHUNK - 1, CHUNK, CHUNK + 1, B - 1]
    return sorted(set(i for i in idx if 0 <= i < B))


@pytest.mark.parametrize("n", [129, 64])
def test_slogdet_beyond_one_chunk(dev, n):
    B = CHUNK + 24
    print(f"slogdet chunked n={n} B={B}", flush=True)
    g = torch.Generator(device=dev).manual_seed(11)
    A = torch.randn((B, n, n), device=dev, generator=g) / n**0.5
    s, l = fermix_amd.slogdet(A)
    idx = _edges(B)
    s1, l1 = fermix_amd.slogdet(A[idx].contiguous())
    assert torch.equal(s[idx], s1) and torch.equal(l[idx], l1)
    if n == 64:
        # the inverse (batch on gridDim.y in its diagonal-block kernel)
        s2, l2, invT, _, _ = _kernels.slogdet_parts(A)
        assert torch.equal(s2, s) and torch.equal(l2, l)
        _, _, inv1, _, _ = _kernels.slogdet_parts(A[idx].contiguous())
        assert torch.equal(invT[idx], inv1)
    del A
    torch.cuda.empty_cache()


def test_slogpf_parts_beyond_one_chunk(dev):
    n = 64
    B = CHUNK + 16
    print(f"slogpf parts chunked n={n} B={B}", flush=True)
    g = torch.Generator(device=dev).manual_seed(12)
    A = torch.randn((B, n, n), device=dev, generator=g) / n**0.5
    s, l, G = _kernels.slogpf_parts(A, True)
    idx = _edges(B)
    s1, l1, G1 = _kernels.slogpf_parts(A[idx].contiguous(), True)
    assert torch.equal(s[idx], s1) and torch.equal(l[idx], l1) and torch.equal(G[idx], G1)
    del A, G
    torch.cuda.empty_cache()


@pytest.mark.parametrize("n", [129, 33])
def test_misaligned_views(dev, n):
    """A[1:] of an odd-n batch starts 4 bytes past a 16-byte boundary (n * n * 4 = 4 mod
    16): the API copies it to aligned memory; the results equal the aligned call's."""
    rng = np.random.default_rng(31 + n)
    A = torch.from_numpy((rng.standard_normal((5, n, n)) / np.sqrt(n)).astype(np.float32)).to(dev)
    V = A[1:]
    assert V.data_ptr() % 16 == 4
    W = V.clone()
    assert W.data_ptr() % 16 == 0
    for f in (fermix_amd.slogdet, fermix_amd.slogpf):
        sv, lv = f(V)
        sw, lw = f(W)
        assert torch.equal(sv, sw) and torch.equal(lv, lw), f.__name__
    Vg = V.detach().clone()  # autograd through an aligned leaf, compared with a view's grad
    Ag = A.clone().requires_grad_()
    _, l = fermix_amd.slogdet(Ag[1:])
    (gv,) = torch.autograd.grad(l.sum(), Ag)
    _, _, invT, _, _ = _kernels.slogdet_parts(Vg)
    assert torch.equal(gv[1:], invT) and torch.all(gv[0] == 0)
    ref = np.linalg.inv(Vg.cpu().numpy().astype(np.float64)).transpose(0, 2, 1)
    assert_grad(invT.cpu().numpy(), ref, Vg.cpu().numpy(), f"misaligned view n={n}")
