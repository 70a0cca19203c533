"""BASELINE configs[4], the singular-mix stress: B = 2048, n = 256.

* slogdet on A iid N(0, 1): a quarter of the members made rank deficient by the literal
  recipe (column j replaced by column j+1 + column j+2, singular only to float32
  round-off: the contract is a finite forward and gradient, no NaN / inf), a quarter
  exactly singular (a zero column: (0, -inf) and a zero gradient), the rest regular
  (parity with float64);
* slogpf on S = A - A^T with a quarter having row / column i zeroed: (0, -inf), zero
  gradient, finite everywhere.
(The reference's own singular tests: tests/test_fermix.py:442-456, 484-545.)"""

import numpy as np
import pytest
import torch

import fermix_amd
from oracle import ref64
from tests.tolerances import assert_logabs

pytestmark = pytest.mark.gpu

B, n = 2048, 256


def _t(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _np(x):
    return x.detach().cpu().numpy()


def test_c5_slogdet_singular_mix(dev):
    rng = np.random.default_rng(5)
    A = rng.standard_normal((B, n, n), dtype=np.float32)
    q = B // 4
    js = rng.integers(0, n - 2, size=q)
    for b in range(q):  # literal recipe: near singular
        j = js[b]
        A[b, :, j] = A[b, :, j + 1] + A[b, :, j + 2]
    for b in range(q, 2 * q):  # exactly singular
        A[b, :, (b * 7) % n] = 0.0
    At = _t(A, dev).requires_grad_()
    s, l = fermix_amd.slogdet(At)
    (gr,) = torch.autograd.grad(l[torch.isfinite(l)].sum(), At)
    s, l, gr = _np(s), _np(l), _np(gr)
    assert not np.any(np.isnan(l)) and np.all(np.isfinite(gr))
    assert np.all(s[q : 2 * q] == 0) and np.all(np.isneginf(l[q : 2 * q]))
    assert np.all(gr[q : 2 * q] == 0)
    assert np.all(np.abs(s[:q]) <= 1) and np.all(np.isfinite(l[:q]) | np.isneginf(l[:q]))
    s64, l64 = ref64.slogdet64(A[2 * q :])
    assert np.array_equal(s[2 * q :], s64)
    assert_logabs(l[2 * q :], l64, n, "C5 regular vs float64", A[2 * q :])
    print(f"C5 near-singular members: {int(np.isneginf(l[:q]).sum())} exact zero pivots, "
          f"min logabs {float(np.min(l[:q][np.isfinite(l[:q])])):.1f}", flush=True)


def test_c5_slogpf_singular_mix(dev):
    rng = np.random.default_rng(6)
    A = rng.standard_normal((B, n, n), dtype=np.float32)
    S = A - A.transpose(0, 2, 1)
    del A
    q = B // 4
    for b in range(q):
        i = (b * 13) % n
        S[b, i, :] = 0.0
        S[b, :, i] = 0.0
    St = _t(S, dev).requires_grad_()
    s, l = fermix_amd.slogpf(St, skew_symmetrize=False)
    (gr,) = torch.autograd.grad(l[torch.isfinite(l)].sum(), St)
    s, l, gr = _np(s), _np(l), _np(gr)
    assert np.all(np.isfinite(gr))
    assert np.all(s[:q] == 0) and np.all(np.isneginf(l[:q])) and np.all(gr[:q] == 0)
    s64, l64 = ref64.slogpf64(S[q : q + 64])
    assert np.array_equal(s[q : q + 64], s64)
    assert_logabs(l[q : q + 64], l64, n, "C5 pf regular vs float64", S[q : q + 64])
