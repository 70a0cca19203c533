"""Every order of the one-workgroup kernels (n = 1 ... 128): slogdet, slogpf (odd n
included, where pf = 0) and the skew-symmetrising slogpf, each against float64 truth
and the CPU oracle's signs on a small seeded batch, and the gradients' inverses (A^-T,
S^-1) against float64 inverses. The kernels are instantiated per 16-padded size and
load ragged orders with masking, so each n is its own case; the reference's tests
sample a few orders (tests/test_fermix.py:148-228)."""

import numpy as np
import pytest
import torch

import fermix_amd
from fermix_amd import _kernels
from oracle import generic as g
from oracle import ref64
from tests.tolerances import assert_grad, assert_logabs

pytestmark = pytest.mark.gpu

B = 6


def _np(x):
    return x.detach().cpu().numpy()


def test_slogdet_every_n(dev):
    for n in range(1, 129):
        rng = np.random.default_rng(7000 + n)
        A = rng.standard_normal((B, n, n)).astype(np.float32)
        print(f"slogdet n={n} B={B}", flush=True)
        s, l = map(_np, fermix_amd.slogdet(torch.from_numpy(A).to(dev)))
        s64, l64 = ref64.slogdet64(A)
        so, _ = g.slogdet_generic(A)
        assert np.array_equal(s, s64), n
        assert np.array_equal(s, so), n
        assert_logabs(l, l64, n, f"slogdet n={n} vs float64", A)


def test_slogpf_every_n(dev):
    for n in range(1, 129):
        rng = np.random.default_rng(8000 + n)
        X = rng.standard_normal((B, n, n)).astype(np.float32)
        S = (X - np.swapaxes(X, -1, -2)).astype(np.float32)
        print(f"slogpf n={n} B={B}", flush=True)
        s, l = map(_np, fermix_amd.slogpf(torch.from_numpy(S).to(dev), skew_symmetrize=False))
        if n % 2:
            # odd order: pf = 0
            assert np.all(s == 0) and np.all(np.isneginf(l)), n
            continue
        s64, l64 = ref64.slogpf64(S)
        so, _ = g.slogpf_generic(S)
        assert np.array_equal(s, s64), n
        assert np.array_equal(s, so), n
        assert_logabs(l, l64, n, f"slogpf n={n} vs float64", S)


def test_slogpf_skew_symmetrize_every_even_n(dev):
    # skew_symmetrize=True reads A and forms (A - A^T) / 2 while loading
    for n in range(2, 129, 2):
        rng = np.random.default_rng(9000 + n)
        A = rng.standard_normal((B, n, n)).astype(np.float32)
        S = ((A - np.swapaxes(A, -1, -2)) / 2).astype(np.float32)
        print(f"slogpf skew n={n} B={B}", flush=True)
        s, l = map(_np, fermix_amd.slogpf(torch.from_numpy(A).to(dev), skew_symmetrize=True))
        s64, l64 = ref64.slogpf64(S)
        assert np.array_equal(s, s64), n
        assert_logabs(l, l64, n, f"slogpf skew n={n} vs float64", S)


def test_slogdet_inverse_every_n(dev):
    for n in range(1, 129):
        rng = np.random.default_rng(10000 + n)
        A = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
        print(f"invT n={n} B={B}", flush=True)
        At = torch.from_numpy(A).to(dev)
        s, l, invT, _, _ = _kernels.slogdet_parts(At)
        s0, l0 = fermix_amd.slogdet(At)
        assert torch.equal(s, s0) and torch.equal(l, l0), f"n={n}: parts primal != forward"
        ref = np.linalg.inv(A.astype(np.float64)).transpose(0, 2, 1)
        assert_grad(_np(invT), ref, A, f"invT n={n} vs float64")


def test_slogpf_inverse_every_even_n(dev):
    for n in range(2, 129, 2):
        rng = np.random.default_rng(11000 + n)
        X = (rng.standard_normal((B, n, n)) / np.sqrt(n)).astype(np.float32)
        S = (X - np.swapaxes(X, -1, -2)).astype(np.float32)
        print(f"Sinv n={n} B={B}", flush=True)
        St = torch.from_numpy(S).to(dev)
        s, l, Sinv = _kernels.slogpf_parts(St, False)
        s0, l0 = fermix_amd.slogpf(St, skew_symmetrize=False)
        assert torch.equal(s, s0) and torch.equal(l, l0), f"n={n}: parts primal != forward"
        assert_grad(_np(Sinv), np.linalg.inv(S.astype(np.float64)), S, f"Sinv n={n} vs float64")
