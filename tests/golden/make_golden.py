"""Write tests/golden/golden.npz: seeded float32 inputs with float64 expected values.

The reference (ChenAo-Phys/fermix) ships no golden vectors: its tests compute the
expected values on the fly in float64 (tests/test_fermix.py:95-144, 148-193). This
script records the same kind of known answers once, as data, so the CPU oracle and the
GPU kernels are checked against fixed vectors:

* slogdet: numpy's float64 LAPACK slogdet of the float32 inputs (the reference's own
  expected value, test_fermix.py:153-155), A^-T from the float64 inverse;
* slogpf: float64 Parlett-Reid of the float32 skew inputs (the reference's pf_ref64,
  test_fermix.py:95-116), cross-checked here against the brute-force perfect-matching
  Pfaffian for n <= 10; S^-1 from the float64 inverse;
* singular members: an exactly zero column (slogdet) / zero row and column (slogpf),
  expected (0, -inf) (test_fermix.py:442-456).

Run from the repository root: ``python tests/golden/make_golden.py``.
"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import ref64  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def main():
    rng = np.random.default_rng(20261201)
    data = {}
    for n, B in [(3, 5), (8, 5), (17, 4), (40, 4), (96, 3), (128, 2)]:
        A = rng.standard_normal((B, n, n)).astype(np.float32)
        if n >= 8:
            A[0, :, n // 3] = 0.0  # exactly singular member
        s, l = ref64.slogdet64(A)
        data[f"det_n{n}_a"] = A
        data[f"det_n{n}_sign"] = s
        data[f"det_n{n}_logabs"] = l
        if n <= 40:
            inv = np.zeros((B, n, n))
            for b in range(B):
                if s[b] != 0:
                    inv[b] = np.linalg.inv(A[b].astype(np.float64)).T
            data[f"det_n{n}_invT"] = inv
    for n, B in [(4, 5), (6, 5), (10, 4), (34, 4), (64, 3), (128, 2)]:
        A = rng.standard_normal((B, n, n)).astype(np.float32)
        S = (A - np.swapaxes(A, 1, 2)).astype(np.float32)
        if n >= 10:
            S[0, n // 2, :] = 0.0
            S[0, :, n // 2] = 0.0
        s, l = ref64.slogpf64(S)
        if n <= 10:
            brute = np.array([ref64.pf_brute(x) for x in S])
            pr = s * np.exp(l)
            assert np.allclose(brute, pr, rtol=1e-9, atol=1e-12), (brute, pr)
        data[f"pf_n{n}_s"] = S
        data[f"pf_n{n}_sign"] = s
        data[f"pf_n{n}_logabs"] = l
        if n <= 34:
            inv = np.zeros((B, n, n))
            for b in range(B):
                if s[b] != 0:
                    inv[b] = np.linalg.inv(S[b].astype(np.float64))
            data[f"pf_n{n}_sinv"] = inv
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
