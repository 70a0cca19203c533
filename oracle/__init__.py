"""CPU oracle for the fermix_amd hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, on the CPU, the algorithm of the reference's generic path
(ChenAo-Phys/fermix ``src/fermix/_fallback.py``, ``_diff.py``, ``_poly.py``) so that the
HIP kernels in ``fermix_amd`` can be checked against it. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it,
and only as the checker (or the timed CPU baseline) -- never as the thing measured on
the GPU, and never as a fallback of the product path.

Modules:

* ``generic`` -- the reference's generic path restated in numpy (dtype preserving:
  float32 inputs compute in float32). The LU itself is the third-party routine the
  reference's generic path calls on the CPU (``lax.linalg.lu`` -> LAPACK ``?getrf``,
  which jaxlib takes from ``scipy.linalg.cython_lapack``), called here through
  ``scipy.linalg.lapack``; the triangular solves are LAPACK ``?trtrs`` through
  ``scipy.linalg.solve_triangular``.
* ``ref64`` -- float64 truth from the mathematics (numpy LAPACK, brute-force perfect
  matchings, cofactors, minor Pfaffians) used to pin ``generic``.

Parity pinning (what checks each function; tests/test_oracle.py):

* slogdet_generic: float64 ``np.linalg.slogdet``, permutation matrices (exact sign,
  logabs 0), triangular matrices (sign and sum of logs of the diagonal), exactly
  singular inputs -> (0, -inf), the golden fixtures.
* slogpf_generic: brute-force perfect-matching Pfaffian (n <= 10), pf^2 = det,
  pf(B S B^T) = det(B) pf(S), pf of a direct sum of 2x2 blocks, zero row -> (0, -inf).
* lu_parts_generic: float64 inverse, central finite differences of log|det|, singular
  members -> zero gradient.
* pf_parts_generic: float64 inverse (inverse mode) and brute-force minor Pfaffians
  (adjugate mode, including rank n-2 inputs with one and two exact zero pivots).
* det_gradT: brute-force cofactor adjugate on regular, rank n-1 and rank n-2 inputs.
* det_poly / pf_poly: float64 LAPACK det / brute-force Pfaffian.

No function is "parity unpinned".
"""
