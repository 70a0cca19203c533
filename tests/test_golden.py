"""The CPU oracle against the committed golden vectors (tests/golden/golden.npz)."""

import numpy as np
import pytest

from oracle import generic as g
from tests.tolerances import assert_logabs, rel_fro

DET_N = [3, 8, 17, 40, 96, 128]
PF_N = [4, 6, 10, 34, 64, 128]


@pytest.mark.parametrize("n", DET_N)
def test_oracle_slogdet_golden(golden, n):
    A = golden[f"det_n{n}_a"]
    s, l = g.slogdet_generic(A)
    assert np.array_equal(s, golden[f"det_n{n}_sign"])
    assert_logabs(l, golden[f"det_n{n}_logabs"], n, "oracle golden", A)
    if f"det_n{n}_invT" in golden:
        _, _, invT, _, _, _ = g.lu_parts_generic(A)
        ref = golden[f"det_n{n}_invT"]
        ok = golden[f"det_n{n}_sign"] != 0
        assert np.all(rel_fro(invT[ok], ref[ok]) < 1e-4)
        assert np.all(invT[~ok] == 0)


@pytest.mark.parametrize("n", PF_N)
def test_oracle_slogpf_golden(golden, n):
    S = golden[f"pf_n{n}_s"]
    s, l = g.slogpf_generic(S)
    assert np.array_equal(s, golden[f"pf_n{n}_sign"])
    assert_logabs(l, golden[f"pf_n{n}_logabs"], n, "oracle golden", S)
    if f"pf_n{n}_sinv" in golden:
        _, _, Sinv, _ = g.pf_parts_generic(S, False)
        ref = golden[f"pf_n{n}_sinv"]
        ok = golden[f"pf_n{n}_sign"] != 0
        assert np.all(rel_fro(Sinv[ok], ref[ok]) < 1e-4)
        assert np.all(Sinv[~ok] == 0)
