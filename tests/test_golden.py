"""The committed golden fixtures still match the oracle (guards both against drift)."""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_q8k_golden():
    g = np.load(os.path.join(GOLDEN, "q8k_vectors.npz"))
    np.testing.assert_array_equal(O.quantize_row_q8_K(g["x"]).reshape(g["q8"].shape), g["q8"])


@pytest.mark.parametrize("name,ty", [("q4_K", O.TYPE_Q4_K), ("q6_K", O.TYPE_Q6_K)])
def test_gemv_golden(name, ty):
    g = np.load(os.path.join(GOLDEN, f"gemv_{name}.npz"))
    k, n = int(g["k"]), int(g["n"])
    y = O.mul_mat(ty, g["w"], k, n, g["x"])[0]
    np.testing.assert_array_equal(y, g["y"])
    assert np.all(np.abs(g["y"] - g["ref"]) <= g["bound"])


@pytest.mark.parametrize("name,ty", [("q4_K", O.TYPE_Q4_K), ("q6_K", O.TYPE_Q6_K)])
def test_mmid_golden(name, ty):
    g = np.load(os.path.join(GOLDEN, f"mmid_{name}.npz"))
    y = O.mul_mat_id(ty, g["w"], int(g["k"]), int(g["n"]), int(g["E"]), g["b"], g["ids"])
    np.testing.assert_array_equal(y, g["y"])
    assert np.all(g["y"][g["ids"] < 0] == 0)
