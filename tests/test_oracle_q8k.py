"""Pins the oracle's Q8_K quantizer (orc_quantize_row_q8_K) to ggml's quantize_row_q8_K_ref.

ggml is not in the reference checkout (vendor/llama.cpp is an empty submodule, vendor/PIN:1-2), and
no reference test commits Q8_K bytes. The checks below fix the algorithm from what the mathematics
and the published rule leave no room for: blocks whose scale is exactly representable (so every byte
is known by hand), round-half-even ties, the first-occurrence argmax, the all-zero block, the bsums
and reconstruction invariants, and d = 1/iscale (not max/-127).
"""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import oracle as O

TIES = [(0.5, 0), (1.5, 2), (2.5, 2), (3.5, 4), (-0.5, 0), (-1.5, -2), (-2.5, -2), (126.5, 126), (-126.5, -126),
        (125.5, 126), (10.0, 10), (-99.0, -99), (127.0, 127)]


def _block(x):
    b = O.quantize_row_q8_K(np.asarray(x, dtype=np.float32)).view(O.BLOCK_Q8_K)
    return b[0] if b.shape == (1,) else b


def _hand_block(scale):
    """x[0] = -127*scale is the largest |x|; iscale = -127/(-127*scale) = 1/scale exactly for
    scale in {1, 2, 0.5}; the other elements are the tie cases times scale."""
    x = np.zeros(256, dtype=np.float32)
    want = np.zeros(256, dtype=np.int64)
    x[0], want[0] = -127.0 * scale, -127
    for i, (v, q) in enumerate(TIES, start=1):
        x[7 * i] = v * scale
        want[7 * i] = q
    return x, want


@pytest.mark.parametrize("scale", [1.0, 2.0, 0.5])
def test_exact_scale_known_answer(scale):
    x, want = _hand_block(scale)
    b = _block(x)
    assert b["d"] == np.float32(scale)  # d = 1/iscale = 1/(1/scale)
    np.testing.assert_array_equal(b["qs"].astype(np.int64), want)
    np.testing.assert_array_equal(b["bsums"].astype(np.int64), want.reshape(16, 16).sum(axis=1))


def test_first_max_wins_ties_of_abs():
    """+3 at index 5 and -3 at index 9 have the same |x|: the first one is the max, so it maps to
    -127 and the later one to +127 (a last-occurrence rule gives the opposite signs)."""
    x = np.zeros(256, dtype=np.float32)
    x[5], x[9], x[100] = 3.0, -3.0, 1.0
    b = _block(x)
    assert b["qs"][5] == -127 and b["qs"][9] == 127
    assert b["d"] < 0
    assert b["qs"][100] == -42  # nearest(-127/3 * 1) = nearest(-42.333...)


def test_d_is_reciprocal_of_iscale():
    """d is 1/iscale with iscale = -127/max, both fp32; for max = 11 this differs from max/-127."""
    x = np.zeros(256, dtype=np.float32)
    x[0] = 11.0
    b = _block(x)
    iscale = np.float32(-127.0) / np.float32(11.0)
    assert b["d"] == np.float32(1.0) / iscale
    assert np.float32(1.0) / iscale != np.float32(11.0) / np.float32(-127.0)


def test_all_zero_block():
    b = _block(np.zeros(256, dtype=np.float32))
    assert b["d"] == 0.0
    assert not b["qs"].any()
    assert not b["bsums"].any()  # ggml leaves them unwritten; this build writes zeros


def test_negative_zero_is_zero_block():
    b = _block(np.full(256, -0.0, dtype=np.float32))
    assert b["d"] == 0.0 and not b["qs"].any()


def test_blocks_are_independent():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256 * 5).astype(np.float32)
    x[256:512] = 0
    whole = O.quantize_row_q8_K(x)
    parts = np.concatenate([O.quantize_row_q8_K(x[256 * i:256 * (i + 1)]) for i in range(5)])
    np.testing.assert_array_equal(whole, parts)


# |x| in [1e-20, 1e20] or 0: iscale = -127/max stays finite (for max below 127/FLT_MAX it overflows, in
# ggml as here, and the bytes are meaningless).
_LO, _HI = float(np.float32(1e-20)), float(np.float32(1e20))
finite = st.one_of(st.just(0.0), st.floats(min_value=_LO, max_value=_HI, width=32),
                   st.floats(min_value=-_HI, max_value=-_LO, width=32))


@settings(max_examples=200, deadline=None)
@given(st.lists(finite, min_size=256, max_size=256))
def test_invariants(xs):
    x = np.asarray(xs, dtype=np.float32)
    b = _block(x)
    amax = np.abs(x).max()
    qs = b["qs"].astype(np.int64)
    if amax == 0:
        assert b["d"] == 0 and not qs.any()
        return
    i = int(np.argmax(np.abs(x)))  # numpy's argmax returns the first of equal maxima
    assert qs[i] == -127
    assert np.all(np.abs(qs) <= 127)
    np.testing.assert_array_equal(b["bsums"].astype(np.int64), qs.reshape(16, 16).sum(axis=1))
    # reconstruction: every element within half a step of d * q (plus fp32 rounding of iscale*x)
    err = np.abs(x.astype(np.float64) - np.float64(b["d"]) * qs)
    assert np.all(err <= np.abs(np.float64(b["d"])) * (0.5 + 1e-5) + 1e-30)
    assert np.sign(b["d"]) == -np.sign(x[i])
