"""Pins the oracle's vec_dot_q4_K_q8_K / vec_dot_q6_K_q8_K and the restated iqk CPU baseline.

Three routes must agree: (1) the oracle's integer vec_dot with the mins / -32 folded in through the
Q8_K bsums, (2) an f64 brute force over the dequantized weights and the dequantized Q8_K activation
with the per-output bound 1e-5 * sum|w x| + 1e-6 of crates/ggml-sys/tests/iqk_kernels.rs:127-148,
(3) the AVX-512 VNNI restatement of the iqk one-column kernel (patches/0002:1812-1849), whose lane
order and summation differ. A dropped min term, a wrong sign of the -32 offset or a transposed
scale index moves (1) or (3) far outside the bound of (2). Hand-built blocks give exact answers.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import half_bits, normal, pack_q4_K_scales, random_blocks, xorshift_noise

TYPES = [O.TYPE_Q4_K, O.TYPE_Q6_K]


def _rows(ty, raw, k):
    rb = O.row_size(ty, k)
    return [raw[i * rb:(i + 1) * rb] for i in range(raw.size // rb)]


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("k", [256, 1536, 4096])
def test_vec_dot_within_f64_bound(ty, k):
    n = 24
    raw = random_blocks(ty, n * k // 256, seed=11 + k)
    x = xorshift_noise(k, 99 + k)  # the reference test's activation generator
    q8 = O.quantize_row_q8_K(x)
    ref, bound = O.ref_f64(ty, raw, k, x)
    got = np.array([O.vec_dot(ty, k, r, q8) for r in _rows(ty, raw, k)], dtype=np.float64)
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("k", [256, 768, 2048])
def test_iqk_baseline_within_f64_bound(ty, k):
    if not O.has_avx512_vnni():
        pytest.skip("skip: host has no AVX-512 VNNI (the baseline falls back to vec_dot)")
    n = 40
    raw = random_blocks(ty, n * k // 256, seed=5 + k)
    x = normal(k, 7 + k)
    q8 = O.quantize_row_q8_K(x)
    ref, bound = O.ref_f64(ty, raw, k, x)
    got = O.iqk_rows(ty, raw, k, q8)
    assert got is not None
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


@pytest.mark.parametrize("ty", TYPES)
def test_iqk_static_split_is_thread_invariant(ty):
    """Each row is computed by one thread whatever the split (iqk_kernels.rs:205-221): the union of
    the shares of nth threads equals the one-thread result bit for bit."""
    if not O.has_avx512_vnni():
        pytest.skip("skip: host has no AVX-512 VNNI")
    k, n = 1536, 97
    raw = random_blocks(ty, n * k // 256, seed=21)
    q8 = O.quantize_row_q8_K(normal(k, 22))
    base = O.iqk_rows(ty, raw, k, q8, 0, 1)
    for nth in (3, 8, 200):
        out = np.full(n, np.nan, dtype=np.float32)
        for ith in range(nth):
            part = O.iqk_rows(ty, raw, k, q8, ith, nth)
            per = (n + nth - 1) // nth
            lo, hi = ith * per, min(n, ith * per + per)
            out[lo:hi] = part[lo:hi]
        np.testing.assert_array_equal(out.view(np.uint32), base.view(np.uint32))


def _q8_const(qs: int, d: float):
    blk = np.zeros(1, dtype=O.BLOCK_Q8_K)
    blk["d"] = d
    blk["qs"] = qs
    blk["bsums"] = 16 * qs
    return blk.view(np.uint8)


def test_q4_K_known_answer():
    """d=1, dmin=0.5, scale j = j+1, min 2, every q = 3: w = (j+1)*3 - 1; activation 0.5*2 = 1;
    the dot is sum_j 32*(3(j+1) - 1) = 32*(3*36 - 8) = 3200."""
    raw = np.zeros(144, dtype=np.uint8)
    b = raw.view(O.BLOCK_Q4_K)[0]
    b["d"], b["dmin"] = half_bits(1.0), half_bits(0.5)
    b["scales"] = pack_q4_K_scales([1, 2, 3, 4, 5, 6, 7, 8], [2] * 8)
    b["qs"] = 0x33
    y = _q8_const(2, 0.5)
    assert O.vec_dot(O.TYPE_Q4_K, 256, raw, y) == 3200.0
    assert O.dequantize(O.TYPE_Q4_K, raw, 256)[255] == 8 * 3 - 1
    if O.has_avx512_vnni():
        assert O.iqk_rows(O.TYPE_Q4_K, raw, 256, y)[0] == 3200.0


def test_q4_K_high_scale_bits_known_answer():
    """Scales and mins above 15 for sub-blocks 4..7 use the packed top bits: scale 63, min 48."""
    raw = np.zeros(144, dtype=np.uint8)
    b = raw.view(O.BLOCK_Q4_K)[0]
    b["d"], b["dmin"] = half_bits(1.0), half_bits(1.0)
    b["scales"] = pack_q4_K_scales([0, 0, 0, 0, 63, 0, 0, 0], [0, 0, 0, 0, 48, 0, 0, 0])
    b["qs"] = 0x01  # every low nibble 1, high nibble 0
    y = _q8_const(1, 1.0)
    # sub-block 4 = elements 128..159 = low nibbles of qs[64..95]: w = 63*1 - 48 = 15; the other
    # sub-blocks have scale 0 and min 0 -> 0
    assert O.vec_dot(O.TYPE_Q4_K, 256, raw, y) == 32 * 15
    w = O.dequantize(O.TYPE_Q4_K, raw, 256)
    assert np.all(w[128:160] == 15) and np.count_nonzero(w) == 32


def test_q6_K_known_answer():
    """d=1, scales = -2 for even groups and 3 for odd, every q = 33 (-> +1): w = sc; activation
    1*3; dot = 3*16*(8*(-2) + 8*3) = 384."""
    raw = np.zeros(210, dtype=np.uint8)
    b = raw.view(O.BLOCK_Q6_K)[0]
    b["d"] = half_bits(1.0)
    b["scales"] = [-2, 3] * 8
    b["ql"] = 0x11
    b["qh"] = 0xAA  # every 2-bit field = 2 -> q = 1 | 2<<4 = 33
    y = _q8_const(3, 1.0)
    assert O.vec_dot(O.TYPE_Q6_K, 256, raw, y) == 384.0
    if O.has_avx512_vnni():
        assert O.iqk_rows(O.TYPE_Q6_K, raw, 256, y)[0] == 384.0
