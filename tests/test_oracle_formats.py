"""Pins the oracle's block decoding (fp16, Q4_K, Q6_K, Q8_K dequantization) to the reference.

The element order and scale packing are checked against an independent restatement of how patch
0002's iqk kernels read the blocks (patches/0002-iqk-avx512-q4k-q6k-decode.patch): make_q4_scales
(:371-380) and Q4Bits::prepare with BlockPermuter (:1425-1441) for Q4_K, which pair 64-byte lanes of
nibbles with q8 quants 64*j..64*j+63; prepare64 + add_high_bits (:1638-1663) and Scale16's shuffles
(:1581-1598) for Q6_K. Those use 32-bit words and 64-bit lane permutes, a different route from the
oracle's per-element indexing, so a wrong nibble half, scale index or high-bit shift fails here.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import random_blocks


def test_fp16_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([O.fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(want)
    np.testing.assert_array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.all(got[np.isinf(want)] == want[np.isinf(want)])


def _iqk_q4_K(raw: np.ndarray) -> np.ndarray:
    """Q4_K dequantization the way the iqk kernel consumes a block."""
    blocks = raw.view(O.BLOCK_Q4_K)
    out = np.zeros((len(blocks), 256), dtype=np.float32)
    for i, b in enumerate(blocks):
        s = b["scales"].astype(np.uint32)
        a0 = s[0] | (s[1] << 8) | (s[2] << 16) | (s[3] << 24)
        a1 = s[4] | (s[5] << 8) | (s[6] << 16) | (s[7] << 24)
        a2 = s[8] | (s[9] << 8) | (s[10] << 16) | (s[11] << 24)
        aux = [a0 & 0x3f3f3f3f, (a2 & 0x0f0f0f0f) | ((a0 >> 2) & 0x30303030),
               a1 & 0x3f3f3f3f, ((a2 >> 4) & 0x0f0f0f0f) | ((a1 >> 2) & 0x30303030)]
        by = np.array(aux, dtype=np.uint32).view(np.uint8)  # sc[0..7] then m[0..7]
        sc, m = by[:8].astype(np.float32), by[8:].astype(np.float32)
        qs = b["qs"]
        # 64-byte register r of nibbles (qs[64r .. 64r+63]): lanes 0..31 = low nibbles of its first
        # 32 bytes, lanes 32..63 = their high nibbles; then the same for the next 32 bytes.
        vals = []
        for r in range(2):
            q = qs[64 * r:64 * r + 64]
            lo, hi = q & 0x0F, q >> 4
            vals.append(np.concatenate([lo[:32], hi[:32]]))
            vals.append(np.concatenate([lo[32:], hi[32:]]))
        q = np.concatenate(vals).astype(np.float32)  # element order 0..255
        d = np.float32(b["d"].view(np.float16))
        dmin = np.float32(b["dmin"].view(np.float16))
        j = np.arange(256) // 32
        out[i] = (d * sc[j]) * q - dmin * m[j]
    return out.reshape(-1)


def _iqk_q6_K(raw: np.ndarray) -> np.ndarray:
    """Q6_K dequantization the way the iqk kernel consumes a block (values[0..3] pair with q8 quants
    0..63, 64..127, 128..191, 192..255)."""
    blocks = raw.view(O.BLOCK_Q6_K)
    out = np.zeros((len(blocks), 256), dtype=np.float32)
    for i, b in enumerate(blocks):
        ql, qh = b["ql"].astype(np.int32), b["qh"].astype(np.int32)
        v = [ql[:64] & 0xF, ql[:64] >> 4, ql[64:] & 0xF, ql[64:] >> 4]
        h0, h1 = qh[:32], qh[32:]
        # add_high_bits: permute1 takes hbits qwords 0..3 (qh[0..31]), permute2 qwords 4..7 (qh[32..63])
        v[0] = v[0] | np.concatenate([(h0 << 4) & 0x30, (h0 << 2) & 0x30])
        v[2] = v[2] | np.concatenate([(h1 << 4) & 0x30, (h1 << 2) & 0x30])
        v[1] = v[1] | np.concatenate([h0 & 0x30, (h0 >> 2) & 0x30])
        v[3] = v[3] | np.concatenate([h1 & 0x30, (h1 >> 2) & 0x30])
        q = np.concatenate(v).astype(np.float32) - 32
        d = np.float32(b["d"].view(np.float16))
        sc = b["scales"].astype(np.float32)
        out[i] = d * sc[np.arange(256) // 16] * q
    return out.reshape(-1)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q4_K_matches_iqk_layout(seed):
    raw = random_blocks(O.TYPE_Q4_K, 16, seed)
    got = O.dequantize(O.TYPE_Q4_K, raw, 16 * 256)
    np.testing.assert_array_equal(got, _iqk_q4_K(raw))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q6_K_matches_iqk_layout(seed):
    raw = random_blocks(O.TYPE_Q6_K, 16, seed)
    got = O.dequantize(O.TYPE_Q6_K, raw, 16 * 256)
    np.testing.assert_array_equal(got, _iqk_q6_K(raw))


def test_q8_K_dequant_is_d_times_qs():
    x = np.random.default_rng(5).standard_normal(1024).astype(np.float32)
    q = O.quantize_row_q8_K(x)
    b = q.view(O.BLOCK_Q8_K)
    got = O.dequantize(O.TYPE_Q8_K, q, 1024)
    np.testing.assert_array_equal(got, (b["d"][:, None] * b["qs"].astype(np.float32)).reshape(-1))


def test_q4_K_single_nibble_moves_one_element():
    """Setting one byte of qs in an otherwise zero block moves exactly the two elements it holds."""
    raw = np.zeros(144, dtype=np.uint8)
    b = raw.view(O.BLOCK_Q4_K)[0]
    b["d"] = 0x3C00  # 1.0
    b["scales"][:] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]  # all scales 1, mins 0
    for byte in [0, 5, 31, 32, 63, 64, 100, 127]:
        b["qs"][:] = 0
        b["qs"][byte] = 0x21  # low nibble 1, high nibble 2
        y = O.dequantize(O.TYPE_Q4_K, raw, 256)
        c, l = byte // 32, byte % 32
        want = np.zeros(256, dtype=np.float32)
        want[64 * c + l] = 1.0
        want[64 * c + 32 + l] = 2.0
        np.testing.assert_array_equal(y, want)


def test_q6_K_single_field_moves_one_element():
    raw = np.zeros(210, dtype=np.uint8)
    b = raw.view(O.BLOCK_Q6_K)[0]
    b["d"] = 0x3C00
    b["scales"][:] = 1
    base = np.full(256, -32.0, dtype=np.float32)  # all-zero quants decode to -32
    for h in range(2):
        for l in [0, 9, 31]:
            for t in range(4):
                b["ql"][:] = 0
                b["qh"][:] = 0
                b["qh"][32 * h + l] = 1 << (2 * t)  # high-bit 1 of quarter t -> +16
                y = O.dequantize(O.TYPE_Q6_K, raw, 256)
                want = base.copy()
                want[128 * h + 32 * t + l] += 16
                np.testing.assert_array_equal(y, want)
