"""Pins the oracle's MUL_MAT and MUL_MAT_ID (ggml semantics, patch 0004's -1 rule).

MUL_MAT: the by-hand F32 case of crates/ggml-sys/tests/ggml.rs:13-30 ([[1,2,3],[4,5,6]] . [1,0.5,2]
= [8, 18.5]) with the weights held exactly in Q6_K, both through the Q8_K rounding of the activation
(within its bound) and with an activation Q8_K represents exactly; the broadcast of src0 over dims 2
and 3 (ggml's i02 = i12 / (ne12/ne02)).
MUL_MAT_ID: the per-expert reassembly of crates/ggml-sys/tests/mul_mat_id_skip.rs:124-206 (one plain
MUL_MAT per expert over the gathered columns, zero rows for -1), for b1 in {1, n_used}.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import half_bits, random_blocks, xorshift_noise


def _q6_K_exact(rows):
    """A Q6_K matrix [256, len(rows)] holding small integers exactly: d = 1, every scale 1, q = w + 32."""
    raw = np.zeros(210 * len(rows), dtype=np.uint8)
    blocks = raw.view(O.BLOCK_Q6_K)
    for r, vals in enumerate(rows):
        w = np.zeros(256, dtype=np.int64)
        w[:len(vals)] = vals
        q = w + 32
        b = blocks[r]
        b["d"] = half_bits(1.0)
        b["scales"] = 1
        ql = np.zeros(128, dtype=np.int64)
        qh = np.zeros(64, dtype=np.int64)
        for e in range(256):
            h, rr = divmod(e, 128)
            t, l = divmod(rr, 32)
            qi = 64 * h + 32 * (t & 1) + l
            ql[qi] |= (q[e] & 0xF) << (0 if t < 2 else 4)
            qh[32 * h + l] |= ((q[e] >> 4) & 3) << (2 * t)
        b["ql"], b["qh"] = ql, qh
    assert np.array_equal(O.dequantize(O.TYPE_Q6_K, raw, 256 * len(rows)).reshape(len(rows), 256)[:, :3],
                          np.array([r + [0] * (3 - len(r)) for r in rows], dtype=np.float32)[:, :3])
    return raw


def test_mul_mat_by_hand_through_q8_K():
    w = _q6_K_exact([[1, 2, 3], [4, 5, 6]])
    x = np.zeros(256, dtype=np.float32)
    x[:3] = [1.0, 0.5, 2.0]
    y = O.mul_mat(O.TYPE_Q6_K, w, 256, 2, x)[0, 0]
    step = abs(float(O.quantize_row_q8_K(x).view(O.BLOCK_Q8_K)["d"][0]))
    assert abs(y[0] - 8.0) <= (1 + 2 + 3) * step / 2
    assert abs(y[1] - 18.5) <= (4 + 5 + 6) * step / 2


def test_mul_mat_by_hand_exact():
    """max |x| = 127 makes iscale = -1 exactly, so integer activations pass Q8_K unchanged."""
    w = _q6_K_exact([[1, 2, 3], [4, 5, 6]])
    x = np.zeros(256, dtype=np.float32)
    x[:4] = [2.0, 1.0, 4.0, 127.0]
    y = O.mul_mat(O.TYPE_Q6_K, w, 256, 2, x)[0, 0]
    np.testing.assert_array_equal(y, np.array([1 * 2 + 2 * 1 + 3 * 4, 4 * 2 + 5 * 1 + 6 * 4], dtype=np.float32))


@pytest.mark.parametrize("ty", [O.TYPE_Q4_K, O.TYPE_Q6_K])
def test_mul_mat_broadcast(ty):
    k, n, ne02, m, ne12 = 512, 5, 2, 3, 4
    raw = random_blocks(ty, ne02 * n * k // 256, seed=9)
    b = xorshift_noise(ne12 * m * k, 4).reshape(ne12, m, k)
    y = O.mul_mat(ty, raw, k, n, b, ne2=ne02)
    mat_bytes = n * O.row_size(ty, k)
    rb = O.row_size(ty, k)
    for i12 in range(ne12):
        i02 = i12 // (ne12 // ne02)
        mat = raw[i02 * mat_bytes:(i02 + 1) * mat_bytes]
        for j in range(m):
            q8 = O.quantize_row_q8_K(b[i12, j])
            want = [O.vec_dot(ty, k, mat[r * rb:(r + 1) * rb], q8) for r in range(n)]
            np.testing.assert_array_equal(y[i12, j], np.array(want, dtype=np.float32))


def make_ids(n_expert, used, tokens, neg_pct, rng):
    """Distinct experts per token with neg_pct percent of slots set to -1 (mul_mat_id_skip.rs:64-84)."""
    ids = np.zeros((tokens, used), dtype=np.int32)
    for t in range(tokens):
        pool = rng.permutation(n_expert)[:used]
        for j in range(used):
            ids[t, j] = -1 if rng.integers(100) < neg_pct else pool[j]
    return ids


def per_expert_reference(ty, raw, k, n, n_expert, b, ids):
    """One plain MUL_MAT per expert over the columns routed to it; zero rows for -1."""
    T, used = ids.shape
    b1 = b.shape[1]
    out = np.zeros((T, used, n), dtype=np.float32)
    eb = n * O.row_size(ty, k)
    for e in range(n_expert):
        slots = [(t, j) for t in range(T) for j in range(used) if ids[t, j] == e]
        if not slots:
            continue
        cols = np.stack([b[t, 0 if b1 == 1 else j] for t, j in slots])
        y = O.mul_mat(ty, raw[e * eb:(e + 1) * eb], k, n, cols)[0]
        for c, (t, j) in enumerate(slots):
            out[t, j] = y[c]
    return out


@pytest.mark.parametrize("ty", [O.TYPE_Q4_K, O.TYPE_Q6_K])
@pytest.mark.parametrize("tokens", [1, 8, 33])
@pytest.mark.parametrize("b1", [1, 4])
def test_mul_mat_id_matches_per_expert_mul_mat(ty, tokens, b1):
    rng = np.random.default_rng(0x9E3779B97F4A7C15 & 0xFFFFFFFF)
    k, n, n_expert, used = 512, 64, 16, 4
    raw = random_blocks(ty, n_expert * n * k // 256, seed=tokens)
    b = xorshift_noise(tokens * b1 * k, tokens + b1).reshape(tokens, b1, k)
    ids = make_ids(n_expert, used, tokens, 30, rng)
    got = O.mul_mat_id(ty, raw, k, n, n_expert, b, ids)
    want = per_expert_reference(ty, raw, k, n, n_expert, b, ids)
    np.testing.assert_array_equal(got, want)
    neg = ids < 0
    assert np.all(got[neg] == 0.0) and np.all(np.signbit(got[neg]) == 0)


def test_sum_experts_adds_left_to_right():
    """sum_experts (crates/model/src/qwen3moe.rs:2917-2923) folds the choice views with fp32 adds from
    the first: (1e8 + 1) - 1e8 is 0 in fp32 (1e8 + 1 rounds to 1e8), where a sum from the right or in
    float64 gives 1; a single choice is returned as is."""
    e = np.array([[[1e8], [1.0], [-1e8]]], dtype=np.float32)
    assert O.sum_experts(e)[0, 0] == np.float32(0.0)
    assert np.float64(1e8) + 1.0 - 1e8 == 1.0
    one = np.array([[[3.5, -2.0]]], dtype=np.float32)
    np.testing.assert_array_equal(O.sum_experts(one), one[:, 0, :])
    rng = np.random.default_rng(3)
    r = rng.standard_normal((5, 8, 64)).astype(np.float32)
    np.testing.assert_allclose(O.sum_experts(r), r.astype(np.float64).sum(axis=1), rtol=0, atol=1e-5)


def test_router_top_k_order_and_weights():
    """The reference's own top-k case (crates/ggml-sys/tests/ggml.rs:33-44: scores [0.1, 0.9, 0.3, 0.5],
    k = 2 -> ids [1, 3]) through the router with one embedding dimension (a one-weight gate row per
    expert makes the logits the scores times xn > 0); the weights are the selected probabilities over
    their sum; rms_norm of a constant row is sign(x) / sqrt(1 + eps / x^2) times the norm weight; a
    probability tie goes to the lower id."""
    x = np.array([[2.0]], dtype=np.float32)
    gate = np.array([[0.1], [0.9], [0.3], [0.5]], dtype=np.float32)
    xn, probs, w, ids = O.router(x, np.ones(1, np.float32), gate, 1e-6, 2)
    assert ids.tolist() == [[1, 3]]
    np.testing.assert_allclose(probs.sum(axis=1), 1.0, rtol=1e-6)
    sel = probs[0, [1, 3]]
    np.testing.assert_allclose(w[0], sel / sel.sum(), rtol=1e-6)
    np.testing.assert_allclose(xn[0, 0], 2.0 / np.sqrt(4.0 + 1e-6), rtol=1e-6)
    c = np.full((1, 8), -3.0, np.float32)
    xn, _, _, _ = O.router(c, np.full(8, 0.5, np.float32), np.ones((2, 8), np.float32), 0.0, 1)
    np.testing.assert_allclose(xn, -0.5, rtol=1e-6)
    _, _, _, ids = O.router(np.ones((1, 4), np.float32), np.ones(4, np.float32), np.ones((3, 4), np.float32), 1e-6, 2)
    assert ids.tolist() == [[0, 1]]


def test_router_softmax_closed_form():
    """soft_max in closed form: logits {0, ln 3} give probabilities {1/4, 3/4} (e^0 : e^ln3 = 1 : 3), and
    {0, ln 3, ln 4} give {1/8, 3/8, 4/8}. x = [1, 1] with eps 0 normalizes to itself exactly, and one-hot
    gate rows make the logits the chosen values. Top-2 of the second case is [2, 1] with weights
    {4/7, 3/7} (the selected probabilities over their sum)."""
    x = np.ones((1, 2), np.float32)
    gate = np.array([[0.0, 0.0], [np.log(3.0), 0.0]], dtype=np.float32)
    xn, probs, w, ids = O.router(x, np.ones(2, np.float32), gate, 0.0, 2)
    np.testing.assert_array_equal(xn, x)
    np.testing.assert_allclose(probs[0], [0.25, 0.75], rtol=0, atol=2e-7)
    assert ids.tolist() == [[1, 0]]
    np.testing.assert_allclose(w[0], [0.75, 0.25], rtol=0, atol=2e-7)
    gate3 = np.array([[0.0, 0.0], [np.log(3.0), 0.0], [0.0, np.log(4.0)]], dtype=np.float32)
    _, probs, w, ids = O.router(x, np.ones(2, np.float32), gate3, 0.0, 2)
    np.testing.assert_allclose(probs[0], [0.125, 0.375, 0.5], rtol=0, atol=2e-7)
    assert ids.tolist() == [[2, 1]]
    np.testing.assert_allclose(w[0], [4 / 7, 3 / 7], rtol=0, atol=2e-7)
