"""Q8_K activation quantization on the GPU is bit-identical to the oracle (ggml's quantize_row_q8_K):
d, every qs byte and every bsum, over seeded inputs with ties, zero blocks, extreme magnitudes and
non-contiguous or misaligned rows. Compares against the committed golden fixture too."""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal, xorshift_noise

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "q8k_vectors.npz")


def _case(name):
    print(f"[q8k] {name}", file=sys.stderr, flush=True)


def _inputs(kind, rows, k, seed):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        return normal((rows, k), seed)
    if kind == "noise":
        return xorshift_noise(rows * k, seed).reshape(rows, k)
    if kind == "ties":  # halves and integers against exact scales: every rounding is a tie case
        x = rng.integers(-254, 255, size=(rows, k)).astype(np.float32) / 2
        x[:, ::256] = -127.0
        return x
    if kind == "zero_blocks":
        x = normal((rows, k), seed)
        x[:, 256:512] = 0.0
        x[0, :256] = -0.0
        return x
    if kind == "dup_max":  # the same |max| several times with both signs
        x = normal((rows, k), seed)
        x[:, 3::97] = 9.0
        x[:, 50::97] = -9.0
        return x
    if kind == "extreme":
        x = normal((rows, k), seed) * np.float32(1e18)
        x[:, 1::7] *= np.float32(1e-30)
        return x
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["normal", "noise", "ties", "zero_blocks", "dup_max", "extreme"])
@pytest.mark.parametrize("rows,k", [(1, 256), (3, 2048), (17, 4096), (64, 768)])
def test_q8_K_bit_exact(gpu, kind, rows, k):
    _case(f"{kind} rows={rows} k={k}")
    x = _inputs(kind, rows, k, seed=rows * 1000 + k)
    got = ggml.quantize_q8_K(torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.quantize_row_q8_K(x).reshape(rows, -1)
    np.testing.assert_array_equal(got, want)


def test_q8_K_strided_and_misaligned_rows(gpu):
    _case("strided / misaligned")
    k = 1024
    wide = torch.from_numpy(normal((5, k + 7), 77)).to(gpu)
    for view in (wide[:, :k], wide[:, 1:k + 1], wide[:, 3:k + 3]):  # row stride k+7 floats; offsets 0,4,12 B
        got = ggml.quantize_q8_K(view).cpu().numpy()
        want = O.quantize_row_q8_K(np.ascontiguousarray(view.cpu().numpy())).reshape(5, -1)
        np.testing.assert_array_equal(got, want)


def test_q8_K_batched_4d(gpu):
    _case("4d")
    x = normal((2, 3, 4, 512), 78)
    got = ggml.quantize_q8_K(torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.quantize_row_q8_K(x.reshape(-1, 512)).reshape(24, -1)
    np.testing.assert_array_equal(got, want)


def test_q8_K_golden(gpu):
    _case("golden")
    g = np.load(GOLDEN)
    got = ggml.quantize_q8_K(torch.from_numpy(g["x"]).to(gpu)).cpu().numpy()
    np.testing.assert_array_equal(got, g["q8"])


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("kind", ["normal", "ties", "zero_blocks", "dup_max", "extreme"])
def test_in_kernel_quantization_matches_the_pass(gpu, tname, kind):
    """Decode-size F32 activations are quantized by the GEMV workgroups into LDS (wave reductions by DPP
    and permlane swaps); the GEMV over them equals, bit for bit, the GEMV over the same activations
    quantized by the Q8_K pass (itself bit-identical to ggml's quantize_row_q8_K above)."""
    from tests.test_gpu_gemv import make_weights
    _case(f"in-kernel {tname} {kind}")
    ty = ggml.Type.Q4_K if tname == "q4_K" else ggml.Type.Q6_K
    k = 2048
    w = make_weights(ty, k, 512, 1, seed=17, device=gpu)
    for m in (1, 2):
        x = torch.from_numpy(np.ascontiguousarray(_inputs(kind, m, k, 40 + m))).to(gpu)
        assert ggml.mul_mat_workspace_size(w, x) == 0  # the in-kernel path
        got = ggml.mul_mat(w, x)
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
        want = ggml.mul_mat(w, xq)
        torch.cuda.synchronize()
        assert got.numel() == want.numel() == m * 512
        assert torch.equal(got.reshape(-1), want.reshape(-1)), f"m={m}: in-kernel Q8_K differs from the pass"



@pytest.mark.parametrize("k", [2048, 4096])
@pytest.mark.parametrize("kind", ["normal", "ties", "zero_blocks", "dup_max", "extreme"])
def test_q6_K_mfma_in_kernel_quantization_matches_the_pass(gpu, kind, k):
    """The Q6_K MFMA kernel (K = 2048 and 4096, 4..8 columns) quantizes F32 activations in its waves; its
    outputs equal, bit for bit, those of the same kernel over the Q8_K pass's bytes."""
    from tests.test_gpu_gemv import make_weights
    _case(f"q6_K mfma in-kernel {kind} k={k}")
    w = make_weights(ggml.Type.Q6_K, k, 700, 1, seed=23, device=gpu)
    for m in (4, 6, 8):
        x = torch.from_numpy(np.ascontiguousarray(_inputs(kind, m, k, 60 + m))).to(gpu)
        assert ggml.mul_mat_workspace_size(w, x) == 0  # the in-kernel path
        got = ggml.mul_mat(w, x)
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
        want = ggml.mul_mat(w, xq)
        torch.cuda.synchronize()
        assert torch.equal(got.reshape(-1), want.reshape(-1)), f"m={m}: in-kernel Q8_K differs from the pass"