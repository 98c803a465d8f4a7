"""MUL_MAT with many activation columns on the GPU against the oracle: 64 or more columns run on the
int8-MFMA kernel, fewer on the streaming GEMV (8 columns per pass); the cases straddle the switch.

Same bar as the GEMV: every output within 1e-3 of the largest reference magnitude (fp32 accumulation
order is the only difference: both sides use the same weight bytes and the same Q8_K activations).
Covers ragged M and N around the 64 x 128 / 128 x 64 / 256 x 64 tile edges, K from one super-block to
12288, broadcast over dims 2 and 3 with strided b and dst, a pre-quantized Q8_K b, activations with a
huge dynamic range and all-zero columns, and the dense prefill shapes (hidden 4096, FFN 12288, Q4_K
gate/up and Q6_K down at M = 512 and 2048) on sampled weight rows.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal

pytestmark = pytest.mark.gpu
TOL = 1e-3
TYPES = {"q4_K": ggml.Type.Q4_K, "q6_K": ggml.Type.Q6_K}


def _case(name):
    print(f"[mmq] {name}", file=sys.stderr, flush=True)


def make_weights(ty, k, n, ne2, seed, device, std=0.02):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((ne2 * n, k), generator=g, device=device) * std
    return ggml.QTensor(ty, (k, n, ne2), ggml.quantize(ty, src, ne2 * n, k))


def check(got, want, what):
    scale = max(float(np.abs(want).max()), 1e-30)
    worst = float(np.abs(got.astype(np.float64) - want).max() / scale)
    assert worst <= TOL, f"{what}: worst {worst:.2e} of the largest > {TOL:.0e}"
    return worst


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("k,n,m", [(256, 1, 9), (256, 33, 31), (512, 64, 32), (512, 129, 33), (1024, 200, 64),
                                   (768, 127, 65), (2048, 300, 100), (1024, 64, 128), (512, 65, 129),
                                   (4096, 96, 300), (12288, 40, 70)])
def test_mmq_matches_oracle(gpu, tname, k, n, m):
    _case(f"{tname} k={k} n={n} m={m}")
    ty = TYPES[tname]
    w = make_weights(ty, k, n, 1, seed=k + 7 * n + 13 * m, device=gpu)
    x = normal((m, k), k * 3 + n + m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"{tname} k={k} n={n} m={m}")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_mmq_broadcast_and_strides(gpu, tname):
    """a [K, N, 2] broadcast over b [K, M, 4] (i02 = i12 / 2); b rows strided; dst a strided view."""
    _case(f"{tname} broadcast")
    ty = TYPES[tname]
    k, n, m = 512, 70, 72
    w = make_weights(ty, k, n, 2, seed=55, device=gpu)
    xb = normal((4, m, k + 64), 56)
    xt = torch.from_numpy(xb).to(gpu)[:, :, 32:32 + k]
    out_big = torch.full((4, m, n + 8), float("nan"), device=gpu)
    out = out_big[:, :, :n]
    ggml.mul_mat(w, xt, out=out)
    got = out_big.cpu().numpy()
    assert np.all(np.isnan(got[:, :, n:])), "wrote outside dst"
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, np.ascontiguousarray(xb[:, :, 32:32 + k]), ne2=2)
    check(got[:, :, :n], want, f"{tname} broadcast")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_mmq_prequantized_b(gpu, tname):
    """b already Q8_K (ggml's vec_dot_type) gives the same result as the F32 b it came from."""
    _case(f"{tname} q8_K b")
    ty = TYPES[tname]
    k, n, m = 1024, 96, 96
    w = make_weights(ty, k, n, 1, seed=3, device=gpu)
    x = torch.from_numpy(normal((m, k), 4)).to(gpu)
    xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
    a = ggml.mul_mat(w, x)
    b = ggml.mul_mat(w, xq)
    assert torch.equal(a, b.view(m, n))


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_mmq_dynamic_range_and_zero_columns(gpu, tname):
    """Columns scaled over 1e-30 .. 1e30 and all-zero columns (Q8_K d = 0)."""
    _case(f"{tname} dynamic range")
    ty = TYPES[tname]
    k, n, m = 768, 64, 80
    w = make_weights(ty, k, n, 1, seed=8, device=gpu)
    x = normal((m, k), 9)
    x *= (10.0 ** np.linspace(-30, 30, m)).astype(np.float32)[:, None]
    x[5] = 0.0
    x[17] = 0.0
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    assert np.all(y[5] == 0) and np.all(y[17] == 0)
    for i in range(m):  # each column against its own magnitude
        if i not in (5, 17):
            check(y[i], want[i], f"{tname} column {i}")


def test_mmq_workspace_argument(gpu):
    _case("workspace")
    w = make_weights(ggml.Type.Q6_K, 1024, 64, 1, seed=7, device=gpu)
    x = torch.from_numpy(normal((80, 1024), 9)).to(gpu)
    need = ggml.mul_mat_workspace_size(w, x)
    assert need >= 80 * 4 * 292
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    a = ggml.mul_mat(w, x, workspace=ws)
    b = ggml.mul_mat(w, x)
    assert torch.equal(a, b)
    with pytest.raises(ggml.Compute):
        ggml.mul_mat(w, x, workspace=ws[: need // 2])


@pytest.mark.parametrize("name,tname,k,n", [("gate", "q4_K", 4096, 12288), ("down", "q6_K", 12288, 4096)])
@pytest.mark.parametrize("m", [512, 2048])
def test_prefill_shapes(gpu, name, tname, k, n, m):
    """The dense prefill GEMMs at full size; 96 sampled weight rows against the oracle for every column."""
    _case(f"prefill {name} m={m}")
    ty = TYPES[tname]
    w = make_weights(ty, k, n, 1, seed=n + m, device=gpu)
    x = normal((m, k), m + k)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    assert y.shape == (m, n) and np.all(np.isfinite(y))
    rows = np.sort(np.random.default_rng(m).choice(n, 96, replace=False))
    rb = ty.row_size(k)
    sub = w.data.view(n, rb)[torch.from_numpy(rows).to(gpu)].cpu().numpy().reshape(-1)
    want = O.mul_mat(ty.id, sub, k, len(rows), x)[0]
    check(y[:, rows], want, f"prefill {name} m={m}")


@pytest.mark.parametrize("k,n,m", [(256, 128, 128), (768, 300, 130), (2048, 515, 257), (4096, 1000, 200),
                                   (12288, 130, 129), (512, 128, 1000), (1280, 129, 300)])
def test_mmq_tile_q6_K(gpu, k, n, m):
    """Q6_K with at least 128 columns and 128 rows runs the 128 x 128 tile kernel (planes built once per
    workgroup in LDS): one tile, ragged last tiles in both directions, odd super-block counts (rows and
    blocks that start 2 bytes past a dword boundary: Q6_K blocks are 210 bytes), K up to 12288."""
    _case(f"q6_K tile k={k} n={n} m={m}")
    ty = TYPES["q6_K"]
    w = make_weights(ty, k, n, 1, seed=k + 5 * n + 13 * m, device=gpu)
    x = normal((m, k), k + 3 * n + 5 * m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q6_K tile k={k} n={n} m={m}")


@pytest.mark.parametrize("k,n,m", [(256, 256, 128), (768, 300, 130), (2048, 515, 257), (4096, 1000, 200),
                                   (12288, 260, 129), (512, 256, 1000)])
def test_mmq_tile_q4_K(gpu, k, n, m):
    """Q4_K with at least 128 columns and 256 rows runs the 128 x 256 tile kernel: one tile, ragged last
    tiles in both directions (computed over the last full window, stored only for their own rows), odd
    and even super-block counts (the kernel walks super-blocks in pairs of LDS buffers), K up to 12288."""
    _case(f"q4_K tile k={k} n={n} m={m}")
    ty = TYPES["q4_K"]
    w = make_weights(ty, k, n, 1, seed=k + 5 * n + 11 * m, device=gpu)
    x = normal((m, k), k + 3 * n + 7 * m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q4_K tile k={k} n={n} m={m}")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_mmq_tile_broadcast_strides_and_range(gpu, tname):
    """The tile kernels under broadcast (a [K, N, 2] over b [K, M, 4]), strided b and dst, columns over
    1e-30 .. 1e30 and all-zero columns."""
    _case(f"{tname} tile broadcast")
    ty = TYPES[tname]
    k, n, m = 768, 300, 140
    w = make_weights(ty, k, n, 2, seed=77, device=gpu)
    xb = normal((4, m, k + 64), 78)
    xb *= (10.0 ** np.linspace(-30, 30, m)).astype(np.float32)[None, :, None]
    xb[1, 9] = 0.0
    xt = torch.from_numpy(xb).to(gpu)[:, :, 32:32 + k]
    out_big = torch.full((4, m, n + 8), float("nan"), device=gpu)
    ggml.mul_mat(w, xt, out=out_big[:, :, :n])
    got = out_big.cpu().numpy()
    assert np.all(np.isnan(got[:, :, n:])), "wrote outside dst"
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, np.ascontiguousarray(xb[:, :, 32:32 + k]), ne2=2)
    assert np.all(got[1, 9, :n] == 0)
    for z in range(4):
        for i in range(m):
            if (z, i) != (1, 9):
                check(got[z, i, :n], want[z, i], f"tile broadcast z={z} column {i}")


@pytest.mark.parametrize("tname,k,n,m", [("q6_K", 4096, 256, 128), ("q4_K", 4096, 256, 130), ("q6_K", 3072, 300, 260)])
def test_mmq_tile_k_split(gpu, tname, k, n, m):
    """Few output tiles run split along k (several workgroups per tile, the last to arrive sums the
    partials in split order): repeated calls give the same bits (the arrival counts reset, the order of
    the sum does not depend on timing), the reported workspace holds the partials, a smaller one is
    rejected, and the result matches the oracle."""
    _case(f"{tname} k split k={k} n={n} m={m}")
    ty = TYPES[tname]
    w = make_weights(ty, k, n, 1, seed=k + n + m, device=gpu)
    x = torch.from_numpy(normal((m, k), 3 * k + m)).to(gpu)
    need = ggml.mul_mat_workspace_size(w, x)
    assert need > m * (k // 256) * 292, "no room for the partial tiles"
    runs = [ggml.mul_mat(w, x) for _ in range(3)]
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    runs.append(ggml.mul_mat(w, x, workspace=ws))
    for r in runs[1:]:
        assert torch.equal(r, runs[0])
    with pytest.raises(ggml.Compute):
        ggml.mul_mat(w, x, workspace=ws[: need - 256])
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x.cpu().numpy())[0]
    check(runs[0].cpu().numpy(), want, f"{tname} k split")
