"""MUL_MAT (decode GEMV, 1..32 columns) on the GPU against the oracle's vec_dot on the same bytes.

Bar: every output within 1e-3 of the largest reference magnitude (the fp32 accumulation-order
tolerance) and within the per-output f64 bound 1e-5 * sum|w x| + 1e-6 of
crates/ggml-sys/tests/iqk_kernels.rs:127-148. Weights come from the device quantizer (N(0, 0.02)),
activations are N(0, 1); the bytes are copied back so both sides consume the same input.
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal

pytestmark = pytest.mark.gpu
TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TYPES = {"q4_K": ggml.Type.Q4_K, "q6_K": ggml.Type.Q6_K}


def _case(name):
    print(f"[gemv] {name}", file=sys.stderr, flush=True)


def make_weights(ty, k, n, ne2, seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((ne2 * n, k), generator=g, device=device) * 0.02
    raw = ggml.quantize(ty, src, ne2 * n, k)
    return ggml.QTensor(ty, (k, n, ne2), raw)


def check(got, want, what, bound=None, ref=None):
    scale = max(float(np.abs(want).max()), 1e-6)
    worst = float(np.abs(got.astype(np.float64) - want).max() / scale)
    assert worst <= TOL, f"{what}: worst {worst:.2e} of the largest > {TOL:.0e}"
    if bound is not None:
        excess = np.abs(got.astype(np.float64) - ref) - bound
        assert np.all(excess <= 0), f"{what}: above the f64 bound by {excess.max():.3e}"
    return worst


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("k", [256, 512, 768, 2048, 4096])
@pytest.mark.parametrize("n", [1, 5, 96, 1031])
def test_gemv_one_column(gpu, tname, k, n):
    _case(f"{tname} k={k} n={n} m=1")
    ty = TYPES[tname]
    w = make_weights(ty, k, n, 1, seed=k * 31 + n, device=gpu)
    x = normal((1, k), k + n)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    raw = w.data.cpu().numpy()
    want = O.mul_mat(ty.id, raw, k, n, x)[0]
    ref, bound = O.ref_f64(ty.id, raw, k, x[0])
    check(y[0], want[0], f"{tname} k={k} n={n}", bound, ref)


@pytest.mark.parametrize("m", [1, 2, 4])
def test_q4_K_4096x4096_full_size(gpu, m):
    """The single Q4_K MUL_MAT of the reference's CPU benchmark at its own shape: weight 4096 x 4096
    (N(0, 0.02), 9,437,184 bytes), activation batch 1 (also 2 and 4) N(0, 1), every output row against
    the oracle and the per-row f64 bound. On a 256-CU part the batch-1 stream runs two passes per wave,
    so the second LDS slot and the stash flush after a multi-pass window are exercised."""
    _case(f"q4_K 4096x4096 m={m}")
    ty = ggml.Type.Q4_K
    k = n = 4096
    w = make_weights(ty, k, n, 1, seed=4096 + m, device=gpu)
    x = normal((m, k), 40960 + m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    raw = w.data.cpu().numpy()
    want = O.mul_mat(ty.id, raw, k, n, x)[0]
    for c in range(m):
        ref, bound = O.ref_f64(ty.id, raw, k, x[c])
        check(y[c], want[c], f"q4_K 4096x4096 m={m} col {c}", bound, ref)


@pytest.mark.parametrize("k,n", [(4096, 8192), (4096, 12289), (4096, 40000), (1024, 300000), (1024, 600000)])
@pytest.mark.parametrize("m", [1, 2])
def test_q4_K_multi_pass(gpu, k, n, m):
    """Q4_K with several LDS-stream passes per wave (2048 waves on 256 CUs): at K = 4096 (one row per
    pass) 8192 rows (4 passes per wave), a ragged 12289 (one wave's last pass holds the last row) and
    40000 (about 20 passes); at K = 1024 (four rows per pass) 300000 and 600000 rows, 37 and 73 passes
    per wave, past the 32 (two columns) and 64 (one column) passes whose row totals one stash window
    holds, so stashed totals are flushed between windows. Every row is checked."""
    _case(f"q4_K k={k} n={n} m={m}")
    ty = ggml.Type.Q4_K
    w = make_weights(ty, k, n, 1, seed=n + 7 * m, device=gpu)
    x = normal((m, k), n + m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q4_K k={k} n={n} m={m}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8, 9, 16, 17, 32])
def test_gemv_columns(gpu, tname, m):
    _case(f"{tname} m={m}")
    ty = TYPES[tname]
    k, n = 2048, 300
    w = make_weights(ty, k, n, 1, seed=m, device=gpu)
    x = normal((m, k), 100 + m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"{tname} m={m}")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("m", [3, 4, 20])
def test_gemv_broadcast_and_strides(gpu, tname, m):
    """a [K, N, 2] broadcast over b [K, M, 4] (i02 = i12 / 2); b rows strided; dst a strided view. Q4_K at
    4 and 20 columns takes the skinny kernel (F32 activations quantized in the workgroup, then Q8_K)."""
    _case(f"{tname} broadcast m={m}")
    ty = TYPES[tname]
    k, n = 512, 40
    w = make_weights(ty, k, n, 2, seed=5, device=gpu)
    xb = normal((4, m, k + 64), 6)
    xt = torch.from_numpy(xb).to(gpu)[:, :, 32:32 + k]
    out_big = torch.full((4, m, n + 8), float("nan"), device=gpu)
    out = out_big[:, :, :n]
    ggml.mul_mat(w, xt, out=out)
    got = out_big.cpu().numpy()
    assert np.all(np.isnan(got[:, :, n:])), "wrote outside dst"
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, np.ascontiguousarray(xb[:, :, 32:32 + k]), ne2=2)
    check(got[:, :, :n], want, f"{tname} broadcast m={m}")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_gemv_golden(gpu, tname):
    _case(f"{tname} golden")
    g = np.load(os.path.join(GOLDEN, f"gemv_{tname}.npz"))
    k, n = int(g["k"]), int(g["n"])
    w = ggml.QTensor(TYPES[tname], (k, n), torch.from_numpy(g["w"]).to(gpu))
    y = ggml.mul_mat(w, torch.from_numpy(g["x"]).to(gpu)).cpu().numpy()
    check(y, g["y"], f"{tname} golden")


def test_workspace_argument(gpu):
    """Decode-size activations are quantized inside the GEMV workgroups and need no workspace; larger
    ones need the reported size and a smaller workspace is rejected."""
    _case("workspace")
    ty = ggml.Type.Q4_K
    w = make_weights(ty, 1024, 64, 1, seed=7, device=gpu)
    small = torch.from_numpy(normal((2, 1024), 8)).to(gpu)
    assert ggml.mul_mat_workspace_size(w, small) == 0
    x = torch.from_numpy(normal((20, 1024), 9)).to(gpu)
    need = ggml.mul_mat_workspace_size(w, x)
    assert need >= 20 * 4 * 292
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    a = ggml.mul_mat(w, x, workspace=ws)
    b = ggml.mul_mat(w, x)
    assert torch.equal(a, b)
    with pytest.raises(ggml.Compute):
        ggml.mul_mat(w, x, workspace=ws[: need // 2])


def test_dequantize_matches_oracle(gpu):
    _case("to_f32")
    for ty in (ggml.Type.Q4_K, ggml.Type.Q6_K):
        w = make_weights(ty, 1024, 16, 1, seed=9, device=gpu)
        got = ggml.to_f32(ty, w.data, 1024 * 16).cpu().numpy()
        want = O.dequantize(ty.id, w.data.cpu().numpy(), 1024 * 16)
        np.testing.assert_array_equal(got, want)


def test_device_quantizer_round_trip(gpu):
    """The device weight quantizer writes valid blocks whose round-trip error shrinks with bits
    (crates/ggml-sys/src/ggml/quant.rs:114-130)."""
    _case("quantizer round trip")
    src = torch.randn((64, 2048), device=gpu) * 0.02
    errs = []
    for ty in (ggml.Type.Q4_K, ggml.Type.Q6_K):
        raw = ggml.quantize(ty, src, 64, 2048)
        back = torch.from_numpy(O.dequantize(ty.id, raw.cpu().numpy(), 64 * 2048)).to(gpu).view(64, 2048)
        rel = float(((back - src).pow(2).mean() / src.pow(2).mean()).sqrt())
        errs.append(rel)
    assert errs[0] < 0.15 and errs[1] < 0.05 and errs[1] < errs[0], errs


@pytest.mark.parametrize("m", [1, 2, 4])
def test_q6_K_output_head_full_size(gpu, m):
    """The Q6_K output head 151936 x 2048 at its real size (the GEMV at 1 column, the Q6_K MFMA kernel at
    2 and 4); a seeded sample of 2048 rows against the oracle (the whole matrix is 255 MB)."""
    _case(f"q6_K head m={m}")
    ty = ggml.Type.Q6_K
    k, n = 2048, 151936
    w = make_weights(ty, k, n, 1, seed=1234, device=gpu)
    x = normal((m, k), 4321 + m)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    rows = np.sort(np.random.default_rng(0).choice(n, 2048, replace=False))
    rb = ty.row_size(k)
    sub = w.data.view(n, rb)[torch.from_numpy(rows).to(gpu)].cpu().numpy().reshape(-1)
    want = O.mul_mat(ty.id, sub, k, len(rows), x)[0]
    check(y[:, rows], want, f"q6_K head m={m}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("m", [1, 2, 4, 16, 32])
def test_attention_projections(gpu, m):
    """q_proj 2048->4096, k/v_proj 2048->512, o_proj 4096->2048, Q4_K, at decode batch m."""
    ty = ggml.Type.Q4_K
    for name, k, n in (("q", 2048, 4096), ("k", 2048, 512), ("v", 2048, 512), ("o", 4096, 2048)):
        _case(f"attn {name} m={m}")
        w = make_weights(ty, k, n, 1, seed=n + k + m, device=gpu)
        x = normal((m, k), m + k)
        y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
        want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
        check(y, want, f"{name}_proj m={m}")


@pytest.mark.parametrize("k,n,m", [(12288, 100, 20), (4096, 2048, 64), (256, 17, 4), (768, 2048, 33)])
def test_q4_K_batched_decode_shapes(gpu, k, n, m):
    """Q4_K with 4..64 columns runs the skinny MFMA kernel: long rows (48 super-blocks over 8 waves), a row
    count that is no multiple of its 16-row tiles, and a column count that is no multiple of 16."""
    _case(f"q4_K skinny k={k} n={n} m={m}")
    ty = TYPES["q4_K"]
    w = make_weights(ty, k, n, 1, seed=k + n + m, device=gpu)
    x = normal((m, k), 7 * m + k)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q4_K k={k} n={n} m={m}")


@pytest.mark.parametrize("n,m", [(17, 3), (17, 4), (300, 7), (4101, 13), (2048, 16), (5000, 20), (1000, 32), (1000, 33),
                                 (4101, 48), (512, 64), (700, 65), (300, 100)])
def test_q6_K_batched_decode_shapes(gpu, n, m):
    """Q6_K at K = 2048 with 3..64 columns (below 64K rows) runs the Q6_K MFMA kernel (16 columns per
    launch, up to 8 of them quantized inside it), from 65 the prefill kernel: row counts that are no
    multiple of the 16-row tiles, fewer tiles than workgroups and several tiles per workgroup, column
    counts that are no multiple of 4."""
    _case(f"q6_K skinny n={n} m={m}")
    ty = TYPES["q6_K"]
    k = 2048
    w = make_weights(ty, k, n, 1, seed=n + m, device=gpu)
    x = normal((m, k), 11 * m + n)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q6_K k={k} n={n} m={m}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("k,m", [(2048, 4), (2048, 13), (4096, 5), (4096, 11)])
def test_q6_K_skinny_broadcast_and_strides(gpu, k, m):
    """The Q6_K MFMA kernel over batches: a [k, 40, 2] broadcast over b [k, m, 4] (i02 = i12 / 2), b rows
    strided and 4-byte aligned only, dst a strided view whose padding must stay untouched."""
    _case(f"q6_K skinny broadcast k={k} m={m}")
    ty = TYPES["q6_K"]
    n = 40
    w = make_weights(ty, k, n, 2, seed=9, device=gpu)
    xb = normal((4, m, k + 68), 10)
    xt = torch.from_numpy(xb).to(gpu)[:, :, 33:33 + k]
    out_big = torch.full((4, m, n + 8), float("nan"), device=gpu)
    out = out_big[:, :, :n]
    ggml.mul_mat(w, xt, out=out)
    got = out_big.cpu().numpy()
    assert np.all(np.isnan(got[:, :, n:])), "wrote outside dst"
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, np.ascontiguousarray(xb[:, :, 33:33 + k]), ne2=2)
    check(got[:, :, :n], want, f"q6_K skinny broadcast k={k} m={m}")


@pytest.mark.parametrize("m", [6, 40])
def test_q6_K_skinny_dynamic_range_and_zero_columns(gpu, m):
    """The Q6_K MFMA kernel with columns scaled over 1e-30 .. 1e30 and all-zero columns (Q8_K d = 0),
    quantized inside the kernel (6 columns) and by the Q8_K pass (40)."""
    _case(f"q6_K skinny dynamic range m={m}")
    ty = TYPES["q6_K"]
    k, n = 2048, 100
    w = make_weights(ty, k, n, 1, seed=12, device=gpu)
    x = normal((m, k), 13)
    x *= (10.0 ** np.linspace(-30, 30, m)).astype(np.float32)[:, None]
    x[1] = 0.0
    x[m - 2] = 0.0
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    assert np.all(y[1] == 0) and np.all(y[m - 2] == 0)
    for i in range(m):  # each column against its own magnitude
        if i not in (1, m - 2):
            check(y[i], want[i], f"q6_K column {i}")


@pytest.mark.parametrize("n,m", [(17, 3), (300, 4), (4101, 8), (1000, 13), (2048, 32), (1000, 2), (700, 48), (700, 49)])
def test_q6_K_k4096_batched_decode_shapes(gpu, n, m):
    """Q6_K at K = 4096: the Q6_K MFMA kernel with two super-blocks per wave (8 columns per launch, the
    activations staged in the second tile buffer) up to 48 columns, the prefill kernel from 49, and the
    GEMV at 2 columns on a small matrix."""
    _case(f"q6_K k=4096 n={n} m={m}")
    ty = TYPES["q6_K"]
    k = 4096
    w = make_weights(ty, k, n, 1, seed=3 * n + m, device=gpu)
    x = normal((m, k), 5 * m + n)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy()
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q6_K k={k} n={n} m={m}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("k,n,m,q8", [(2048, 4101, 5, False), (4096, 8200, 20, False), (2048, 20000, 64, False),
                                      (4096, 4096, 4, True), (2048, 20000, 3, False), (4096, 16400, 4, False)])
def test_q4_K_persistent_skinny_shapes(gpu, k, n, m, q8):
    """Q4_K at K = 2048 / 4096 with 256 and more row tiles runs the persistent skinny kernel (tiles
    streamed two at a time per workgroup, activation operands held in registers): a partial last tile,
    two super-blocks per wave with two column tiles, four column tiles, Q8_K columns given as such, and
    3 / 4 F32 columns on matrices of 16K rows and more (smaller ones keep those on the GEMV)."""
    _case(f"q4_K persistent skinny k={k} n={n} m={m} q8={q8}")
    ty = TYPES["q4_K"]
    w = make_weights(ty, k, n, 1, seed=k + 3 * n + m, device=gpu)
    x = normal((m, k), 13 * m + n)
    xt = torch.from_numpy(x).to(gpu)
    if q8:
        xt = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(xt).view(-1))
    y = ggml.mul_mat(w, xt).cpu().numpy().reshape(m, n)
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x)[0]
    check(y, want, f"q4_K k={k} n={n} m={m}")
    assert np.all(np.isfinite(y))


@pytest.mark.parametrize("k,n,m,ne2", [(2048, 4100, 65, 1), (4096, 4096, 128, 1), (2048, 1000, 96, 1),
                                       (2048, 4100, 100, 2), (2048, 4096, 129, 1)])
def test_q4_K_wide_skinny_shapes(gpu, k, n, m, ne2):
    """Q4_K below 16K rows with 65..128 columns runs the skinny kernels in 64-column launches, each on
    its part of the Q8_K columns (129 columns go to the prefill kernel): a partial last launch, the
    persistent and the per-tile kernel (1000 rows: fewer than 256 tiles), and batches of b broadcast
    over a [k, n, 1] matrix, so the batch stride of the Q8_K columns is the full column count."""
    _case(f"q4_K wide skinny k={k} n={n} m={m} ne2={ne2}")
    ty = TYPES["q4_K"]
    w = make_weights(ty, k, n, 1, seed=k + n + 5 * m, device=gpu)
    x = normal((ne2, m, k), 17 * m + n)
    y = ggml.mul_mat(w, torch.from_numpy(x).to(gpu)).cpu().numpy().reshape(ne2, m, n)
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, x, ne2=1).reshape(ne2, m, n)
    check(y, want, f"q4_K wide skinny k={k} n={n} m={m} ne2={ne2}")
    assert np.all(np.isfinite(y))


def test_q4_K_persistent_skinny_broadcast(gpu):
    """The persistent Q4_K kernel over batches: a [2048, 4100, 2] broadcast over b [2048, 9, 4], b rows
    strided, dst a strided view whose padding must stay untouched."""
    _case("q4_K persistent skinny broadcast")
    ty = TYPES["q4_K"]
    k, n, m = 2048, 4100, 9
    w = make_weights(ty, k, n, 2, seed=21, device=gpu)
    xb = normal((4, m, k + 64), 22)
    xt = torch.from_numpy(xb).to(gpu)[:, :, 32:32 + k]
    out_big = torch.full((4, m, n + 8), float("nan"), device=gpu)
    out = out_big[:, :, :n]
    ggml.mul_mat(w, xt, out=out)
    got = out_big.cpu().numpy()
    assert np.all(np.isnan(got[:, :, n:])), "wrote outside dst"
    want = O.mul_mat(ty.id, w.data.cpu().numpy(), k, n, np.ascontiguousarray(xb[:, :, 32:32 + k]), ne2=2)
    check(got[:, :, :n], want, "q4_K persistent skinny broadcast")
