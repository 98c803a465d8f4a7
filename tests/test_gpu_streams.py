"""Calls in flight on several streams of one GPU at once, as the reference's executor issues them when
two backends share a GPU (crates/executor/tests/gpu.rs:16-18): the single-launch MoE step (whose
workgroups count each other's phases), a prefill MUL_MAT split along k (whose workgroups count tile
arrivals) and the router (per-token arrival counts) run concurrently on different streams, with no host
synchronization between the launches, and every result matches the oracle (or its own result computed
alone, bit for bit). Each stream holds its own counter block, so no call sees another's counts."""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal
from tests.test_gpu_mmid import make_experts, qwen3_moe_ids

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[streams] {name}", file=sys.stderr, flush=True)


def make_weights(ty, k, n, seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((n, k), generator=g, device=device) * 0.02
    return ggml.QTensor(ty, (k, n), ggml.quantize(ty, src, n, k))


def test_moe_split_and_router_on_three_streams(gpu):
    _case("moe + k split + router")
    n_embd, n_ff, E = 2048, 768, 128
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=51, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=52, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=53, device=gpu)
    # a Q6_K 12288 -> 4096 prefill MUL_MAT at 512 columns: 128 output tiles, split in two along k
    wp = make_weights(ggml.Type.Q6_K, 12288, 4096, seed=54, device=gpu)
    xp = torch.from_numpy(normal((512, 12288), 55)).to(gpu)
    gate_inp = torch.from_numpy((0.02 * np.random.default_rng(56).standard_normal((E, n_embd))).astype(np.float32)).to(gpu)
    norm = torch.ones(n_embd, device=gpu)
    T = 4
    ids = [torch.from_numpy(qwen3_moe_ids(T, seed=600 + i)).to(gpu) for i in range(6)]
    xs = [torch.from_numpy(normal((T, 1, n_embd), 700 + i)).to(gpu) for i in range(6)]
    rx = [torch.from_numpy(normal((16, n_embd), 800 + i)).to(gpu) for i in range(6)]

    # alone, one stream: the reference results
    ws_p = torch.empty(ggml.mul_mat_workspace_size(wp, xp), dtype=torch.uint8, device=gpu)
    ws_m = torch.empty(ggml.moe_ffn_workspace_size(gate, xs[0], ids[0]), dtype=torch.uint8, device=gpu)
    ws_r = torch.empty(max(1, ggml.moe_router_workspace_size(gate_inp, rx[0])), dtype=torch.uint8, device=gpu)
    alone_p = ggml.mul_mat(wp, xp, workspace=ws_p).clone()
    alone_m = [ggml.moe_ffn(gate, up, down, xs[i], ids[i], workspace=ws_m).clone() for i in range(6)]
    alone_r = [tuple(t.clone() for t in ggml.moe_router(rx[i], norm, gate_inp, 1e-6, 8, workspace=ws_r))
               for i in range(6)]
    torch.cuda.synchronize()

    # concurrently: three streams, each with its own workspaces and outputs, launched interleaved
    sp, sm, sr = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    ws_p2, ws_m2, ws_r2 = torch.empty_like(ws_p), torch.empty_like(ws_m), torch.empty_like(ws_r)
    out_p = [torch.empty_like(alone_p) for _ in range(3)]
    out_m = [torch.empty_like(alone_m[i]) for i in range(6)]
    out_r = []
    ggml.moe_sync_errors(clear=True)
    for i in range(6):
        if i % 2 == 0:
            with torch.cuda.stream(sp):
                ggml.mul_mat(wp, xp, out=out_p[i // 2], workspace=ws_p2, stream=sp)
        with torch.cuda.stream(sm):
            ggml.moe_ffn(gate, up, down, xs[i], ids[i], out=out_m[i], workspace=ws_m2, stream=sm)
        with torch.cuda.stream(sr):
            out_r.append(ggml.moe_router(rx[i], norm, gate_inp, 1e-6, 8, workspace=ws_r2, stream=sr))
    torch.cuda.synchronize()
    assert ggml.moe_sync_errors() == 0, "a MoE wait ran out"
    for i in range(3):
        assert torch.equal(out_p[i], alone_p), f"k-split MUL_MAT {i} differs from its result alone"
    for i in range(6):
        assert torch.equal(out_m[i], alone_m[i]), f"MoE step {i} differs from its result alone"
        for a, b in zip(out_r[i], alone_r[i]):
            assert torch.equal(a, b), f"router call {i} differs from its result alone"
    # and the results themselves against the oracle
    rows = np.sort(np.random.default_rng(0).choice(4096, 256, replace=False))
    rb = wp.type.row_size(12288)
    sub = wp.data.view(4096, rb)[torch.from_numpy(rows).to(gpu)].cpu().numpy().reshape(-1)
    want = O.mul_mat(wp.type.id, sub, 12288, len(rows), xp[:64].cpu().numpy())[0]
    got = out_p[0][:64][:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
    assert float(np.abs(got - want).max() / np.abs(want).max()) <= 1e-3
    for i in (0, 5):
        ids_np = ids[i].cpu().numpy()
        g = ggml.mul_mat_id(gate, xs[i], ids[i]).cpu().numpy()
        u = ggml.mul_mat_id(up, xs[i], ids[i]).cpu().numpy()
        act = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
        want = O.mul_mat_id(down.type.id, down.data.cpu().numpy(), n_ff, n_embd, E, act, ids_np)
        want[ids_np < 0] = 0.0
        got = out_m[i].cpu().numpy()
        assert np.all(got[ids_np < 0] == 0.0)
        assert float(np.abs(got - want).max() / np.abs(want).max()) <= 1e-3


def test_two_streams_same_split_matmul(gpu):
    """The same k-split MUL_MAT (Q6_K 12288 -> 4096 at 512 columns, split in two along k) on two streams at
    once, 4 launches each, outputs and workspaces separate: every output equals the single-stream result
    bit for bit (the split's partial sums are added in split order, so the bits do not depend on timing)."""
    _case("k split on two streams")
    wp = make_weights(ggml.Type.Q6_K, 12288, 4096, seed=61, device=gpu)
    xp = torch.from_numpy(normal((512, 12288), 62)).to(gpu)
    need = ggml.mul_mat_workspace_size(wp, xp)
    assert need > 512 * 48 * 292, "the shape no longer splits along k"
    ws = [torch.empty(need, dtype=torch.uint8, device=gpu) for _ in range(2)]
    alone = ggml.mul_mat(wp, xp, workspace=ws[0]).clone()
    s = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty_like(alone) for _ in range(4)] for _ in range(2)]
    torch.cuda.synchronize()
    for i in range(4):
        for j in range(2):
            with torch.cuda.stream(s[j]):
                ggml.mul_mat(wp, xp, out=outs[j][i], workspace=ws[j], stream=s[j])
    torch.cuda.synchronize()
    for j in range(2):
        for i in range(4):
            assert torch.equal(outs[j][i], alone), f"stream {j} launch {i}"
