"""Capture safety: every entry point, called with caller-provided outputs and workspaces, records into a
HIP graph (the decode-graph replay of the reference's patches 0005/0006) and each replay reproduces
the eager result bit for bit. Between replays the outputs are poisoned and other eager work runs on
the same stream, so a replay that skipped a node, depended on a memset, or left a device counter
unreset would show. The kernels are deterministic (fixed summation orders, the k split sums its
partial tiles in split order), so equality is exact."""
import sys

import numpy as np
import pytest
import torch

from tetraeder_amd import ggml
from tests.helpers import normal
from tests.test_gpu_gemv import make_weights
from tests.test_gpu_mmid import make_experts, qwen3_moe_ids

pytestmark = pytest.mark.gpu
REPLAYS = 3


def _case(name):
    print(f"[graph] {name}", file=sys.stderr, flush=True)


def _check_replays(op, outs, noise):
    """op() writes outs; capture it, then replay REPLAYS times against the eager result."""
    op()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op()
    for r in range(REPLAYS):
        for o in outs:
            o.fill_(float("nan"))
        noise()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), f"replay {r} differs from the eager result"
    del g


@pytest.mark.parametrize("tname,k,n,m", [("q6_K", 2048, 20000, 1), ("q4_K", 2048, 4096, 2), ("q4_K", 4096, 300, 4),
                                         ("q6_K", 2048, 1000, 6), ("q6_K", 2048, 1000, 12), ("q6_K", 4096, 700, 5),
                                         ("q6_K", 512, 300, 6),
                                         ("q4_K", 2048, 4096, 16), ("q4_K", 2048, 8192, 24)])
def test_mul_mat_decode_in_graph(gpu, tname, k, n, m):
    """Decode MUL_MAT: the LDS-streamed GEMV (batch 1..4), the register GEMV (Q6_K at K = 512, 6
    columns), the Q6_K MFMA kernel (K = 2048: 6 columns quantized inside it, 12 with the Q8_K pass in the
    workspace; K = 4096, 5 columns) and the skinny Q4_K MFMA kernels (16 and 24 columns, the second
    persistent, with the Q8_K pass in the workspace)."""
    _case(f"mul_mat {tname} k={k} n={n} m={m}")
    ty = ggml.Type.Q4_K if tname == "q4_K" else ggml.Type.Q6_K
    w = make_weights(ty, k, n, 1, seed=k + n + m, device=gpu)
    x = torch.from_numpy(normal((m, k), 31 * m + n)).to(gpu)
    out = torch.empty((m, n), device=gpu)
    ws = torch.empty(max(1, ggml.mul_mat_workspace_size(w, x)), dtype=torch.uint8, device=gpu)
    other_w = make_weights(ty, k, 64, 1, seed=7, device=gpu)
    other_out = torch.empty((m, 64), device=gpu)
    _check_replays(lambda: ggml.mul_mat(w, x, out=out, workspace=ws), [out],
                   lambda: ggml.mul_mat(other_w, x, out=other_out, workspace=ws))


@pytest.mark.parametrize("tname,k,n,m", [("q4_K", 4096, 1024, 256), ("q6_K", 12288, 512, 128)])
def test_mul_mat_prefill_in_graph(gpu, tname, k, n, m):
    """Prefill MUL_MAT on the tile kernels; both shapes have few output tiles, so the k split (partial
    tiles in the workspace, device arrival counts reset by the last workgroup) is part of the graph."""
    _case(f"prefill {tname} k={k} n={n} m={m}")
    ty = ggml.Type.Q4_K if tname == "q4_K" else ggml.Type.Q6_K
    w = make_weights(ty, k, n, 1, seed=k + n, device=gpu)
    x = torch.from_numpy(normal((m, k), m + k)).to(gpu)
    out = torch.empty((m, n), device=gpu)
    ws = torch.empty(max(1, ggml.mul_mat_workspace_size(w, x)), dtype=torch.uint8, device=gpu)
    x2 = torch.from_numpy(normal((m, k), 5)).to(gpu)
    out2 = torch.empty((m, n), device=gpu)
    _check_replays(lambda: ggml.mul_mat(w, x, out=out, workspace=ws), [out],
                   lambda: ggml.mul_mat(w, x2, out=out2, workspace=ws))


@pytest.mark.parametrize("tokens", [1, 16])
def test_mul_mat_id_and_moe_ffn_in_graph(gpu, tokens):
    """MUL_MAT_ID with device routing and the one-launch MoE step, per slot and summed over the slots
    (the step's phase-1 completion counts and exit count live on the device and are reset by the
    call's last workgroup), Qwen3-30B-A3B shapes, 10% of the ids -1."""
    _case(f"moe tokens={tokens}")
    n_embd, n_ff, E = 2048, 768, 128
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=51, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=52, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=53, device=gpu)
    ids = torch.from_numpy(qwen3_moe_ids(tokens, seed=600 + tokens)).to(gpu)
    ids2 = torch.from_numpy(qwen3_moe_ids(tokens, seed=700 + tokens)).to(gpu)
    x = torch.from_numpy(normal((tokens, 1, n_embd), 800 + tokens)).to(gpu)
    rw = torch.from_numpy(np.random.default_rng(tokens).random((tokens, 8, 1)).astype(np.float32)).to(gpu)
    out_id = torch.empty((tokens, 8, n_ff), device=gpu)
    ws_id = torch.empty(max(1, ggml.mul_mat_id_workspace_size(gate, x, ids)), dtype=torch.uint8, device=gpu)
    out_ffn = torch.empty((tokens, 8, n_embd), device=gpu)
    ws_ffn = torch.empty(max(1, ggml.moe_ffn_workspace_size(gate, x, ids)), dtype=torch.uint8, device=gpu)
    out_noise = torch.empty((tokens, 8, n_embd), device=gpu)
    out_sum = torch.empty((tokens, n_embd), device=gpu)

    def op():
        ggml.mul_mat_id(gate, x, ids, out=out_id, workspace=ws_id)
        ggml.moe_ffn(gate, up, down, x, ids, rw, out=out_ffn, workspace=ws_ffn)
        ggml.moe_ffn_sum(gate, up, down, x, ids, rw, out=out_sum, workspace=ws_ffn)

    # the noise runs the same step on other ids: the device counters must be back at zero after it
    _check_replays(op, [out_id, out_ffn, out_sum],
                   lambda: ggml.moe_ffn(gate, up, down, x, ids2, rw, out=out_noise, workspace=ws_ffn))
    assert ggml.moe_sync_errors(clear=True) == 0
