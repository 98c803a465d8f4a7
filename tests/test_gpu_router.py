"""The MoE router (crates/model/src/qwen3moe.rs:2869-2887) on the GPU against the oracle's restatement of
ggml's CPU nodes (rms_norm, MUL_MAT with the F32 gate_inp, soft_max, argsort_top_k, get_rows, sum_rows,
clamp, div).

Bars: xn within 2e-6 relative (the same float32 operations; the squares summed in double on both
sides); probabilities and weights within 2e-6 absolute (the logits are float32 dots in another
summation order); ids equal, except where the oracle's probabilities of two candidates for a place are
within 1e-6 of each other (another summation order may swap them: the test then requires the GPU's
choice to be one of the tied candidates). The reference's own top-k case (crates/ggml-sys/tests/ggml.rs:
33-44) fixes the order exactly."""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal
from tests.test_gpu_mmid import make_experts

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[router] {name}", file=sys.stderr, flush=True)


def _inputs(T, n_embd=2048, E=128, seed=0):
    rng = np.random.default_rng(seed)
    x = normal((T, n_embd), 1000 + seed + T)
    norm = (1.0 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)
    gate = (0.02 * rng.standard_normal((E, n_embd))).astype(np.float32)
    return x, norm, gate


def _check_ids(got, want, probs):
    for t in range(want.shape[0]):
        for j in range(want.shape[1]):
            if got[t, j] == want[t, j]:
                continue
            p = probs[t]
            gap = abs(float(p[got[t, j]]) - float(p[want[t, j]]))
            assert gap <= 1e-6, f"token {t} place {j}: id {got[t, j]} vs {want[t, j]} (gap {gap:.2e})"


@pytest.mark.parametrize("T", [1, 4, 16, 40])
def test_router_matches_oracle(gpu, T):
    """Qwen3-30B-A3B shapes: n_embd 2048, 128 experts, top-8, rms eps 1e-6."""
    _case(f"T={T}")
    x, norm, gate = _inputs(T)
    xn, w, ids = ggml.moe_router(torch.from_numpy(x).to(gpu), torch.from_numpy(norm).to(gpu),
                                 torch.from_numpy(gate).to(gpu), 1e-6, 8)
    oxn, oprobs, ow, oids = O.router(x, norm, gate, 1e-6, 8)
    np.testing.assert_allclose(xn.cpu().numpy(), oxn, rtol=2e-6, atol=1e-7)
    got_ids = ids.cpu().numpy()
    _check_ids(got_ids, oids, oprobs)
    # the GPU's weights against the oracle's probabilities of the GPU's own choice
    sel = np.take_along_axis(oprobs, got_ids.astype(np.int64), axis=1)
    np.testing.assert_allclose(w.cpu().numpy()[:, :, 0], sel / sel.sum(axis=1, keepdims=True), rtol=0, atol=2e-6)
    if np.array_equal(got_ids, oids):
        np.testing.assert_allclose(w.cpu().numpy()[:, :, 0], ow, rtol=0, atol=2e-6)
    assert np.all(np.sort(got_ids, axis=1)[:, 1:] != np.sort(got_ids, axis=1)[:, :-1]), "an expert chosen twice"


def test_router_reference_top_k_case(gpu):
    """crates/ggml-sys/tests/ggml.rs:33-44: top-2 of [0.1, 0.9, 0.3, 0.5] is [1, 3], largest first."""
    _case("reference top-k case")
    x = torch.tensor([[2.0]], device=gpu)
    gate = torch.tensor([[0.1], [0.9], [0.3], [0.5]], device=gpu)
    _, w, ids = ggml.moe_router(x, torch.ones(1, device=gpu), gate, 1e-6, 2)
    assert ids.cpu().tolist() == [[1, 3]]
    _, probs, ow, _ = O.router(np.array([[2.0]], np.float32), np.ones(1, np.float32), gate.cpu().numpy(), 1e-6, 2)
    np.testing.assert_allclose(w.cpu().numpy()[0, :, 0], ow[0], rtol=0, atol=1e-6)


def test_router_ties_and_invalid_arguments(gpu):
    """Equal probabilities go to the lower id; n_used above n_expert is refused."""
    _case("ties and invalid arguments")
    x = torch.ones((2, 64), device=gpu)
    gate = torch.ones((5, 64), device=gpu)
    _, w, ids = ggml.moe_router(x, torch.ones(64, device=gpu), gate, 1e-6, 3)
    assert ids.cpu().tolist() == [[0, 1, 2], [0, 1, 2]]
    np.testing.assert_allclose(w.cpu().numpy()[:, :, 0], 1.0 / 3.0, rtol=1e-6)
    with pytest.raises(ggml.Compute):
        ggml.moe_router(x, torch.ones(64, device=gpu), gate, 1e-6, 6)


@pytest.mark.parametrize("T", [1, 16])
def test_router_feeds_the_moe_step_in_a_graph(gpu, T):
    """Router and summed MoE step on one stream with device-only hand-off, captured in a HIP graph and
    replayed three times (poisoned outputs between replays): each replay equals the eager run, whose
    step output equals the step run on the router's ids and weights taken separately."""
    _case(f"router + moe_ffn_sum T={T}")
    n_embd, n_ff, E = 2048, 768, 128
    x, norm, gate_inp = _inputs(T, seed=5)
    xt, nt, gt = (torch.from_numpy(a).to(gpu) for a in (x, norm, gate_inp))
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=61, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=62, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=63, device=gpu)
    wsr = torch.empty(max(1, ggml.moe_router_workspace_size(gt, xt)), dtype=torch.uint8, device=gpu)
    ids0 = torch.zeros((T, 8), dtype=torch.int32, device=gpu)
    wsm = torch.empty(max(1, ggml.moe_ffn_workspace_size(gate, xt.view(T, 1, n_embd), ids0)), dtype=torch.uint8,
                      device=gpu)
    out = torch.empty((T, n_embd), device=gpu)
    keep = {}

    def op():
        xn, w, ids = ggml.moe_router(xt, nt, gt, 1e-6, 8, workspace=wsr)
        keep["r"] = (xn, w, ids)
        ggml.moe_ffn_sum(gate, up, down, xn.view(T, 1, n_embd), ids, w, out=out, workspace=wsm)

    op()
    torch.cuda.synchronize()
    want = out.clone()
    xn, w, ids = (t.clone() for t in keep["r"])
    again = ggml.moe_ffn_sum(gate, up, down, xn.view(T, 1, n_embd), ids, w)
    torch.cuda.synchronize()
    assert torch.equal(again, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op()
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    assert ggml.moe_sync_errors(clear=True) == 0


def test_router_softmax_closed_form(gpu):
    """logits {0, ln 3, ln 4} (x = [1, 1], eps 0, one-hot gate rows) give probabilities {1/8, 3/8, 4/8}:
    top-2 is [2, 1] with weights {4/7, 3/7}."""
    _case("closed form")
    x = torch.ones((1, 2), device=gpu)
    gate = torch.tensor([[0.0, 0.0], [float(np.log(3.0)), 0.0], [0.0, float(np.log(4.0))]], device=gpu)
    xn, w, ids = ggml.moe_router(x, torch.ones(2, device=gpu), gate, 0.0, 2)
    assert torch.equal(xn, x)
    assert ids.cpu().tolist() == [[2, 1]]
    np.testing.assert_allclose(w.cpu().numpy()[0, :, 0], [4 / 7, 3 / 7], rtol=0, atol=2e-7)
