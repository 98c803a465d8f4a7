"""The fused MoE expert FFN (tq_moe_ffn) against the oracle's node sequence of weighted_experts
(crates/model/src/qwen3moe.rs:2899-2914): up and gate MUL_MAT_ID on the token rows, swiglu_split in fp32
(ggml's silu: x / (1 + exp(-x))), MUL_MAT_ID of down on the per-slot act rows, times the router weight.

Two bars. Per node with the same inputs (the 1e-3 of the largest magnitude that holds for every
MUL_MAT_ID): the down node is checked against the oracle fed with act built from the GPU's own gate/up
outputs. End to end against the all-CPU chain: act is a computed fp32 value whose Q8_K rounding flips
where the GPU's and the CPU's fp32 evaluations of it fall on both sides of a rounding boundary, and
each flip moves an output by about |w| * step; 3e-3 of the largest magnitude bounds that. -1 slots are
exact zeros in both."""
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
    print(f"[moe] {name}", file=sys.stderr, flush=True)


def oracle_moe(gate, up, down, x, ids, w, n_embd, n_ff, E):
    g = O.mul_mat_id(gate.type.id, gate.data.cpu().numpy(), n_embd, n_ff, E, x, ids)
    u = O.mul_mat_id(up.type.id, up.data.cpu().numpy(), n_embd, n_ff, E, x, ids)
    act = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    y = O.mul_mat_id(down.type.id, down.data.cpu().numpy(), n_ff, n_embd, E, act, ids)
    if w is not None:
        y = y * w
    y[ids < 0] = 0.0
    return y


def _setup(gpu, tokens, weighted):
    n_embd, n_ff, E = 2048, 768, 128
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=21, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=22, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=23, device=gpu)
    ids = qwen3_moe_ids(tokens, seed=300 + tokens)
    x = normal((tokens, 1, n_embd), 400 + tokens)
    w = np.random.default_rng(tokens).random((tokens, 8, 1)).astype(np.float32) if weighted else None
    out = torch.full((tokens, 8, n_embd), 3.0, device=gpu)  # stale values must not survive
    ggml.moe_ffn(gate, up, down, torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu),
                 torch.from_numpy(w).to(gpu) if weighted else None, out=out)
    return gate, up, down, ids, x, w, out.cpu().numpy(), (n_embd, n_ff, E)


@pytest.mark.parametrize("tokens", [1, 2, 4, 8, 16, 40])
@pytest.mark.parametrize("weighted", [False, True])
def test_moe_ffn_down_node(gpu, tokens, weighted):
    """Qwen3-30B-A3B: 128 experts, n_embd 2048, n_ff 768, gate/up Q4_K, down Q6_K, top-8, 10% -1.
    40 tokens (320 slots) runs the composed path. The down node against the oracle on act formed from
    the GPU's gate/up MUL_MAT_ID outputs."""
    _case(f"down node tokens={tokens} weighted={weighted}")
    gate, up, down, ids, x, w, got, (n_embd, n_ff, E) = _setup(gpu, tokens, weighted)
    xt, it = torch.from_numpy(x).to(gpu), torch.from_numpy(ids).to(gpu)
    g = ggml.mul_mat_id(gate, xt, it).cpu().numpy()
    u = ggml.mul_mat_id(up, xt, it).cpu().numpy()
    act = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    want = O.mul_mat_id(down.type.id, down.data.cpu().numpy(), n_ff, n_embd, E, act, ids)
    if w is not None:
        want = want * w
    want[ids < 0] = 0.0
    assert np.all(got[ids < 0] == 0.0)
    worst = float(np.abs(got - want).max() / np.abs(want).max())
    assert worst <= 1e-3, f"worst {worst:.2e} of the largest"


@pytest.mark.parametrize("tokens", [1, 16, 40])
def test_moe_ffn_end_to_end(gpu, tokens):
    _case(f"end to end tokens={tokens}")
    gate, up, down, ids, x, w, got, (n_embd, n_ff, E) = _setup(gpu, tokens, True)
    want = oracle_moe(gate, up, down, x, ids, w, n_embd, n_ff, E)
    assert np.all(got[ids < 0] == 0.0)
    worst = float(np.abs(got - want).max() / np.abs(want).max())
    assert worst <= 3e-3, f"worst {worst:.2e} of the largest"


def test_moe_ffn_matches_composed_ops(gpu):
    """The fused step equals its own nodes run one by one through mul_mat_id (same GPU arithmetic
    up to the act rounding into Q8_K)."""
    _case("fused vs composed")
    n_embd, n_ff, E, T = 512, 256, 16, 6
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=1, device=gpu)
    up = make_experts(ggml.Type.Q6_K, n_embd, n_ff, E, seed=2, device=gpu)
    down = make_experts(ggml.Type.Q4_K, n_ff, n_embd, E, seed=3, device=gpu)
    ids = torch.from_numpy(qwen3_moe_ids(T, 5, n_expert=E, used=4)).to(gpu)
    x = torch.from_numpy(normal((T, 1, n_embd), 6)).to(gpu)
    fused = ggml.moe_ffn(gate, up, down, x, ids)
    g = ggml.mul_mat_id(gate, x, ids)
    u = ggml.mul_mat_id(up, x, ids)
    act = (g / (1 + torch.exp(-g)) * u).contiguous()
    ref = ggml.mul_mat_id(down, act, ids)
    worst = float((fused - ref).abs().max() / ref.abs().max())
    assert worst <= 1e-3, worst


def test_moe_ffn_back_to_back_calls(gpu):
    """Consecutive single-launch steps with changing token counts and ids, on one stream with no host
    synchronization between them (as a decode loop issues them): each equals its own nodes run through
    mul_mat_id, so the cross-workgroup progress counters start from zero on every call, and no wait
    ran out."""
    _case("back to back")
    n_embd, n_ff, E = 2048, 768, 128
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=31, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=32, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=33, device=gpu)
    ggml.moe_sync_errors(clear=True)
    cases = []
    for i, T in enumerate((1, 16, 3, 1, 32, 8, 2, 1)):
        ids = torch.from_numpy(qwen3_moe_ids(T, seed=700 + i)).to(gpu)
        x = torch.from_numpy(normal((T, 1, n_embd), 800 + i)).to(gpu)
        w = torch.from_numpy(np.random.default_rng(i).random((T, 8, 1)).astype(np.float32)).to(gpu)
        cases.append((ids, x, w, ggml.moe_ffn(gate, up, down, x, ids, w)))
    torch.cuda.synchronize()
    assert ggml.moe_sync_errors() == 0
    for ids, x, w, fused in cases:
        g = ggml.mul_mat_id(gate, x, ids)
        u = ggml.mul_mat_id(up, x, ids)
        act = (g / (1 + torch.exp(-g)) * u).contiguous()
        ref = ggml.mul_mat_id(down, act, ids) * w
        ref[ids < 0] = 0.0
        assert bool((fused[ids < 0] == 0).all())
        worst = float((fused - ref).abs().max() / ref.abs().max())
        assert worst <= 3e-3, worst


def test_sum_experts_matches_oracle(gpu):
    """sum_experts on its own (qwen3moe.rs:2917-2923): bit-equal to the oracle's left-to-right fp32 fold,
    also on a strided view (every other slot of a wider tensor)."""
    _case("sum_experts")
    rng = np.random.default_rng(11)
    e = rng.standard_normal((6, 8, 2048)).astype(np.float32)
    got = ggml.sum_experts(torch.from_numpy(e).to(gpu)).cpu().numpy()
    np.testing.assert_array_equal(got, O.sum_experts(e))
    wide = torch.from_numpy(rng.standard_normal((3, 16, 2048)).astype(np.float32)).to(gpu)
    view = wide[:, ::2, :]
    got = ggml.sum_experts(view).cpu().numpy()
    np.testing.assert_array_equal(got, O.sum_experts(view.cpu().numpy()))
    # slot counts around the kernel's batch of 8 loads, and all -0.0 rows (a stand-in +0 would show)
    for n_used in (1, 7, 9, 11, 16):
        e2 = rng.standard_normal((2, n_used, 96)).astype(np.float32)
        e2[:, :, :5] = -0.0
        got = ggml.sum_experts(torch.from_numpy(e2).to(gpu)).cpu().numpy()
        np.testing.assert_array_equal(got, O.sum_experts(e2))
        assert np.all(np.signbit(got[:, :5])), f"n_used={n_used}: -0.0 sums lost their sign"


@pytest.mark.parametrize("tokens", [1, 2, 4, 16, 32, 40])
def test_moe_ffn_sum(gpu, tokens):
    """moe_ffn (qwen3moe.rs:2892-2895) = sum_experts(weighted_experts): the summed step equals the
    oracle's fold of the per-slot step's rows bit for bit (the slot rows are the same arithmetic); 40
    tokens (320 slots) runs the composed path and a sum launch. No wait ran out."""
    _case(f"moe_ffn_sum tokens={tokens}")
    n_embd, n_ff, E = 2048, 768, 128
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=41, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=42, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=43, device=gpu)
    ids = torch.from_numpy(qwen3_moe_ids(tokens, seed=900 + tokens)).to(gpu)
    x = torch.from_numpy(normal((tokens, 1, n_embd), 950 + tokens)).to(gpu)
    w = torch.from_numpy(np.random.default_rng(tokens).random((tokens, 8, 1)).astype(np.float32)).to(gpu)
    ggml.moe_sync_errors(clear=True)
    slots = ggml.moe_ffn(gate, up, down, x, ids, w)
    out = torch.full((tokens, n_embd), float("nan"), device=gpu)
    ggml.moe_ffn_sum(gate, up, down, x, ids, w, out=out)
    torch.cuda.synchronize()
    assert ggml.moe_sync_errors() == 0
    np.testing.assert_array_equal(out.cpu().numpy(), O.sum_experts(slots.cpu().numpy()))
    # again with every slot of one token skipped (-1): its sum is an exact zero row
    ids2 = ids.clone()
    ids2[0, :] = -1
    out2 = ggml.moe_ffn_sum(gate, up, down, x, ids2, w)
    slots2 = ggml.moe_ffn(gate, up, down, x, ids2, w)
    torch.cuda.synchronize()
    assert ggml.moe_sync_errors() == 0
    np.testing.assert_array_equal(out2.cpu().numpy(), O.sum_experts(slots2.cpu().numpy()))
    assert bool((out2[0] == 0).all())
