"""MUL_MAT_ID on the GPU against the oracle (ggml semantics with patch 0004's -1 rule).

Mirrors crates/ggml-sys/tests/mul_mat_id_skip.rs:220-274: types {q4_K, q6_K} x tokens {1, 8, 64, 512}
x b1 in {1, n_used}; k=512, n=64, 16 experts, 4 used, 30% of slots -1; a warm run with other ids first
leaves stale nonzero rows (:86-122). Checks: -1 rows exactly zero, the rest within 1e-3 of the largest
reference magnitude (the GPU and the oracle both quantize activations to Q8_K, so only fp32
accumulation order differs). Then the Qwen3-30B-A3B expert shapes with top-8 routing and 10% -1, the
expert-parallel rank share (other ranks' experts as -1), out-of-range ids and the golden fixtures.
"""
import os
import zlib
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import ggml
from tests.helpers import normal, xorshift_noise
from tests.test_oracle_mulmat import make_ids

pytestmark = pytest.mark.gpu
TOL = 1e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TYPES = {"q4_K": ggml.Type.Q4_K, "q6_K": ggml.Type.Q6_K}


def _case(name):
    print(f"[mmid] {name}", file=sys.stderr, flush=True)


def make_experts(ty, k, n, n_expert, seed, device, std=0.02):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((n_expert * n, k), generator=g, device=device) * std
    return ggml.QTensor(ty, (k, n, n_expert), ggml.quantize(ty, src, n_expert * n, k))


def check(got, want, ids, what):
    neg = ids < 0
    assert np.all(got[neg] == 0.0), f"{what}: a -1 slot has a nonzero row"
    assert not np.any(np.signbit(got[neg])), f"{what}: a -1 slot has -0.0"
    scale = max(float(np.abs(want).max()), 1e-6)
    worst = float(np.abs(got[~neg] - want[~neg]).max() / scale) if (~neg).any() else 0.0
    assert worst <= TOL, f"{what}: worst {worst:.2e} of the largest > {TOL:.0e}"
    return worst


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
@pytest.mark.parametrize("tokens", [1, 8, 64, 512])
@pytest.mark.parametrize("b1", [1, 4])
def test_mul_mat_id_negative_ids_match_oracle(gpu, tname, tokens, b1):
    _case(f"{tname} tokens={tokens} b1={b1}")
    ty = TYPES[tname]
    k, n, E, used = 512, 64, 16, 4
    rng = np.random.default_rng(0x9E3779B9 + tokens * 10 + b1)
    w = make_experts(ty, k, n, E, seed=tokens + b1, device=gpu, std=0.5)
    b = xorshift_noise(tokens * b1 * k, tokens * 7 + b1).reshape(tokens, b1, k)
    ids = make_ids(E, used, tokens, 30, rng)
    warm = make_ids(E, used, tokens, 0, rng)
    bt = torch.from_numpy(b).to(gpu)
    out = torch.empty((tokens, used, n), device=gpu)
    ggml.mul_mat_id(w, bt, torch.from_numpy(warm).to(gpu), out=out)  # stale nonzero rows
    ggml.mul_mat_id(w, bt, torch.from_numpy(ids).to(gpu), out=out)
    got = out.cpu().numpy()
    want = O.mul_mat_id(ty.id, w.data.cpu().numpy(), k, n, E, b, ids)
    check(got, want, ids, f"{tname} tokens={tokens} b1={b1}")


def qwen3_moe_ids(tokens, seed, neg_frac=0.1, n_expert=128, used=8):
    """top-8 of softmax over N(0,1) router logits, then neg_frac of the slots set to -1."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((tokens, n_expert)).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :used].astype(np.int32)
    ids[rng.random(ids.shape) < neg_frac] = -1
    return ids


@pytest.mark.parametrize("tokens", [1, 2, 4, 8, 16])
def test_qwen3_moe_shapes(gpu, tokens):
    """gate/up Q4_K [2048 -> 768] with one activation row per token; down Q6_K [768 -> 2048] with one
    activation row per slot; 128 experts, top-8, 10% -1."""
    ids = qwen3_moe_ids(tokens, seed=100 + tokens)
    idt = torch.from_numpy(ids).to(gpu)
    for name, ty, k, n, b1 in (("gate", ggml.Type.Q4_K, 2048, 768, 1), ("up", ggml.Type.Q4_K, 2048, 768, 1),
                               ("down", ggml.Type.Q6_K, 768, 2048, 8)):
        _case(f"qwen3 {name} tokens={tokens}")
        w = make_experts(ty, k, n, 128, seed={"gate": 11, "up": 12, "down": 13}[name] * 100 + tokens, device=gpu)
        b = normal((tokens, b1, k), tokens * 3 + b1)
        got = ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), idt).cpu().numpy()
        want = O.mul_mat_id(ty.id, w.data.cpu().numpy(), k, n, 128, b, ids)
        check(got, want, ids, f"qwen3 {name} tokens={tokens}")


@pytest.mark.parametrize("g", [2, 4, 8])
def test_expert_parallel_rank_share(gpu, g):
    """Rank 0 of g holds experts [0, 128/g); the other ranks' slots are -1 (mul_mat_id_skip.rs:352-372)."""
    _case(f"ep share g={g}")
    tokens = 64
    ids = qwen3_moe_ids(tokens, seed=7, neg_frac=0.0)
    local = 128 // g
    ids = np.where(ids < local, ids, -1).astype(np.int32)
    w = make_experts(ggml.Type.Q4_K, 2048, 768, 128, seed=3, device=gpu)
    b = normal((tokens, 1, 2048), 5)
    got = ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), torch.from_numpy(ids).to(gpu)).cpu().numpy()
    want = O.mul_mat_id(12, w.data.cpu().numpy(), 2048, 768, 128, b, ids)
    check(got, want, ids, f"ep g={g}")


def test_out_of_range_ids_give_zero_rows(gpu):
    _case("out of range ids")
    w = make_experts(ggml.Type.Q6_K, 256, 32, 4, seed=1, device=gpu)
    ids = np.array([[0, 7, 3, -5], [4, 1, -1, 2]], dtype=np.int32)  # 7 and 4 are >= n_expert
    b = normal((2, 1, 256), 2)
    got = ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), torch.from_numpy(ids).to(gpu)).cpu().numpy()
    valid = np.where((ids >= 0) & (ids < 4), ids, -1).astype(np.int32)
    want = O.mul_mat_id(14, w.data.cpu().numpy(), 256, 32, 4, b, valid)
    check(got, want, valid, "out of range")


def test_all_slots_negative(gpu):
    _case("all -1")
    w = make_experts(ggml.Type.Q4_K, 512, 16, 4, seed=1, device=gpu)
    ids = np.full((3, 2), -1, dtype=np.int32)
    out = torch.full((3, 2, 16), 7.0, device=gpu)
    ggml.mul_mat_id(w, torch.from_numpy(normal((3, 1, 512), 1)).to(gpu), torch.from_numpy(ids).to(gpu), out=out)
    assert torch.all(out == 0)


def test_same_expert_many_tokens(gpu):
    """One expert routed for all 40 tokens: more columns than one staging pass holds."""
    _case("one expert, 40 tokens")
    w = make_experts(ggml.Type.Q4_K, 1024, 48, 3, seed=2, device=gpu)
    ids = np.ones((40, 1), dtype=np.int32)
    b = normal((40, 1, 1024), 3)
    got = ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), torch.from_numpy(ids).to(gpu)).cpu().numpy()
    want = O.mul_mat_id(12, w.data.cpu().numpy(), 1024, 48, 3, b, ids)
    check(got, want, ids, "one expert")


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_mmid_golden(gpu, tname):
    _case(f"golden {tname}")
    g = np.load(os.path.join(GOLDEN, f"mmid_{tname}.npz"))
    k, n, E = int(g["k"]), int(g["n"]), int(g["E"])
    w = ggml.QTensor(TYPES[tname], (k, n, E), torch.from_numpy(g["w"]).to(gpu))
    got = ggml.mul_mat_id(w, torch.from_numpy(g["b"]).to(gpu), torch.from_numpy(g["ids"]).to(gpu)).cpu().numpy()
    check(got, g["y"], g["ids"], f"golden {tname}")


def test_mul_mat_id_workspace_argument(gpu):
    """Decode-size MUL_MAT_ID (up to 256 slots) routes in LDS and quantizes inside its workgroups: it
    reports no workspace and runs with none (nothing is allocated, so it is capture-safe). Above 256
    slots the reported size is needed and a smaller workspace is rejected."""
    _case("workspace")
    ty = ggml.Type.Q4_K
    k, n, E, used = 512, 64, 16, 4
    w = make_experts(ty, k, n, E, seed=11, device=gpu)
    rng = np.random.default_rng(12)
    ids_small = torch.from_numpy(make_ids(E, used, 8, 20, rng)).to(gpu)
    b_small = torch.from_numpy(normal((8, 1, k), 13)).to(gpu)
    assert ggml.mul_mat_id_workspace_size(w, b_small, ids_small) == 0
    a = ggml.mul_mat_id(w, b_small, ids_small, workspace=torch.empty(0, dtype=torch.uint8, device=gpu))
    want = O.mul_mat_id(ty.id, w.data.cpu().numpy(), k, n, E, b_small.cpu().numpy(), ids_small.cpu().numpy())
    check(a.cpu().numpy(), want, ids_small.cpu().numpy(), "decode size, no workspace")
    ids_big = torch.from_numpy(make_ids(E, used, 80, 20, rng)).to(gpu)
    b_big = torch.from_numpy(normal((80, 1, k), 14)).to(gpu)
    need = ggml.mul_mat_id_workspace_size(w, b_big, ids_big)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    c = ggml.mul_mat_id(w, b_big, ids_big, workspace=ws)
    d = ggml.mul_mat_id(w, b_big, ids_big)
    assert torch.equal(c, d)
    with pytest.raises(ggml.Compute):
        ggml.mul_mat_id(w, b_big, ids_big, workspace=ws[: need // 2])


@pytest.mark.parametrize("case", ["uniform_T128", "skew32_T128", "skew32_K4096_T128", "skew16_T128", "skew8_T256",
                                  "neg90_T512", "q6_K_T128"])
def test_mul_mat_id_prefill_routings(gpu, case):
    """MUL_MAT_ID above 256 slots at the Qwen3-30B-A3B gate shape (Q4_K 2048 -> 768, 128 experts, top-8), on
    the grouped MFMA kernel: uniform routing (about 8 tokens per expert, one 16-column chunk), every slot on
    32 experts (32 tokens each: one 32-column chunk, activations staged in LDS; at K = 4096 the chunk does
    not fit the LDS and the waves read the activations themselves), on 16 experts (64 tokens each: one
    64-column chunk), on 8 experts (128 each: two chunks), 90% -1 (a few tokens on most experts); and a
    Q6_K matrix (the grouped Q6_K MFMA kernel, 16-column chunks at K = 2048), all against the oracle."""
    _case(case)
    ty = ggml.Type.Q6_K if case.startswith("q6_K") else ggml.Type.Q4_K
    k = 4096 if "_K4096" in case else 2048
    n, E, used = 768, 128, 8
    T = int(case.split("_T")[1])
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    ids = np.zeros((T, used), dtype=np.int32)
    for t in range(T):
        pool = {"skew32": 32, "skew16": 16, "skew8": 8}.get(case.split("_")[0], E)
        ids[t] = rng.permutation(pool)[:used] if pool >= used else rng.integers(0, pool, used)
    if case.startswith("neg90"):
        ids[rng.random(ids.shape) < 0.9] = -1
    w = make_experts(ty, k, n, E, seed=T + 5, device=gpu)
    b = normal((T, 1, k), T + 6)
    out = torch.full((T, used, n), 5.0, device=gpu)
    ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), torch.from_numpy(ids).to(gpu), out=out)
    want = O.mul_mat_id(ty.id, w.data.cpu().numpy(), k, n, E, b, ids)
    check(out.cpu().numpy(), want, ids, case)


@pytest.mark.parametrize("case", ["uniform_T128", "uniform_T512", "skew16_T256", "neg90_T512"])
def test_mul_mat_id_q6_K_down_prefill(gpu, case):
    """The Qwen3-30B-A3B down projections at prefill size (Q6_K 768 -> 2048, 128 experts, top-8, one
    activation row per slot) on the grouped Q6_K MFMA kernel: about 8 and 32 tokens per expert (one 16- or
    32-column chunk), 128 tokens on each of 16 experts (four 32-column chunks), 90% -1."""
    _case(f"q6_K down {case}")
    ty = ggml.Type.Q6_K
    k, n, E, used = 768, 2048, 128, 8
    T = int(case.split("_T")[1])
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    ids = np.zeros((T, used), dtype=np.int32)
    for t in range(T):
        pool = 16 if case.startswith("skew16") else E
        ids[t] = rng.permutation(pool)[:used]
    if case.startswith("neg90"):
        ids[rng.random(ids.shape) < 0.9] = -1
    w = make_experts(ty, k, n, E, seed=T + 15, device=gpu)
    b = normal((T, used, k), T + 16)
    out = torch.full((T, used, n), 5.0, device=gpu)
    ggml.mul_mat_id(w, torch.from_numpy(b).to(gpu), torch.from_numpy(ids).to(gpu), out=out)
    want = O.mul_mat_id(ty.id, w.data.cpu().numpy(), k, n, E, b, ids)
    check(out.cpu().numpy(), want, ids, case)
