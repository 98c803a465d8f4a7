"""The backend module on the GPU: one decode layer of a Qwen3-MoE-shaped model (n_embd 2048, 128 experts,
top-8) as a node list (attention projections q/k/v/o as MUL_MAT, the router, the expert FFN summed over
slots, an output head as MUL_MAT), reserved once and computed on the backend's stream (the path of
Sched::compute / Backend::compute_async, crates/ggml-sys/src/ggml/sched.rs:112, backend.rs:262). Every
node's output equals the same entry point called on its own (bit for bit: the same kernels) and the
MUL_MAT nodes match the oracle; the compute records into a HIP graph whose replays reproduce it; a node
the backend does not take, or one needing more workspace than reserved, fails before anything of it
is issued."""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import backend as B, ggml
from tests.helpers import normal
from tests.test_gpu_mmid import make_experts

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[backend] {name}", file=sys.stderr, flush=True)


def q8(x):
    """x [m, k] float32 as the Q8_K tensor tq_quantize_q8_K makes of it."""
    return ggml.QTensor(ggml.Type.Q8_K, (x.shape[-1], x.shape[0]), ggml.quantize_q8_K(x).view(-1))


def make_weights(ty, k, n, seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((n, k), generator=g, device=device) * 0.02
    return ggml.QTensor(ty, (k, n), ggml.quantize(ty, src, n, k))


def layer(gpu, T):
    n_embd, n_ff, E, vocab = 2048, 768, 128, 32000
    W = {"q": make_weights(ggml.Type.Q4_K, n_embd, 4096, 1, gpu), "k": make_weights(ggml.Type.Q4_K, n_embd, 512, 2, gpu),
         "v": make_weights(ggml.Type.Q4_K, n_embd, 512, 3, gpu), "o": make_weights(ggml.Type.Q4_K, 4096, n_embd, 4, gpu),
         "head": make_weights(ggml.Type.Q6_K, n_embd, vocab, 5, gpu)}
    gate = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=6, device=gpu)
    up = make_experts(ggml.Type.Q4_K, n_embd, n_ff, E, seed=7, device=gpu)
    down = make_experts(ggml.Type.Q6_K, n_ff, n_embd, E, seed=8, device=gpu)
    gate_inp = torch.from_numpy((0.02 * np.random.default_rng(9).standard_normal((E, n_embd))).astype(np.float32)).to(gpu)
    norm = torch.from_numpy((1 + 0.1 * np.random.default_rng(10).standard_normal(n_embd)).astype(np.float32)).to(gpu)
    x = torch.from_numpy(normal((T, n_embd), 11)).to(gpu)
    attn = torch.from_numpy(normal((T, 4096), 12)).to(gpu)
    nq, nk, nv = B.mul_mat(W["q"], x), B.mul_mat(W["k"], x), B.mul_mat(W["v"], x)
    no = B.mul_mat(W["o"], attn)
    nr = B.moe_router(no.out, norm, gate_inp, 1e-6, 8)
    xn, w, ids = nr.out
    nm = B.moe_ffn_sum(gate, up, down, xn.view(T, 1, n_embd), ids, w)
    nh = B.mul_mat(W["head"], nm.out)
    nodes = [nq, nk, nv, no, nr, nm, nh]
    return nodes, W, (gate, up, down, gate_inp, norm, x, attn)


@pytest.mark.parametrize("T", [1, 4, 16])
def test_decode_layer_through_the_backend(gpu, T):
    _case(f"layer T={T}")
    assert B.Backend.gpu_count() >= 1
    be = B.Backend.gpu(0)
    assert "gfx950" in be.description()
    nodes, W, (gate, up, down, gate_inp, norm, x, attn) = layer(gpu, T)
    for n in nodes:
        assert B.supports(n)
    be.reserve(nodes)
    be.compute_async(nodes)
    be.synchronize()
    nq, nk, nv, no, nr, nm, nh = nodes
    # each node against its entry point called alone, on the node's own inputs
    torch.cuda.synchronize()
    # (q/k/v share one Q8_K pass from 4 columns: each equals tq_mul_mat on the Q8_K rows of x)
    for n, w, inp in ((nq, W["q"], x), (nk, W["k"], x), (nv, W["v"], x), (no, W["o"], attn), (nh, W["head"], nm.out)):
        ref = ggml.mul_mat(w, q8(inp) if inp is x and T >= 4 else inp).reshape(n.out.shape)
        assert torch.equal(n.out, ref), "MUL_MAT node differs from tq_mul_mat"
    xn, wts, ids = ggml.moe_router(no.out, norm, gate_inp, 1e-6, 8)
    assert torch.equal(nr.out[0], xn) and torch.equal(nr.out[1], wts) and torch.equal(nr.out[2], ids)
    y = ggml.moe_ffn_sum(gate, up, down, nr.out[0].view(T, 1, -1), nr.out[2], nr.out[1])
    assert torch.equal(nm.out, y), "MoE node differs from tq_moe_ffn_sum"
    # the MUL_MAT nodes against the oracle
    for n, w, inp in ((nq, W["q"], x), (no, W["o"], attn)):
        want = O.mul_mat(w.type.id, w.data.cpu().numpy(), w.ne[0], w.ne[1], inp.cpu().numpy())[0]
        got = n.out.cpu().numpy()
        assert float(np.abs(got - want).max() / np.abs(want).max()) <= 1e-3
    be.close()


@pytest.mark.parametrize("T", [2, 16])
def test_backend_compute_in_a_graph(gpu, T):
    """A reserved compute records into a HIP graph (nothing allocated, no host synchronization); three
    replays, with the outputs poisoned and other work on the stream between them, equal the eager run
    (at 16 columns q/k/v share one Q8_K pass)."""
    _case(f"graph capture T={T}")
    nodes, W, _ = layer(gpu, T)
    be = B.Backend.gpu(0)
    be.reserve(nodes)
    be.compute_async(nodes)
    be.synchronize()
    eager = [[t.clone() for t in (n.dsts)] for n in nodes]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=be.stream):
        be.compute_async(nodes)
    for rep in range(3):
        for n in nodes:
            for t in n.dsts:
                t.fill_(-7 if t.dtype == torch.int32 else float("nan"))
        ggml.mul_mat(W["q"], torch.randn((3, 2048), device=gpu))  # other work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, ref in zip(nodes, eager):
            for t, r in zip(n.dsts, ref):
                assert torch.equal(t, r), f"replay {rep}: node op {n.op} differs from the eager compute"
    be.close()


@pytest.mark.parametrize("T", [2, 4, 8, 16, 40])
def test_backend_shared_q8_pass(gpu, T):
    """Consecutive MUL_MAT nodes on one F32 b share one Q8_K pass (Q4_K from 4 columns, Q6_K from 9),
    each bit for bit tq_mul_mat on the Q8_K rows of b; at 2 columns and for the Q6_K node up to 8 the
    nodes run alone, bit for bit tq_mul_mat on the F32 b. A node that writes its output over b ends the
    run: the nodes after it read the new b, as in node order."""
    _case(f"shared q8 pass T={T}")
    be = B.Backend.gpu(0)
    wq, wk, wv = (make_weights(ggml.Type.Q4_K, 2048, n, 30 + n, gpu) for n in (4096, 512, 512))
    wsq = make_weights(ggml.Type.Q4_K, 2048, 2048, 31, gpu)
    w6 = make_weights(ggml.Type.Q6_K, 2048, 1000, 32, gpu)
    x = torch.from_numpy(normal((T, 2048), 33 + T)).to(gpu)
    x0 = x.clone()
    nodes = [B.mul_mat(wq, x), B.mul_mat(wk, x), B.mul_mat(w6, x), B.mul_mat(wv, x),
             B.mul_mat(wsq, x, out=x),  # writes over b
             B.mul_mat(wk, x), B.mul_mat(wv, x)]
    be.reserve(nodes)
    be.compute_async(nodes)
    be.synchronize()
    torch.cuda.synchronize()
    def ref(w, b):
        shared = T >= 9 or (T >= 4 and w.type == ggml.Type.Q4_K)
        return ggml.mul_mat(w, q8(b) if shared else b).reshape(b.shape[0], w.ne[1])

    for n, w in zip(nodes[:4], (wq, wk, w6, wv)):
        assert torch.equal(n.out, ref(w, x0)), "node differs from tq_mul_mat"
    x1 = ref(wsq, x0)
    assert torch.equal(x, x1)
    for n, w in zip(nodes[5:], (wk, wv)):
        assert torch.equal(n.out, ref(w, x1)), "node after the overwrite did not read the new b"
    want = O.mul_mat(wq.type.id, wq.data.cpu().numpy(), 2048, 4096, x0.cpu().numpy())[0]
    got = nodes[0].out.cpu().numpy()
    assert float(np.abs(got - want).max() / np.abs(want).max()) <= 1e-3
    be.close()


def test_backend_refusals(gpu):
    _case("refusals")
    be = B.Backend.gpu(0)
    w = make_weights(ggml.Type.Q4_K, 2048, 512, 21, gpu)
    small = B.mul_mat(w, torch.randn((1, 2048), device=gpu))
    big = B.mul_mat(w, torch.randn((300, 2048), device=gpu))  # needs a Q8_K copy in the workspace
    be.reserve([small])
    with pytest.raises(ggml.Compute, match="node 1"):
        be.compute_async([small, big])
    bad = B.mul_mat(w, torch.randn((1, 1024), device=gpu))
    with pytest.raises(ggml.Compute, match="not supported"):
        be.reserve([small, bad])
    be.reserve([small, big])
    be.compute_async([small, big])
    be.synchronize()
    assert torch.equal(big.out, ggml.mul_mat(w, big.srcs[1]))
    be.close()
