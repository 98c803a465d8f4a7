"""The backend module's supports_node answers without a GPU (the shape checks touch no device, as ggml's
supports_op sees unallocated tensors): MUL_MAT / MUL_MAT_ID over Q4_K and Q6_K with F32 (or Q8_K) b, the
Qwen3-MoE router and expert FFN nodes, and refusals for other types, mismatched shapes and unknown ops
(the scheduler then gives the node to another backend)."""
import ctypes as C

import torch

from tetraeder_amd import _lib, backend as B
from tetraeder_amd.ggml import QTensor, Type


def q(ty, k, n, e=1):
    return QTensor(ty, (k, n, e), torch.zeros(ty.row_size(k) * n * e, dtype=torch.uint8))


def test_registry_name():
    assert _lib.lib().tq_backend_reg_name() == b"TQ-HIP"
    assert B.Backend.gpu_count() >= 0


def test_mul_mat_nodes():
    x = torch.zeros((4, 2048))
    assert B.supports(B.mul_mat(q(Type.Q4_K, 2048, 4096), x))
    assert B.supports(B.mul_mat(q(Type.Q6_K, 2048, 512), x))
    assert not B.supports(B.mul_mat(q(Type.Q4_K, 4096, 4096), x))   # K mismatch
    n = B.mul_mat(q(Type.Q4_K, 2048, 64), x)
    raw = n.raw()
    raw.src[1].contents.type = 1                                     # F16 b: ggml keeps it
    assert not _lib.lib().tq_backend_supports_node(C.byref(raw))
    n = B.mul_mat(q(Type.Q4_K, 2048, 64), x)
    n.raw().src[0].contents.type = 8                                 # Q8_0 weights: not this backend's
    assert not _lib.lib().tq_backend_supports_node(C.byref(n.raw()))
    bad = B.Node(B.MUL_MAT, [q(Type.Q4_K, 2048, 64), x], [torch.zeros((4, 65))])  # dst shape
    assert not B.supports(bad)


def test_mul_mat_id_and_moe_nodes():
    E, n_embd, n_ff, T = 128, 2048, 768, 4
    gate, up, down = q(Type.Q4_K, n_embd, n_ff, E), q(Type.Q4_K, n_embd, n_ff, E), q(Type.Q6_K, n_ff, n_embd, E)
    b = torch.zeros((T, 1, n_embd))
    ids = torch.zeros((T, 8), dtype=torch.int32)
    w = torch.zeros((T, 8, 1))
    assert B.supports(B.mul_mat_id(gate, b, ids))
    assert B.supports(B.moe_ffn(gate, up, down, b, ids, w))
    assert B.supports(B.moe_ffn_sum(gate, up, down, b, ids, w))
    assert B.supports(B.moe_ffn_sum(gate, up, down, b, ids, None))
    assert not B.supports(B.moe_ffn(gate, up, q(Type.Q6_K, n_ff, 1024, E), b, ids, w))  # down rows != n_embd
    assert not B.supports(B.mul_mat_id(gate, torch.zeros((T + 1, 1, n_embd)), ids))    # b tokens != ids tokens
    assert B.supports(B.sum_experts(torch.zeros((T, 8, n_embd))))


def test_router_nodes():
    x = torch.zeros((4, 2048))
    norm = torch.zeros(2048)
    assert B.supports(B.moe_router(x, norm, torch.zeros((128, 2048)), 1e-6, 8))
    assert not B.supports(B.moe_router(x, norm, torch.zeros((128, 2048)), 1e-6, 65))   # n_used above 64
    assert not B.supports(B.moe_router(x, torch.zeros(1024), torch.zeros((128, 2048)), 1e-6, 8))


def test_unknown_op():
    assert not B.supports(B.Node(99, [], [torch.zeros(1)]))
