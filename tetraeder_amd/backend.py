"""The backend module of libtq (include/tq.h, `tq_backend_*`) for Python hosts.

Mirrors the reference's backend handles over ggml's module registry: ``Backend.gpu(i)`` and
``Backend.gpu_count()`` (crates/ggml-sys/src/ggml/backend.rs:174-205, 244-258), ``Backend.compute_async``
and ``Backend.synchronize`` (backend.rs:262-283), and the scheduler's ``reserve`` (sched.rs:63-77), whose
compute buffers are sized once so later computes allocate nothing. A graph is a list of ``Node``s built
by the functions below, with ggml's operand order and shapes (``mul_mat``, ``mul_mat_id``: context.rs:
294-299, 320-336; the Qwen3-MoE router and expert FFN: crates/model/src/qwen3moe.rs:2869-2923). Torch
provides device memory and streams only; there is no fallback: ``supports`` answering False means
another backend (ggml's) must take the node.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .ggml import Compute, Invalid, QTensor, Type, _dense

MUL_MAT, MUL_MAT_ID, MOE_ROUTER, MOE_FFN, MOE_FFN_SUM, SUM_EXPERTS = 1, 2, 3, 4, 5, 6


class Node:
    """One graph node: operator, sources, destinations (torch tensors or QTensors) and parameters."""

    def __init__(self, op: int, srcs, dsts, f_param: float = 0.0, i_param: int = 0):
        self.op, self.srcs, self.dsts = op, list(srcs), list(dsts)
        self.f_param, self.i_param = float(f_param), int(i_param)
        self._raw = None

    def raw(self) -> _lib.TqNode:
        if self._raw is None:
            n = _lib.TqNode()
            n.op = self.op
            keep = []
            for i, t in enumerate(self.srcs):
                if t is not None:
                    r = _as_raw(t)
                    keep.append(r)
                    n.src[i] = C.pointer(r)
            for i, t in enumerate(self.dsts):
                r = _as_raw(t)
                keep.append(r)
                n.dst[i] = C.pointer(r)
            n.f_param, n.i_param = self.f_param, self.i_param
            self._raw, self._keep = n, keep
        return self._raw

    @property
    def out(self):
        return self.dsts[0] if len(self.dsts) == 1 else tuple(self.dsts)


def _as_raw(t) -> _lib.TqTensor:
    if isinstance(t, QTensor):
        return t.raw()
    if t.dtype == torch.float32:
        return _dense(t, Type.F32)
    if t.dtype == torch.int32:
        return _dense(t, Type.I32)
    raise Invalid(f"tensor of dtype {t.dtype} in a node")


def mul_mat(a: QTensor, b: torch.Tensor, out: torch.Tensor | None = None) -> Node:
    """MUL_MAT: a [K, N] quantized, b float32 [..., M, K] -> out [..., M, N]."""
    if out is None:
        out = torch.empty(tuple(b.shape[:-1]) + (a.ne[1],), dtype=torch.float32, device=b.device)
    return Node(MUL_MAT, [a, b], [out])


def mul_mat_id(experts: QTensor, b: torch.Tensor, ids: torch.Tensor, out: torch.Tensor | None = None) -> Node:
    """MUL_MAT_ID: experts [K, N, n_expert], b float32 [T, ne11, K], ids int32 [T, n_used] -> [T, n_used, N]."""
    if out is None:
        out = torch.empty((ids.shape[0], ids.shape[1], experts.ne[1]), dtype=torch.float32, device=b.device)
    return Node(MUL_MAT_ID, [experts, b, ids], [out])


def moe_router(ffn_inp: torch.Tensor, ffn_norm: torch.Tensor, gate_inp: torch.Tensor, eps: float, n_used: int) -> Node:
    """The router: ffn_inp [T, n_embd], ffn_norm [n_embd], gate_inp [n_expert, n_embd] -> (xn [T, n_embd],
    weights [T, n_used, 1], ids int32 [T, n_used])."""
    T, n_embd = ffn_inp.shape
    dev = ffn_inp.device
    xn = torch.empty((T, n_embd), dtype=torch.float32, device=dev)
    w = torch.empty((T, n_used, 1), dtype=torch.float32, device=dev)
    ids = torch.empty((T, n_used), dtype=torch.int32, device=dev)
    return Node(MOE_ROUTER, [ffn_inp, ffn_norm, gate_inp], [xn, w, ids], f_param=eps, i_param=n_used)


def moe_ffn_sum(gate: QTensor, up: QTensor, down: QTensor, b: torch.Tensor, ids: torch.Tensor,
                weights: torch.Tensor | None = None, out: torch.Tensor | None = None) -> Node:
    """The expert FFN summed over each token's slots: b [T, 1, n_embd] -> [T, n_embd]."""
    if out is None:
        out = torch.empty((ids.shape[0], gate.ne[0]), dtype=torch.float32, device=b.device)
    return Node(MOE_FFN_SUM, [gate, up, down, b, ids, weights], [out])


def moe_ffn(gate: QTensor, up: QTensor, down: QTensor, b: torch.Tensor, ids: torch.Tensor,
            weights: torch.Tensor | None = None, out: torch.Tensor | None = None) -> Node:
    """The expert FFN per slot: b [T, 1, n_embd] -> [T, n_used, n_embd]."""
    if out is None:
        out = torch.empty((ids.shape[0], ids.shape[1], gate.ne[0]), dtype=torch.float32, device=b.device)
    return Node(MOE_FFN, [gate, up, down, b, ids, weights], [out])


def sum_experts(experts: torch.Tensor, out: torch.Tensor | None = None) -> Node:
    if out is None:
        out = torch.empty((experts.shape[0], experts.shape[2]), dtype=torch.float32, device=experts.device)
    return Node(SUM_EXPERTS, [experts], [out])


def supports(node: Node) -> bool:
    """ggml_backend_dev_supports_op for this node (operator, types and shapes; no device touched)."""
    return bool(_lib.lib().tq_backend_supports_node(C.byref(node.raw())))


def _nodes_array(nodes):
    arr = (_lib.TqNode * len(nodes))()
    for i, n in enumerate(nodes):
        arr[i] = n.raw()
    return arr


class Backend:
    """A libtq backend instance on one gfx950 device, issuing on one stream."""

    def __init__(self, index: int, stream: torch.cuda.Stream | None = None):
        L = _lib.lib()
        self._ptr = L.tq_backend_init(index, stream.cuda_stream if stream is not None else None)
        if not self._ptr:
            raise Compute(-1, _lib.last_error())
        self.index = index
        self.stream = stream if stream is not None else torch.cuda.ExternalStream(L.tq_backend_get_stream(self._ptr))

    @staticmethod
    def gpu_count() -> int:
        return int(_lib.lib().tq_backend_dev_count())

    @staticmethod
    def gpu(index: int = 0, stream: torch.cuda.Stream | None = None) -> "Backend":
        if index >= Backend.gpu_count():
            raise Compute(-1, f"GPU {index}: the registry has {Backend.gpu_count()} gfx950 devices")
        return Backend(index, stream)

    def name(self) -> str:
        return _lib.lib().tq_backend_name(self._ptr).decode()

    def description(self) -> str:
        buf = C.create_string_buffer(256)
        _lib.lib().tq_backend_dev_description(self.index, buf, 256)
        return buf.value.decode()

    def reserve(self, nodes) -> None:
        arr = _nodes_array(nodes)
        rc = _lib.lib().tq_backend_reserve(self._ptr, arr, len(nodes))
        if rc != 0:
            raise Compute(rc, _lib.last_error())

    def compute_async(self, nodes) -> None:
        arr = _nodes_array(nodes)
        rc = _lib.lib().tq_backend_graph_compute(self._ptr, arr, len(nodes))
        if rc != 0:
            raise Compute(rc, _lib.last_error())

    def synchronize(self) -> None:
        if _lib.lib().tq_backend_synchronize(self._ptr) != 0:
            raise Compute(-1, "synchronize failed")

    def close(self) -> None:
        if self._ptr:
            _lib.lib().tq_backend_free(self._ptr)
            self._ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
