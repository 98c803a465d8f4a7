"""The ggml operator surface for Q4_K / Q6_K weights on MI355X, over libtq.so.

Mirrors the names, argument meaning and errors of the reference's safe ggml layer
(crates/ggml-sys/src/ggml): ``Type`` (mod.rs:45-118), ``mul_mat`` / ``mul_mat_id``
(context.rs:294-299, 320-336), ``quantize`` / ``to_f32`` (quant.rs:20-101) and ``GgmlError``
(mod.rs:31-41: ``Invalid`` for bad arguments, ``Compute`` for a failed compute status). Ops run
eagerly on the current HIP stream instead of building graph nodes; tensors are torch device buffers
(torch is used for device memory and streams only). Quantized tensors are raw ggml block bytes in a
uint8 buffer with ggml's ``ne`` (dimension 0 fastest) and byte strides ``nb``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib

QK_K = 256


class GgmlError(RuntimeError):
    pass


class Invalid(GgmlError):
    """Arguments that can never work (ggml-sys GgmlError::Invalid)."""


class Compute(GgmlError):
    """A compute call returned a failed status (ggml-sys GgmlError::Compute(i32))."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"status {status}: {msg}")
        self.status = status


@dataclass(frozen=True)
class Type:
    """A ggml tensor storage type; the id is ggml's enum ggml_type (also the GGUF type id)."""

    id: int
    name: str
    block_size: int
    type_size: int

    def row_size(self, ne: int) -> int:
        if ne % self.block_size:
            raise Invalid(f"{ne} elements per row is not a multiple of the {self.name} block size {self.block_size}")
        return self.type_size * (ne // self.block_size)

    @staticmethod
    def from_name(name: str) -> "Type | None":
        return _BY_NAME.get(name.lower())

    @staticmethod
    def from_id(i: int) -> "Type | None":
        return _BY_ID.get(i)


Type.F32 = Type(0, "f32", 1, 4)
Type.Q4_K = Type(12, "q4_K", QK_K, 144)
Type.Q6_K = Type(14, "q6_K", QK_K, 210)
Type.Q8_K = Type(15, "q8_K", QK_K, 292)
Type.I32 = Type(26, "i32", 1, 4)
_BY_NAME = {t.name.lower(): t for t in (Type.F32, Type.Q4_K, Type.Q6_K, Type.Q8_K, Type.I32)}
_BY_ID = {t.id: t for t in _BY_NAME.values()}

OP_MUL_MAT, OP_MUL_MAT_ID = 1, 2


@dataclass
class QTensor:
    """Quantized weights in device memory: ggml type, ne (dim 0 fastest) and a uint8 byte buffer."""

    type: Type
    ne: tuple
    data: torch.Tensor
    nb: tuple | None = None

    def __post_init__(self):
        ne = tuple(int(x) for x in self.ne) + (1,) * (4 - len(self.ne))
        self.ne = ne
        if self.nb is None:
            rs = self.type.row_size(ne[0])
            self.nb = (self.type.type_size, rs, rs * ne[1], rs * ne[1] * ne[2])
        if self.data.dtype != torch.uint8:
            raise Invalid("QTensor data must be a uint8 buffer")
        if self.data.numel() < self.nb[3] * ne[3]:
            raise Invalid(f"{self.data.numel()} bytes hold less than the {self.nb[3] * ne[3]} the shape needs")

    def raw(self) -> _lib.TqTensor:
        return _raw(self.type.id, self.ne, self.nb, self.data.data_ptr())


def _raw(type_id: int, ne, nb, ptr: int) -> _lib.TqTensor:
    t = _lib.TqTensor()
    t.type = type_id
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    t.data = ptr
    return t


def _dense(x: torch.Tensor, ty: Type) -> _lib.TqTensor:
    """A torch tensor as a ggml tensor: torch's last dimension is ggml's dimension 0."""
    d = x.dim()
    if d > 4:
        raise Invalid("at most 4 dimensions")
    es = x.element_size()
    ne, nb = [1] * 4, [0] * 4
    for i in range(d):
        ne[i] = x.shape[d - 1 - i]
        nb[i] = x.stride(d - 1 - i) * es
    for i in range(d, 4):
        nb[i] = nb[i - 1] * ne[i - 1] if i > 0 else es
    return _raw(ty.id, ne, nb, x.data_ptr())


def _stream(stream) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _check(rc: int):
    if rc != 0:
        raise Compute(rc, _lib.last_error())


def supports_op(op: int, type_a: Type, type_b: Type = Type.F32) -> bool:
    return bool(_lib.lib().tq_supports_op(op, type_a.id, type_b.id))


def quantize_q8_K(x: torch.Tensor, stream=None) -> torch.Tensor:
    """Q8_K blocks of the rows of x (float32, last dim a multiple of 256) as a uint8 tensor
    [rows, row_size]; bit-identical to ggml's quantize_row_q8_K."""
    if x.dtype != torch.float32:
        raise Invalid("quantize_q8_K takes float32")
    k = x.shape[-1]
    rows = x.numel() // k if k else 0
    out = torch.empty((rows, Type.Q8_K.row_size(k)), dtype=torch.uint8, device=x.device)
    src = _dense(x, Type.F32)
    _check(_lib.lib().tq_quantize_q8_K(C.byref(src), out.data_ptr(), _stream(stream)))
    return out


def mul_mat(a: QTensor, b, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            stream=None) -> torch.Tensor:
    """ggml MUL_MAT: a [K, N, ne02, ne03] quantized, b float32 torch [..., M, K] -> [..., M, N].
    b may also be a Q8_K QTensor [K, M, ne12, ne13] (already quantized; ggml's vec_dot_type)."""
    if isinstance(b, QTensor):
        if b.type != Type.Q8_K:
            raise Invalid("a quantized b must be Q8_K")
        bt = b.raw()
        if out is None:
            out = torch.empty((b.ne[3], b.ne[2], b.ne[1], a.ne[1]), dtype=torch.float32, device=b.data.device)
    else:
        if b.dtype != torch.float32:
            raise Invalid("b must be float32")
        bt = _dense(b, Type.F32)
        if out is None:
            out = torch.empty(tuple(b.shape[:-1]) + (a.ne[1],), dtype=torch.float32, device=b.device)
    dt = _dense(out, Type.F32)
    at = a.raw()
    ws_ptr, ws_size = 0, 0
    if workspace is not None:
        ws_ptr, ws_size = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _check(_lib.lib().tq_mul_mat(C.byref(at), C.byref(bt), C.byref(dt), ws_ptr, ws_size, _stream(stream)))
    return out


def mul_mat_workspace_size(a: QTensor, b: torch.Tensor) -> int:
    at, bt = a.raw(), _dense(b, Type.F32)
    return int(_lib.lib().tq_mul_mat_workspace_size(C.byref(at), C.byref(bt)))


def mul_mat_id(experts: QTensor, b: torch.Tensor, ids: torch.Tensor, out: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """ggml MUL_MAT_ID: experts [K, N, n_expert], b float32 torch [T, ne11, K] (ne11 = 1 or n_used),
    ids int32 torch [T, n_used] -> [T, n_used, N]; negative ids give exact zero rows."""
    if b.dtype != torch.float32 or ids.dtype != torch.int32:
        raise Invalid("b must be float32 and ids int32")
    if b.dim() != 3 or ids.dim() != 2:
        raise Invalid("b is [T, ne11, K] and ids [T, n_used]")
    T, n_used = ids.shape
    if out is None:
        out = torch.empty((T, n_used, experts.ne[1]), dtype=torch.float32, device=b.device)
    at, bt, it, dt = experts.raw(), _dense(b, Type.F32), _dense(ids, Type.I32), _dense(out, Type.F32)
    ws_ptr, ws_size = 0, 0
    if workspace is not None:
        ws_ptr, ws_size = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _check(_lib.lib().tq_mul_mat_id(C.byref(at), C.byref(bt), C.byref(it), C.byref(dt), ws_ptr, ws_size,
                                    _stream(stream)))
    return out


def mul_mat_id_workspace_size(experts: QTensor, b: torch.Tensor, ids: torch.Tensor) -> int:
    at, bt, it = experts.raw(), _dense(b, Type.F32), _dense(ids, Type.I32)
    return int(_lib.lib().tq_mul_mat_id_workspace_size(C.byref(at), C.byref(bt), C.byref(it)))


def moe_ffn(gate: QTensor, up: QTensor, down: QTensor, b: torch.Tensor, ids: torch.Tensor,
            weights: torch.Tensor | None = None, out: torch.Tensor | None = None,
            workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """The MoE expert FFN (weighted_experts, crates/model/src/qwen3moe.rs:2899-2914):
    down(swiglu(gate(b), up(b))) per routed slot, times the router weight.
    b float32 torch [T, 1, n_embd], ids int32 [T, n_used], weights float32 [T, n_used, 1] or None;
    returns [T, n_used, n_embd]."""
    if b.dtype != torch.float32 or ids.dtype != torch.int32 or b.dim() != 3 or ids.dim() != 2:
        raise Invalid("b is float32 [T, 1, n_embd] and ids int32 [T, n_used]")
    T, n_used = ids.shape
    if out is None:
        out = torch.empty((T, n_used, gate.ne[0]), dtype=torch.float32, device=b.device)
    gt, ut, dt_, bt, it, ot = gate.raw(), up.raw(), down.raw(), _dense(b, Type.F32), _dense(ids, Type.I32), \
        _dense(out, Type.F32)
    wt = C.byref(_dense(weights, Type.F32)) if weights is not None else None
    ws_ptr, ws_size = 0, 0
    if workspace is not None:
        ws_ptr, ws_size = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _check(_lib.lib().tq_moe_ffn(C.byref(gt), C.byref(ut), C.byref(dt_), C.byref(bt), C.byref(it), wt, C.byref(ot),
                                 ws_ptr, ws_size, _stream(stream)))
    return out


def moe_ffn_sum(gate: QTensor, up: QTensor, down: QTensor, b: torch.Tensor, ids: torch.Tensor,
                weights: torch.Tensor | None = None, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """moe_ffn (crates/model/src/qwen3moe.rs:2892-2895): the expert FFN above summed over each token's
    slots in choice order (sum_experts, qwen3moe.rs:2917-2923). Operands as for moe_ffn; returns
    [T, n_embd]."""
    if b.dtype != torch.float32 or ids.dtype != torch.int32 or b.dim() != 3 or ids.dim() != 2:
        raise Invalid("b is float32 [T, 1, n_embd] and ids int32 [T, n_used]")
    T = ids.shape[0]
    if out is None:
        out = torch.empty((T, gate.ne[0]), dtype=torch.float32, device=b.device)
    gt, ut, dt_, bt, it, ot = gate.raw(), up.raw(), down.raw(), _dense(b, Type.F32), _dense(ids, Type.I32), \
        _dense(out, Type.F32)
    wt = C.byref(_dense(weights, Type.F32)) if weights is not None else None
    ws_ptr, ws_size = 0, 0
    if workspace is not None:
        ws_ptr, ws_size = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _check(_lib.lib().tq_moe_ffn_sum(C.byref(gt), C.byref(ut), C.byref(dt_), C.byref(bt), C.byref(it), wt,
                                     C.byref(ot), ws_ptr, ws_size, _stream(stream)))
    return out


def sum_experts(experts: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """sum_experts (crates/model/src/qwen3moe.rs:2917-2923): float32 [T, n_used, n_embd] -> [T, n_embd],
    each token's slots added left to right."""
    if experts.dtype != torch.float32 or experts.dim() != 3:
        raise Invalid("experts is float32 [T, n_used, n_embd]")
    T, _, n_embd = experts.shape
    if out is None:
        out = torch.empty((T, n_embd), dtype=torch.float32, device=experts.device)
    et, ot = _dense(experts, Type.F32), _dense(out, Type.F32)
    _check(_lib.lib().tq_sum_experts(C.byref(et), C.byref(ot), _stream(stream)))
    return out


def moe_router(ffn_inp: torch.Tensor, ffn_norm: torch.Tensor, gate_inp: torch.Tensor, eps: float, n_used: int,
               workspace: torch.Tensor | None = None, stream=None):
    """The MoE router (crates/model/src/qwen3moe.rs:2869-2887): ffn_inp float32 [T, n_embd], ffn_norm
    [n_embd], gate_inp float32 [n_expert, n_embd] (ggml's [n_embd, n_expert]) -> (xn [T, n_embd],
    weights [T, n_used, 1], ids int32 [T, n_used]), as moe_ffn takes them."""
    for t, nm in ((ffn_inp, "ffn_inp"), (ffn_norm, "ffn_norm"), (gate_inp, "gate_inp")):
        if t.dtype != torch.float32:
            raise Invalid(f"{nm} must be float32")
    if ffn_inp.dim() != 2 or ffn_norm.dim() != 1 or gate_inp.dim() != 2:
        raise Invalid("ffn_inp is [T, n_embd], ffn_norm [n_embd], gate_inp [n_expert, n_embd]")
    T, n_embd = ffn_inp.shape
    dev = ffn_inp.device
    xn = torch.empty((T, n_embd), dtype=torch.float32, device=dev)
    w = torch.empty((T, n_used, 1), dtype=torch.float32, device=dev)
    ids = torch.empty((T, n_used), dtype=torch.int32, device=dev)
    xt, nt, gt = _dense(ffn_inp, Type.F32), _dense(ffn_norm, Type.F32), _dense(gate_inp, Type.F32)
    ot, wt, it = _dense(xn, Type.F32), _dense(w, Type.F32), _dense(ids, Type.I32)
    ws_ptr, ws_size = 0, 0
    if workspace is not None:
        ws_ptr, ws_size = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _check(_lib.lib().tq_moe_router(C.byref(xt), C.byref(nt), C.byref(gt), eps, n_used, C.byref(ot), C.byref(wt),
                                    C.byref(it), ws_ptr, ws_size, _stream(stream)))
    return xn, w, ids


def moe_router_workspace_size(gate_inp: torch.Tensor, ffn_inp: torch.Tensor) -> int:
    gt, xt = _dense(gate_inp, Type.F32), _dense(ffn_inp, Type.F32)
    return int(_lib.lib().tq_moe_router_workspace_size(C.byref(gt), C.byref(xt)))


COPY_AUTO, COPY_KERNEL, COPY_DMA = 0, 1, 2


def copy_expert_slots(src: list, dst: list, from_slots, to_slots, engine: int = COPY_AUTO, stream=None) -> None:
    """Makes experts resident in device slots: for every pair (from_slots[i], to_slots[i]) and every
    tensor p, the raw slab of host slot from_slots[i] of src[p] goes to device slot to_slots[i] of dst[p]
    (the device side of copy_slot, crates/model/src/experts.rs:1880-1893, for a batch of experts).
    src: QTensors over host bytes (pinned for COPY_KERNEL: torch's pin_memory=True), dst: QTensors over
    device bytes, [K, N, n_slots] with the same type and rows. Asynchronous on the stream: the host
    bytes must not change until the stream has passed the copy."""
    if len(src) != len(dst):
        raise Invalid("src and dst list different tensor counts")
    n = len(from_slots)
    if len(to_slots) != n:
        raise Invalid("from_slots and to_slots differ in length")
    for t in src:
        if t.data.is_cuda:
            raise Invalid("src slabs must be in host memory")
    for t in dst:
        if not t.data.is_cuda:
            raise Invalid("dst slots must be in device memory")
    k = len(src)
    srcs = (_lib.TqTensor * max(1, k))(*[t.raw() for t in src])
    dsts = (_lib.TqTensor * max(1, k))(*[t.raw() for t in dst])
    fr = (C.c_uint32 * max(1, n))(*[int(v) for v in from_slots])
    to = (C.c_uint32 * max(1, n))(*[int(v) for v in to_slots])
    _check(_lib.lib().tq_copy_expert_slots(srcs, dsts, k, fr, to, n, int(engine), _stream(stream)))


def moe_sync_errors(clear: bool = False) -> int:
    """Failed cross-workgroup waits of the single-launch MoE step on the current device (0: none)."""
    v = C.c_uint(0)
    _check(_lib.lib().tq_moe_ffn_sync_errors(C.byref(v), 1 if clear else 0))
    return int(v.value)


def moe_ffn_workspace_size(gate: QTensor, b: torch.Tensor, ids: torch.Tensor) -> int:
    gt, bt, it = gate.raw(), _dense(b, Type.F32), _dense(ids, Type.I32)
    return int(_lib.lib().tq_moe_ffn_workspace_size(C.byref(gt), C.byref(bt), C.byref(it)))


def to_f32(ty: Type, src: torch.Tensor, n: int, stream=None) -> torch.Tensor:
    """Dequantizes n elements (whole blocks of ty) from a uint8 device buffer."""
    if src.numel() < ty.row_size(n):
        raise Invalid(f"{src.numel()} bytes for {n} elements of {ty.name}")
    out = torch.empty(n, dtype=torch.float32, device=src.device)
    _check(_lib.lib().tq_to_f32(ty.id, src.data_ptr(), out.data_ptr(), n, _stream(stream)))
    return out


def quantize(ty: Type, src: torch.Tensor, n_rows: int, n_per_row: int, stream=None) -> torch.Tensor:
    """Quantizes n_rows rows of n_per_row float32 values (a contiguous device tensor) to ty (Q4_K or
    Q6_K) with the device one-pass fit; returns n_rows * row_size bytes."""
    if src.dtype != torch.float32 or not src.is_contiguous():
        raise Invalid("src must be contiguous float32")
    if src.numel() != n_rows * n_per_row:
        raise Invalid(f"quantize to {ty.name}: {src.numel()} floats for {n_rows} rows of {n_per_row}")
    out = torch.empty(n_rows * ty.row_size(n_per_row), dtype=torch.uint8, device=src.device)
    _check(_lib.lib().tq_quantize_weights(ty.id, src.data_ptr(), out.data_ptr(), n_rows, n_per_row, _stream(stream)))
    return out
