"""ctypes access to the CPU oracle (``libtq_oracle.so``) -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module. It is the checker and the reported CPU baseline, never the thing measured or shipped.

The block layouts below are ggml's (b12426): ``block_q4_K`` 144 B, ``block_q6_K`` 210 B and
``block_q8_K`` 292 B per 256 elements (reference: patches/0002-iqk-avx512-q4k-q6k-decode.patch
:1277-1294, :1474-1487, :1638-1663).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtq_oracle.so")

QK_K = 256
TYPE_F32, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K, TYPE_I32 = 0, 12, 14, 15, 26

BLOCK_Q4_K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)])
BLOCK_Q6_K = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])
BLOCK_Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert BLOCK_Q4_K.itemsize == 144 and BLOCK_Q6_K.itemsize == 210 and BLOCK_Q8_K.itemsize == 292

BLOCK_DTYPE = {TYPE_Q4_K: BLOCK_Q4_K, TYPE_Q6_K: BLOCK_Q6_K, TYPE_Q8_K: BLOCK_Q8_K}
TYPE_SIZE = {TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q8_K: 292, TYPE_F32: 4, TYPE_I32: 4}


def row_size(ty: int, ne: int) -> int:
    if ty in (TYPE_F32, TYPE_I32):
        return 4 * ne
    assert ne % QK_K == 0, ne
    return TYPE_SIZE[ty] * (ne // QK_K)


class OrcTensor(C.Structure):
    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


_lib = None


def build() -> str:
    """Compiles the oracle with make (gcc). Called by __graft_entry__.build() and on first use."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, f32p, i32 = C.c_void_p, C.c_int64, C.POINTER(C.c_float), C.c_int
        L.orc_fp16_to_fp32.argtypes, L.orc_fp16_to_fp32.restype = [C.c_uint16], C.c_float
        for name in ("orc_quantize_row_q8_K",):
            getattr(L, name).argtypes, getattr(L, name).restype = [vp, vp, i64], None
        for name in ("orc_dequantize_row_q8_K", "orc_dequantize_row_q4_K", "orc_dequantize_row_q6_K"):
            getattr(L, name).argtypes, getattr(L, name).restype = [vp, vp, i64], None
        for name in ("orc_vec_dot_q4_K_q8_K", "orc_vec_dot_q6_K_q8_K"):
            getattr(L, name).argtypes, getattr(L, name).restype = [i64, vp, vp], C.c_float
        tp = C.POINTER(OrcTensor)
        L.orc_mul_mat.argtypes, L.orc_mul_mat.restype = [tp, tp, tp], i32
        L.orc_mul_mat_id.argtypes, L.orc_mul_mat_id.restype = [tp, tp, tp, tp], i32
        L.orc_ref_f64_rows.argtypes = [i32, vp, C.c_size_t, i64, i64, vp, vp, vp]
        L.orc_ref_f64_rows.restype = i32
        L.orc_iqk_mul_mat.argtypes = [C.c_long, C.c_long, C.c_long, i32, vp, C.c_long, i32, vp, C.c_long, vp,
                                      C.c_long, i32, i32]
        L.orc_iqk_mul_mat.restype = i32
        L.orc_cpu_has_avx512_vnni.argtypes, L.orc_cpu_has_avx512_vnni.restype = [], i32
        L.orc_pool_init.argtypes, L.orc_pool_init.restype = [i32], i32
        L.orc_pool_free.argtypes, L.orc_pool_free.restype = [], None
        L.orc_pool_threads.argtypes, L.orc_pool_threads.restype = [], i32
        L.orc_baseline_mul_mat.argtypes = [i32, vp, i64, i64, vp, i64, vp, vp, i32]
        L.orc_baseline_mul_mat.restype = i32
        L.orc_baseline_mul_mat_id.argtypes = [i32, vp, C.c_size_t, i64, i64, vp, i64, vp, i64, vp, vp, i32]
        L.orc_baseline_mul_mat_id.restype = i32
        del f32p
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def fp16_to_fp32(h: int) -> float:
    return lib().orc_fp16_to_fp32(h)


def quantize_row_q8_K(x: np.ndarray) -> np.ndarray:
    """Q8_K blocks (uint8 bytes) of a float32 array whose last dimension is a multiple of 256."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.size
    out = np.zeros(row_size(TYPE_Q8_K, k), dtype=np.uint8)
    lib().orc_quantize_row_q8_K(_ptr(x), _ptr(out), k)
    return out.reshape(x.shape[:-1] + (row_size(TYPE_Q8_K, x.shape[-1]),))


def dequantize(ty: int, raw: np.ndarray, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    assert raw.size == row_size(ty, k)
    out = np.zeros(k, dtype=np.float32)
    fn = {TYPE_Q8_K: lib().orc_dequantize_row_q8_K, TYPE_Q4_K: lib().orc_dequantize_row_q4_K,
          TYPE_Q6_K: lib().orc_dequantize_row_q6_K}[ty]
    fn(_ptr(raw), _ptr(out), k)
    return out


def vec_dot(ty: int, k: int, x_raw: np.ndarray, y_raw: np.ndarray) -> float:
    x_raw = np.ascontiguousarray(x_raw, dtype=np.uint8)
    y_raw = np.ascontiguousarray(y_raw, dtype=np.uint8)
    fn = lib().orc_vec_dot_q4_K_q8_K if ty == TYPE_Q4_K else lib().orc_vec_dot_q6_K_q8_K
    return fn(k, _ptr(x_raw), _ptr(y_raw))


def tensor(ty: int, ne, arr: np.ndarray, nb=None) -> OrcTensor:
    """An OrcTensor over a numpy buffer with ggml's contiguous strides unless nb is given."""
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        nb = [TYPE_SIZE[ty] if ty in (TYPE_F32, TYPE_I32) else TYPE_SIZE[ty]]
        nb.append(row_size(ty, ne[0]))
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    t = OrcTensor()
    t.type = ty
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.data = _ptr(arr)
    return t


def mul_mat(ty: int, w: np.ndarray, k: int, n: int, b: np.ndarray, ne2: int = 1) -> np.ndarray:
    """ggml MUL_MAT: w holds ne2 stacked [k, n] quantized matrices, b is float32 [ne12][m][k]."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    if b.ndim == 1:
        b = b[None, None, :]
    elif b.ndim == 2:
        b = b[None]
    ne12, m = b.shape[0], b.shape[1]
    w = np.ascontiguousarray(w, dtype=np.uint8)
    dst = np.zeros((ne12, m, n), dtype=np.float32)
    a_t = tensor(ty, [k, n, ne2], w)
    b_t = tensor(TYPE_F32, [k, m, ne12], b)
    d_t = tensor(TYPE_F32, [n, m, ne12], dst)
    rc = lib().orc_mul_mat(C.byref(a_t), C.byref(b_t), C.byref(d_t))
    assert rc == 0, rc
    return dst


def mul_mat_id(ty: int, w: np.ndarray, k: int, n: int, n_expert: int, b: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """ggml MUL_MAT_ID: w [k, n, n_expert] stacked, b float32 [T][ne11][k], ids int32 [T][n_used]."""
    b = np.ascontiguousarray(b, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, ne11 = b.shape[0], b.shape[1]
    n_used = ids.shape[1]
    w = np.ascontiguousarray(w, dtype=np.uint8)
    dst = np.full((T, n_used, n), np.nan, dtype=np.float32)
    a_t = tensor(ty, [k, n, n_expert], w)
    b_t = tensor(TYPE_F32, [k, ne11, T], b)
    i_t = tensor(TYPE_I32, [n_used, T], ids)
    d_t = tensor(TYPE_F32, [n, n_used, T], dst)
    rc = lib().orc_mul_mat_id(C.byref(a_t), C.byref(b_t), C.byref(i_t), C.byref(d_t))
    assert rc == 0, rc
    return dst


def sum_experts(experts: np.ndarray) -> np.ndarray:
    """sum_experts (crates/model/src/qwen3moe.rs:2917-2923): float32 [T][n_used][n_embd] -> [T][n_embd]
    by the reference's chain of ADD nodes over the choice views, view(0) + view(1), then + view(2), ...,
    each an fp32 add."""
    e = np.asarray(experts, dtype=np.float32)
    acc = e[:, 0, :].copy()
    for j in range(1, e.shape[1]):
        acc = (acc + e[:, j, :]).astype(np.float32)
    return acc


def router(x: np.ndarray, norm: np.ndarray, gate: np.ndarray, eps: float, n_used: int):
    """The MoE router (crates/model/src/qwen3moe.rs:2869-2887) on float32 x [T][n_embd], norm [n_embd]
    and gate [n_expert][n_embd], with ggml's CPU arithmetic for each node: rms_norm sums the float32
    squares in double (mean = sum / n as float32, scale = 1 / sqrtf(mean + eps)); the logits (MUL_MAT)
    here are float64 dots rounded to float32 (ggml's SIMD order is another fp32 rounding of the same
    sum); soft_max subtracts the max, sums the float32 exponentials in double and scales by
    (float)(1 / sum); argsort_top_k keeps the n_used largest, largest first, equal values by the lower
    id (crates/ggml-sys/tests/ggml.rs:33-44 fixes the order on [0.1, 0.9, 0.3, 0.5]: ids [1, 3]);
    get_rows, sum_rows (double), clamp(sum, 2^-14, inf) and div. Returns (xn, probs, weights, ids)."""
    x = np.asarray(x, dtype=np.float32)
    norm = np.asarray(norm, dtype=np.float32)
    gate = np.asarray(gate, dtype=np.float32)
    n = x.shape[1]
    ss = (x * x).astype(np.float64).sum(axis=1)
    mean = (ss / n).astype(np.float32)
    scale = (np.float32(1.0) / np.sqrt(mean + np.float32(eps), dtype=np.float32)).astype(np.float32)
    xn = ((x * scale[:, None]).astype(np.float32) * norm).astype(np.float32)
    logits = (xn.astype(np.float64) @ gate.astype(np.float64).T).astype(np.float32)
    mx = logits.max(axis=1, keepdims=True)
    e = np.exp((logits - mx).astype(np.float32)).astype(np.float32)
    inv = (1.0 / e.astype(np.float64).sum(axis=1)).astype(np.float32)
    probs = (e * inv[:, None]).astype(np.float32)
    T, E = probs.shape
    ids = np.zeros((T, n_used), dtype=np.int32)
    for t in range(T):
        order = sorted(range(E), key=lambda i: (-float(probs[t, i]), i))
        ids[t] = order[:n_used]
    sel = np.take_along_axis(probs, ids.astype(np.int64), axis=1)
    ssum = sel.astype(np.float64).sum(axis=1).astype(np.float32)
    div = np.maximum(ssum, np.float32(6.103515625e-5))
    w = (sel / div[:, None]).astype(np.float32)
    return xn, probs, w, ids


def ref_f64(ty: int, w_rows: np.ndarray, k: int, x: np.ndarray):
    """(y, bound): f64 dot of dequantized rows with the Q8_K round trip of x, and 1e-5*sum|wx|+1e-6."""
    w_rows = np.ascontiguousarray(w_rows, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rb = row_size(ty, k)
    n = w_rows.size // rb
    out = np.zeros(n, dtype=np.float64)
    bound = np.zeros(n, dtype=np.float64)
    rc = lib().orc_ref_f64_rows(ty, _ptr(w_rows), rb, n, k, _ptr(x), _ptr(out), _ptr(bound))
    assert rc == 0, rc
    return out, bound


def has_avx512_vnni() -> bool:
    return bool(lib().orc_cpu_has_avx512_vnni())


def iqk_rows(ty: int, w_rows: np.ndarray, k: int, q8: np.ndarray, ith: int = 0, nth: int = 1) -> np.ndarray | None:
    """The restated iqk one-column kernel on this thread's static share; None when not handled."""
    w_rows = np.ascontiguousarray(w_rows, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    rb = row_size(ty, k)
    n = w_rows.size // rb
    out = np.full(n, np.nan, dtype=np.float32)
    ok = lib().orc_iqk_mul_mat(n, 1, k, ty, _ptr(w_rows), rb // TYPE_SIZE[ty], TYPE_Q8_K, _ptr(q8), k // QK_K,
                               _ptr(out), n, ith, nth)
    return out if ok else None


class Baseline:
    """The restated CPU decode path on a pool of threads (the reported CPU baseline)."""

    def __init__(self, threads: int):
        self.threads = max(1, int(threads))
        rc = lib().orc_pool_init(self.threads)
        assert rc == 0, rc
        self.iqk = has_avx512_vnni()

    def close(self):
        lib().orc_pool_free()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def mul_mat(self, ty, w, n, k, x, q8, y, use_iqk=True):
        rc = lib().orc_baseline_mul_mat(ty, _ptr(w), n, k, _ptr(x), x.size // k, _ptr(q8), _ptr(y), int(use_iqk))
        assert rc == 0, rc

    def mul_mat_id(self, ty, w, expert_bytes, n, k, x, ids, q8, y, use_iqk=True):
        ne11 = x.size // k
        rc = lib().orc_baseline_mul_mat_id(ty, _ptr(w), expert_bytes, n, k, _ptr(x), ne11, _ptr(ids), ids.size,
                                           _ptr(q8), _ptr(y), int(use_iqk))
        assert rc == 0, rc
