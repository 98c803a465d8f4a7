"""Loads libtq.so (the gfx950 kernels behind include/tq.h) through ctypes.

There is no fallback: when the library is missing or fails to load, every entry point raises. Build it
with ``python -m tetraeder_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtq.so")


class TqTensor(C.Structure):
    """struct tq_tensor: ggml's type, ne[4], nb[4] and data (include/tq.h)."""

    _fields_ = [("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


_lib: C.CDLL | None = None

# name -> (argtypes, restype); the list is checked against include/tq.h by the CPU test suite.
_SIGNATURES = {
    "tq_last_error": ([], C.c_char_p),
    "tq_version": ([], C.c_char_p),
    "tq_supports_op": ([C.c_int, C.c_int, C.c_int], C.c_int),
    "tq_quantize_q8_K": ([C.POINTER(TqTensor), C.c_void_p, C.c_void_p], C.c_int),
    "tq_mul_mat_workspace_size": ([C.POINTER(TqTensor), C.POINTER(TqTensor)], C.c_size_t),
    "tq_mul_mat": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor), C.c_void_p, C.c_size_t,
                    C.c_void_p], C.c_int),
    "tq_mul_mat_noalloc": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor), C.c_void_p], C.c_int),
    "tq_mul_mat_id_workspace_size": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor)], C.c_size_t),
    "tq_mul_mat_id": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor),
                       C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "tq_moe_ffn_workspace_size": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.POINTER(TqTensor)], C.c_size_t),
    "tq_moe_ffn": ([C.POINTER(TqTensor)] * 6 + [C.POINTER(TqTensor), C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "tq_moe_ffn_sum": ([C.POINTER(TqTensor)] * 6 + [C.POINTER(TqTensor), C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "tq_sum_experts": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.c_void_p], C.c_int),
    "tq_moe_router_workspace_size": ([C.POINTER(TqTensor), C.POINTER(TqTensor)], C.c_size_t),
    "tq_moe_router": ([C.POINTER(TqTensor)] * 3 + [C.c_float, C.c_int] + [C.POINTER(TqTensor)] * 3 +
                      [C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "tq_copy_expert_slots": ([C.POINTER(TqTensor), C.POINTER(TqTensor), C.c_int, C.POINTER(C.c_uint32),
                              C.POINTER(C.c_uint32), C.c_int, C.c_int, C.c_void_p], C.c_int),
    "tq_moe_ffn_sync_errors": ([C.POINTER(C.c_uint), C.c_int], C.c_int),
    "tq_to_f32": ([C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p], C.c_int),
    "tq_quantize_weights": ([C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p], C.c_int),
    "tq_backend_reg_name": ([], C.c_char_p),
    "tq_backend_dev_count": ([], C.c_int),
    "tq_backend_dev_hip_ordinal": ([C.c_int], C.c_int),
    "tq_backend_dev_description": ([C.c_int, C.c_char_p, C.c_size_t], C.c_int),
    "tq_backend_dev_memory": ([C.c_int, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)], C.c_int),
    "tq_backend_supports_node": ([C.c_void_p], C.c_int),
    "tq_backend_init": ([C.c_int, C.c_void_p], C.c_void_p),
    "tq_backend_free": ([C.c_void_p], None),
    "tq_backend_name": ([C.c_void_p], C.c_char_p),
    "tq_backend_get_stream": ([C.c_void_p], C.c_void_p),
    "tq_backend_reserve": ([C.c_void_p, C.c_void_p, C.c_int], C.c_int),
    "tq_backend_graph_compute": ([C.c_void_p, C.c_void_p, C.c_int], C.c_int),
    "tq_backend_synchronize": ([C.c_void_p], C.c_int),
}


class TqNode(C.Structure):
    """struct tq_node (include/tq.h): operator, sources, destinations, scalar parameters."""

    _fields_ = [("op", C.c_int32), ("src", C.POINTER(TqTensor) * 6), ("dst", C.POINTER(TqTensor) * 3),
                ("f_param", C.c_float), ("i_param", C.c_int32)]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m tetraeder_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


def last_error() -> str:
    return lib().tq_last_error().decode()
