"""The C ABI boundary without a GPU: libtq.so loads, exports every entry point include/tq.h declares,
and rejects invalid arguments with ggml's failed status before touching a device."""
import ctypes as C
import os
import re
import subprocess

import pytest

from tetraeder_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "tq.h")]


def declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(tq_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("tq_mul_mat", "tq_mul_mat_id", "tq_quantize_q8_K", "tq_supports_op", "tq_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (tq_\w+)", out.stdout))
    for name in declared_functions():
        assert name in exported, f"{name} declared in include/tq.h but not exported"
        assert hasattr(L, name)
        assert name in _lib._SIGNATURES, f"{name} has no ctypes signature"


def test_supports_op():
    L = _lib.lib()
    assert L.tq_supports_op(1, 12, 0) == 1 and L.tq_supports_op(2, 14, 0) == 1
    assert L.tq_supports_op(1, 8, 0) == 0  # Q8_0 stays on ggml's backend
    assert L.tq_supports_op(1, 12, 1) == 0  # F16 activations are not handled
    assert L.tq_supports_op(7, 12, 0) == 0


def _t(ty, ne, nb, ptr=0x1000):
    t = _lib.TqTensor()
    t.type = ty
    for i in range(4):
        t.ne[i], t.nb[i] = ne[i], nb[i]
    t.data = ptr
    return t


def _contig(ty, ne, tsize, bsize=1):
    rs = tsize * ne[0] // bsize
    return [tsize, rs, rs * ne[1], rs * ne[1] * ne[2]]


@pytest.mark.parametrize("case", ["wrong_type", "k_not_multiple", "k_mismatch", "dst_shape", "broadcast",
                                  "null_a", "misaligned_q4"])
def test_mul_mat_rejects_invalid_arguments(case):
    L = _lib.lib()
    K, N, M = 512, 8, 2
    a = _t(12, [K, N, 1, 1], _contig(12, [K, N, 1, 1], 144, 256))
    b = _t(0, [K, M, 1, 1], _contig(0, [K, M, 1, 1], 4))
    d = _t(0, [N, M, 1, 1], _contig(0, [N, M, 1, 1], 4))
    if case == "wrong_type":
        a.type = 8
    elif case == "k_not_multiple":
        a.ne[0] = b.ne[0] = 300
    elif case == "k_mismatch":
        b.ne[0] = 256
    elif case == "dst_shape":
        d.ne[0] = N + 1
    elif case == "broadcast":
        a.ne[2], b.ne[2], d.ne[2] = 3, 4, 4
    elif case == "null_a":
        a = None
    elif case == "misaligned_q4":
        a.data = 0x1008
    rc = L.tq_mul_mat(C.byref(a) if a is not None else None, C.byref(b), C.byref(d), None, 0, None)
    assert rc == -1
    assert _lib.last_error()


def test_mul_mat_id_rejects_invalid_arguments():
    L = _lib.lib()
    K, N, E, used, T = 512, 8, 4, 2, 3
    a = _t(14, [K, N, E, 1], _contig(14, [K, N, E, 1], 210, 256))
    b = _t(0, [K, 1, T, 1], _contig(0, [K, 1, T, 1], 4))
    ids = _t(26, [used, T + 1, 1, 1], _contig(26, [used, T + 1, 1, 1], 4))  # T mismatch
    d = _t(0, [N, used, T, 1], _contig(0, [N, used, T, 1], 4))
    assert L.tq_mul_mat_id(C.byref(a), C.byref(b), C.byref(ids), C.byref(d), None, 0, None) == -1
    assert _lib.last_error()


def test_to_f32_and_quantize_reject_bad_sizes():
    L = _lib.lib()
    assert L.tq_to_f32(12, 0x1000, 0x2000, 300, None) == -1
    assert L.tq_to_f32(0, 0x1000, 0x2000, 256, None) == -1
    assert L.tq_quantize_weights(15, 0x1000, 0x2000, 1, 256, None) == -1
    assert L.tq_quantize_weights(12, 0x1000, 0x2000, 1, 100, None) == -1
