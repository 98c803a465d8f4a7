"""The C++ host layer (include/tq_ggml.hpp) through its test driver tests/cpp/tq_ggml_test.cpp.

CPU: types, strides and the error behaviour of the ggml-sys-shaped surface (GgmlError kinds, status
codes, messages). GPU: MUL_MAT and MUL_MAT_ID on device buffers through the layer against the oracle.
The driver is built by __graft_entry__.build() (make -C tests/cpp); the CPU test rebuilds it here.
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER = os.path.join(HERE, "cpp", "tq_ggml_test")


def _run(mode):
    print(f"[host cpp] {mode}", file=sys.stderr, flush=True)
    r = subprocess.run([DRIVER, mode], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, f"driver {mode} failed ({r.returncode}):\n{r.stdout}\n{r.stderr}"
    assert r.stdout.strip().endswith("ok"), r.stdout
    return r.stdout


def test_cpp_layer_cpu():
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True, capture_output=True)
    _run("cpu")


@pytest.mark.gpu
def test_cpp_layer_gpu(gpu):
    assert os.path.exists(DRIVER), "tests/cpp/tq_ggml_test is not built (run __graft_entry__.build())"
    out = _run("gpu")
    print(out)
