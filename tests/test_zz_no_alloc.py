"""tq_mul_mat_noalloc (the MUL_MAT entry point that allocates nothing: its scratch is a 32 MiB device
array of the library) through the C ABI, against tq_mul_mat with a workspace of its own on the same
operands: bit-identical outputs (the same kernels), on two calls in a row, the second with a smaller
input, so the second runs on the array the first left behind; operands that need more scratch than the
array holds are rejected with a message."""
import ctypes as C
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tetraeder_amd import _lib, ggml
from tests.helpers import normal

pytestmark = pytest.mark.gpu


def _case(name):
    print(f"[no_alloc] {name}", file=sys.stderr, flush=True)


def make_weights(ty, k, n, seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    src = torch.randn((n, k), generator=g, device=device) * 0.02
    return ggml.QTensor(ty, (k, n), ggml.quantize(ty, src, n, k))


def noalloc(a, b, out):
    at, bt, dt = a.raw(), ggml._dense(b, ggml.Type.F32), ggml._dense(out, ggml.Type.F32)
    return _lib.lib().tq_mul_mat_noalloc(C.byref(at), C.byref(bt), C.byref(dt),
                                         torch.cuda.current_stream().cuda_stream)


def with_workspace(a, b):
    ws = torch.empty(max(1, ggml.mul_mat_workspace_size(a, b)), dtype=torch.uint8, device=b.device)
    return ggml.mul_mat(a, b, workspace=ws)


def test_noalloc_matches_mul_mat_two_calls(gpu):
    # first call: Q6_K 12288 -> 4096 at 512 columns (the Q8_K copy and the k split's partial tiles in the
    # array, about 24 MB); second, smaller: Q4_K 2048 -> 4096 at 20 columns (the Q8_K copy only)
    cases = [(ggml.Type.Q6_K, 12288, 4096, 512, 71), (ggml.Type.Q4_K, 2048, 4096, 20, 72),
             (ggml.Type.Q4_K, 4096, 4096, 1, 73)]
    for ty, k, n, m, seed in cases:
        _case(f"{ty.name} {k}->{n} m={m}")
        a = make_weights(ty, k, n, seed, gpu)
        b = torch.from_numpy(normal((m, k), seed + 1)).to(gpu)
        want = with_workspace(a, b)
        out = torch.full((m, n), float("nan"), device=gpu)
        assert noalloc(a, b, out) == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"{ty.name} {k}->{n} m={m} differs from tq_mul_mat"
        if m <= 20:  # and the result itself, against the oracle
            ref = O.mul_mat(ty.id, a.data.cpu().numpy(), k, n, b.cpu().numpy())[0]
            assert float(np.abs(out.cpu().numpy() - ref).max() / np.abs(ref).max()) <= 1e-3


def test_noalloc_rejects_operands_above_the_array(gpu):
    _case("too large")
    a = make_weights(ggml.Type.Q4_K, 12288, 256, 74, gpu)
    b = torch.zeros((4000, 12288), device=gpu)  # Q8_K copy: 4000 x 48 x 292 bytes = 56 MB > 32 MiB
    out = torch.zeros((4000, 256), device=gpu)
    assert noalloc(a, b, out) == -1
    assert "scratch" in _lib.last_error()
    assert torch.count_nonzero(out) == 0
