"""Writes the small golden fixtures under tests/golden/ from seeded inputs and the CPU oracle.

The reference commits no golden vectors for this path (every reference test computes its expected
values by calling ggml at run time, and ggml is an absent submodule), so these fixtures come from the
oracle after it has been pinned by tests/test_oracle_*.py. They anchor the GPU tests to fixed bytes:
  q8k_vectors.npz   x [8, 1024] (normal, ties, a zero block, duplicate |max|) and its Q8_K bytes
  gemv_q4_K.npz     Q4_K w [1024 x 64], x [4, 1024], oracle y [4, 64], f64 reference and bound
  gemv_q6_K.npz     the same for Q6_K
  mmid_q4_K.npz     MUL_MAT_ID: 8 experts of [512 x 16] Q4_K, b [4, 1, 512], ids [4, 4] with -1,
                    oracle y [4, 4, 16]
  mmid_q6_K.npz     the same for Q6_K with b [4, 4, 512] (one activation row per slot)
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.helpers import normal, random_blocks  # noqa: E402


def q8k():
    rng = np.random.default_rng(2024)
    x = normal((8, 1024), 1)
    x[1] = rng.integers(-254, 255, size=1024).astype(np.float32) / 2
    x[1, ::256] = -127.0
    x[2, 256:512] = 0.0
    x[3, 7::61] = 5.5
    x[3, 9::61] = -5.5
    x[4] *= np.float32(1e-3)
    x[5] *= np.float32(1e6)
    np.savez_compressed(os.path.join(HERE, "q8k_vectors.npz"), x=x, q8=O.quantize_row_q8_K(x).reshape(8, -1))


def gemv(ty, name):
    k, n, m = 1024, 64, 4
    w = random_blocks(ty, n * k // 256, seed=ty)
    x = normal((m, k), 10 + ty)
    y = O.mul_mat(ty, w, k, n, x)[0]
    refs, bounds = zip(*(O.ref_f64(ty, w, k, x[i]) for i in range(m)))
    np.savez_compressed(os.path.join(HERE, f"gemv_{name}.npz"), w=w, x=x, y=y, ref=np.stack(refs),
                        bound=np.stack(bounds), k=k, n=n)


def mmid(ty, name, b1):
    k, n, E, used, T = 512, 16, 8, 4, 4
    w = random_blocks(ty, E * n * k // 256, seed=100 + ty)
    b = normal((T, b1, k), 20 + ty)
    ids = np.array([[3, 7, -1, 0], [7, 1, 2, 5], [-1, -1, 4, 6], [0, 3, 5, -1]], dtype=np.int32)
    y = O.mul_mat_id(ty, w, k, n, E, b, ids)
    np.savez_compressed(os.path.join(HERE, f"mmid_{name}.npz"), w=w, b=b, ids=ids, y=y, k=k, n=n, E=E)


if __name__ == "__main__":
    q8k()
    gemv(O.TYPE_Q4_K, "q4_K")
    gemv(O.TYPE_Q6_K, "q6_K")
    mmid(O.TYPE_Q4_K, "q4_K", 1)
    mmid(O.TYPE_Q6_K, "q6_K", 4)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
