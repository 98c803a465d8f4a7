"""tetraeder_amd: MI355X-native (gfx950) Q4_K / Q6_K MUL_MAT and MUL_MAT_ID for the Tetraeder engine.

The product is libtq.so (hand-written HIP kernels behind the C ABI in include/tq.h); ``ggml`` is the
Python mirror of the reference's ggml operator surface over that library.
"""
from . import ggml  # noqa: F401

__all__ = ["ggml"]
