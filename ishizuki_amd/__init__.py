"""ishizuki_amd — Ishizuki's quantized-weight matmul path on MI355X (gfx950).

Host-side mirror of the reference's kernel API (GGMLKernels, VerifyMatmul, EXL3Kernels,
hadamardRotate, the MoE expert FFN) over the C ABI of libishizuki_hip.so (include/ishizuki_hip.h).
"""
from . import _lib  # noqa: F401

__all__ = ["ggml"]
