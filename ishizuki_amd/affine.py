"""Affine (MLX) quantized projections and the Hadamard rotation on MI355X.

Mirrors hadamardRotate and the rotated PackedLinear forward (Sources/IshizukiKit/Core/
Hadamard.swift:8-23,180-231) and VerifyMatmul.apply/applyAny (Core/VerifyMatmul.swift:63-120)
over libishizuki_hip. Kernel calls return None when declined, like the reference's nil.
"""
import torch

from . import _lib
from ._torch import DTYPES, ptr, require_cuda, stream

supported_rows = range(2, 9)   # VerifyMatmul.supportedRows (:12)


def minimum_rows(nbytes):
    """VerifyMatmul.minimumRows (Core/VerifyMatmul.swift:19-26), re-measured on MI355X.

    The reference's thresholds (2 rows from 100 MB, 3 from 10 MB, 4 from 5 MB, else 6) are where
    its verify kernel beats MLX's per-row path on an M1 Max. Here the alternative is M one-row
    GEMV calls, and one M-row verify call is faster from M = 2 at every size measured (1.6 MB
    attention k/v to the 397 MB vocabulary head, `python bench.py --policy`), so the minimum is 2.
    """
    return 2


def hadamard_rotate(x, block, signs=None, inverse=False):
    """hadamardRotate: y = WHT_block(x * signs)/sqrt(block) in fp32, cast back to x.dtype."""
    require_cuda(x)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1]).contiguous()
    y = torch.empty_like(x2)
    s = None if signs is None else signs.to(device=x.device, dtype=torch.float32).contiguous()
    rc = _lib.lib().ishz_hadamard(ptr(x2), DTYPES.get(x.dtype, -1), x2.shape[0], x2.shape[1], block,
                                  ptr(s), int(inverse), ptr(y), stream())
    if not _lib.check(rc, "hadamard"):
        raise ValueError(_lib.last_error())
    return y.reshape(shape)


def _args(weight, scales, biases):
    return (ptr(weight), ptr(scales), ptr(biases), DTYPES.get(scales.dtype, -1))


def quantized_matmul(x, weight, scales, biases, group_size=64, bits=2):
    """y = x . dequant(weight)^T for x [M, K], M in 1..16; None if declined."""
    require_cuda(x, weight, scales, biases)
    x = x.contiguous()
    M, K = x.shape
    N = weight.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    w, s, b, sdt = _args(weight, scales, biases)
    rc = _lib.lib().ishz_affine_matmul(ptr(x), DTYPES.get(x.dtype, -1), M, K, w, s, b, sdt, N, bits,
                                       group_size, ptr(y), stream())
    return y if _lib.check(rc, "affine_matmul") else None


def verify_apply(x, weight, scales, biases, group_size=64, bits=2):
    """VerifyMatmul.apply: declines below the weight's minimum row count (and above 8)."""
    if x.dim() != 2 or x.shape[0] not in supported_rows:
        return None
    if x.shape[0] < minimum_rows(weight.numel() * weight.element_size()):
        return None
    return quantized_matmul(x, weight, scales, biases, group_size, bits)


def linear(x, weight, scales, biases, signs=None, block=0, group_size=64, bits=2, _prestage=True):
    """Rotated PackedLinear forward: rotate (fused for one row) then the quantized matmul.

    With block <= 128 and more than two rows the workspace holds every row's x rotated and staged
    once for all workgroups (with one or two rows each workgroup rotates x itself, which measured
    faster); `_prestage=False` passes none, so each workgroup rotates x itself at any row count
    (test hook; the general path for other blocks needs the workspace)."""
    require_cuda(x, weight, scales, biases)
    x = x.contiguous()
    M, K = x.shape
    N = weight.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    L = _lib.lib()
    ws_bytes = L.ishz_affine_workspace_size(M, K) if block and _prestage else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    s = None
    if block and signs is not None:
        s = signs.to(device=x.device, dtype=torch.float32).contiguous()
    w, sc, b, sdt = _args(weight, scales, biases)
    rc = L.ishz_affine_linear(ptr(x), DTYPES.get(x.dtype, -1), M, K, ptr(s), block, w, sc, b, sdt, N,
                              bits, group_size, ptr(y), ptr(ws), ws_bytes, stream())
    return y if _lib.check(rc, "affine_linear") else None
