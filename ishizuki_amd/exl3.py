"""EXL3 trellis-coded projections on MI355X: EXL3Tensor and EXL3Kernels over libishizuki_hip.

Mirrors Sources/IshizukiKit/Core/EXL3.swift: EXL3Tensor (:9-77, validation of rate, codebook and
shape), EXL3Kernels.apply/matvec/dequantize/rotate (:79-164).
"""
import torch

from . import _lib
from ._torch import DTYPES, ptr, require_cuda, stream

THREE_INST, MCG, MUL1 = 0, 1, 2
SUPPORTED_BITS = (1, 1.5, 2, 2.5, 3, 3.5, 4, 5, 6, 7, 8)
matvec_rows = range(1, 17)


class EXL3Tensor:
    """trellis int16 [K/16, N/16, 16*bits] plus fp16 input/output channel scales (suh, svh)."""

    def __init__(self, trellis, input_scales, output_scales, codebook=THREE_INST):
        if trellis.dim() != 3 or trellis.dtype != torch.int16:
            raise ValueError("EXL3 trellis must be int16 [k/16, n/16, words]")
        bits = trellis.shape[2] / 16
        if bits not in SUPPORTED_BITS:
            raise ValueError(f"EXL3 tile of {trellis.shape[2]} words is not a rate")
        if bits != int(bits) and codebook != MUL1:
            raise ValueError(f"half-integer EXL3 rate {bits} needs the mul1 codebook")
        k, n = trellis.shape[0] * 16, trellis.shape[1] * 16
        if k % 128 or n % 128:
            raise ValueError(f"EXL3 {k}x{n} is not a whole number of 128 blocks")
        if input_scales.numel() != k or output_scales.numel() != n:
            raise ValueError("EXL3 scale vectors do not match the tensor")
        self.trellis = trellis.contiguous()
        self.suh = input_scales.reshape(k).to(torch.float16).contiguous()
        self.svh = output_scales.reshape(n).to(torch.float16).contiguous()
        self.bits2 = int(round(bits * 2))
        self.codebook = codebook
        self.input_dim, self.output_dim = k, n


def dequantize(t, dtype=torch.float16):
    out = torch.empty((t.input_dim, t.output_dim), dtype=dtype, device=t.trellis.device)
    rc = _lib.lib().ishz_exl3_dequant(ptr(t.trellis), t.input_dim, t.output_dim, t.bits2, t.codebook,
                                      ptr(out), DTYPES[dtype], stream())
    return out if _lib.check(rc, "exl3_dequant") else None


def rotate(x, scales, before, out_dtype):
    x = x.contiguous()
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rc = _lib.lib().ishz_exl3_rotate(ptr(x), DTYPES[x.dtype], x.shape[0], x.shape[1], ptr(scales),
                                     int(before), ptr(y), DTYPES[out_dtype], stream())
    if not _lib.check(rc, "exl3_rotate"):
        raise ValueError(_lib.last_error())
    return y


def matvec(xh, t, workspace=None):
    """xh [M, K] (already rotated; fp16, bf16 or fp32) -> fp32 [M, N]. With `workspace` (a uint8
    device tensor of matvec_workspace_size bytes) the call allocates nothing."""
    require_cuda(xh, t.trellis)
    xh = xh.contiguous()
    M = xh.shape[0]
    y = torch.empty((M, t.output_dim), dtype=torch.float32, device=xh.device)
    L = _lib.lib()
    if workspace is None:
        rc = L.ishz_exl3_matvec(ptr(xh), DTYPES.get(xh.dtype, -1), M, t.input_dim, ptr(t.trellis), t.output_dim,
                                t.bits2, t.codebook, ptr(y), stream())
    else:
        rc = L.ishz_exl3_matvec_ws(ptr(xh), DTYPES.get(xh.dtype, -1), M, t.input_dim, ptr(t.trellis), t.output_dim,
                                   t.bits2, t.codebook, ptr(y), ptr(workspace), workspace.numel(), stream())
    return y if _lib.check(rc, "exl3_matvec") else None


def matvec_workspace_size(M, t):
    return _lib.lib().ishz_exl3_matvec_workspace_size(M, t.input_dim, t.output_dim)


def apply(x, t):
    """EXL3Kernels.apply: rotate in, matvec, rotate out; x [..., K] fp16 with up to 16 rows."""
    require_cuda(x, t.trellis)
    shape = x.shape
    x2 = x.reshape(-1, t.input_dim).contiguous()
    M = x2.shape[0]
    L = _lib.lib()
    ws = torch.empty(L.ishz_exl3_workspace_size(M, t.input_dim, t.output_dim), dtype=torch.uint8, device=x.device)
    y = torch.empty((M, t.output_dim), dtype=x.dtype, device=x.device)
    rc = L.ishz_exl3_apply(ptr(x2), DTYPES.get(x.dtype, -1), M, t.input_dim, ptr(t.trellis), ptr(t.suh),
                           ptr(t.svh), t.output_dim, t.bits2, t.codebook, ptr(y), ptr(ws), ws.numel(), stream())
    if not _lib.check(rc, "exl3_apply"):
        return None
    return y.reshape(*shape[:-1], t.output_dim)
