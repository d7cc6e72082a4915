"""GGMLKernels for MI355X: the reference's quantized GGUF matmul API over libishizuki_hip.

Mirrors Sources/IshizukiKit/Core/GGMLKernels.swift: each call returns a fresh tensor, or None
when the kernel declines (the reference's nil: unsupported type, rows out of range, K not a whole
number of blocks, short buffer), so the caller can fall back.
"""
import torch

from . import _lib
from ._torch import DTYPES, TORCH, ptr, require_cuda, stream

Q4_0, Q2_K, Q4_K, Q6_K = 2, 10, 12, 14
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 17, 18, 19, 21, 22, 23, 29
NAMES = {Q4_0: "Q4_0", Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS",
         IQ3_XXS: "IQ3_XXS", IQ1_S: "IQ1_S", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS", IQ1_M: "IQ1_M"}
# GGMLDequant.supported (Core/GGMLDequant.swift:19-24) plus Q4_0
SUPPORTED = tuple(NAMES)

matvec_batch = range(1, 17)     # GGMLKernels.matvecBatch (:146)
matmul_few_rows = range(2, 9)   # GGMLKernels.matmulFewRows (:217)


def block_size(t):
    return _lib.lib().ishz_ggml_block_size(t)


def type_size(t):
    return _lib.lib().ishz_ggml_type_size(t)


def row_bytes(t, K):
    return K // block_size(t) * type_size(t)


def matvec(x, blocks, type_, output_dim):
    """GGMLKernels.matvec (Core/GGMLKernels.swift:177): x [M, K] -> [M, N] in x.dtype. A narrow
    output with M >= 2 is split along K into a temporary fp32 workspace, as the reference's
    split-K verify returns [split, m, n] fp32 parts and sums them."""
    require_cuda(x, blocks)
    if x.dim() != 2:
        return None
    x = x.contiguous()
    M, K = x.shape
    L = _lib.lib()
    y = torch.empty((M, output_dim), dtype=x.dtype, device=x.device)
    wsb = L.ishz_ggml_workspace_size(type_, M, K, output_dim)
    ws = torch.empty(wsb, dtype=torch.uint8, device=x.device) if wsb else None
    rc = L.ishz_ggml_matvec_ws(type_, ptr(x), DTYPES.get(x.dtype, -1), M, K, ptr(blocks),
                               blocks.numel() * blocks.element_size(), output_dim, ptr(y),
                               ptr(ws) if ws is not None else None, wsb, stream())
    return y if _lib.check(rc, "ggml_matvec") else None


def matmul_few(x, blocks, type_, output_dim, row_blocks=2):
    """GGMLKernels.matmulFew (:219): M in 2..8, 256-element blocks."""
    require_cuda(x, blocks)
    if x.dim() != 2:
        return None
    x = x.contiguous()
    M, K = x.shape
    y = torch.empty((M, output_dim), dtype=x.dtype, device=x.device)
    rc = _lib.lib().ishz_ggml_matmul_few(type_, ptr(x), DTYPES.get(x.dtype, -1), M, K, ptr(blocks),
                                         blocks.numel() * blocks.element_size(), output_dim,
                                         row_blocks, ptr(y), stream())
    return y if _lib.check(rc, "ggml_matmul_few") else None


def dequantize(blocks, type_, shape, dtype=torch.bfloat16):
    """GGMLKernels.dequantize (:60): blocks -> dense array of `shape`."""
    require_cuda(blocks)
    count = 1
    for s in shape:
        count *= s
    out = torch.empty(count, dtype=dtype, device=blocks.device)
    rc = _lib.lib().ishz_ggml_dequant(type_, ptr(blocks), blocks.numel() * blocks.element_size(),
                                      count, ptr(out), DTYPES.get(dtype, -1), stream())
    return out.view(*shape) if _lib.check(rc, "ggml_dequant") else None


def gather(ids, blocks, type_, input_dim, dtype=torch.bfloat16, rows=None):
    """GGMLKernels.gather (:102): rows `ids` of W [rows, input_dim] -> [len(ids), input_dim]."""
    require_cuda(ids, blocks)
    ids = ids.reshape(-1).to(torch.int32).contiguous()
    nbytes = blocks.numel() * blocks.element_size()
    if rows is None:
        rb = row_bytes(type_, input_dim) if block_size(type_) else 0
        rows = nbytes // rb if rb else 0
    out = torch.empty((ids.numel(), input_dim), dtype=dtype, device=blocks.device)
    rc = _lib.lib().ishz_ggml_gather(type_, ptr(ids), ids.numel(), ptr(blocks), nbytes, rows,
                                     input_dim, ptr(out), DTYPES.get(dtype, -1), stream())
    return out if _lib.check(rc, "ggml_gather") else None


def dense_from_rows(nbytes):
    """Fewest rows at which dequantize + fp16 GEMM beats 16-row streaming passes (measured on
    MI355X with Q4_K, `python bench.py --policy`: 32 rows for a 2.9 MB attention projection, 48
    for the 74 MB MLP projections)."""
    return 32 if nbytes < 10_000_000 else 48


def apply(h, blocks, type_, output_dim):
    """PackedLinear.ggmlApply (Core/Hadamard.swift:145-178) with the row policy re-measured on
    MI355X: up to 16 rows is one matvec call (the reference splits 5..16 rows into matmulFew calls
    of 8; here the matvec's MFMA path already decodes each weight once for all 16); more rows are
    16-row calls until the dense path pays, then the weight is expanded once and multiplied."""
    shape = h.shape
    x = h.reshape(-1, shape[-1])
    rows, K = x.shape
    if rows <= 16:
        y = matvec(x, blocks, type_, output_dim)
    elif rows < dense_from_rows(blocks.numel()):
        parts = [matvec(x[r:r + 16], blocks, type_, output_dim) for r in range(0, rows, 16)]
        y = None if any(p is None for p in parts) else torch.cat(parts, 0)
    else:
        w = dequantize(blocks, type_, (output_dim, K), dtype=x.dtype)
        y = None if w is None else x @ w.t()
    if y is None:
        return None
    return y.reshape(*shape[:-1], output_dim)
