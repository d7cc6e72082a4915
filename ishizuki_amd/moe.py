"""MoE expert-gathered quantized FFN on MI355X.

Mirrors MoEBlock.callAsFunction / ResidentExperts.swiglu (Sources/IshizukiKit/Text/MoEBlock.swift:
124-171) for GGML-block experts over libishizuki_hip: routing, gate+up with SwiGLU, down, weighted
sum. Only the routed experts' blocks are read.
"""
import torch

from . import _lib, ggml
from ._torch import DTYPES, ptr, require_cuda, stream


def route(logits, top_k, normalize=True):
    """fp32 softmax over experts, top-k (ties to the lower index), renormalised."""
    require_cuda(logits)
    logits = logits.float().contiguous()
    T, E = logits.shape
    ids = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    rc = _lib.lib().ishz_moe_route(ptr(logits), T, E, top_k, int(normalize), ptr(ids), ptr(w), stream())
    if not _lib.check(rc, "moe_route"):
        raise ValueError(_lib.last_error())
    return ids, w


class GGMLExperts:
    """E experts' gate/up [E, I, H] and down [E, H, I] as GGML blocks (raw bytes, uint8)."""

    def __init__(self, gate, up, down, type_, experts, hidden, intermediate):
        self.gate, self.up, self.down = gate.contiguous(), up.contiguous(), down.contiguous()
        self.type, self.E, self.H, self.I = type_, experts, hidden, intermediate
        self.expert_bytes = intermediate * ggml.row_bytes(type_, hidden)


def swiglu(x, logits, experts, top_k=8, normalize=True, return_routing=False):
    """y [T, H] = sum_k w_k * down_k(silu(gate_k(x)) * up_k(x)); None if declined."""
    require_cuda(x, logits)
    x = x.contiguous()
    logits = logits.float().contiguous()
    T, H = x.shape
    ex = experts
    L = _lib.lib()
    ws = torch.empty(L.ishz_moe_workspace_size(T, H, ex.E, ex.I, top_k), dtype=torch.uint8, device=x.device)
    y = torch.empty((T, H), dtype=x.dtype, device=x.device)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    rc = L.ishz_moe_swiglu(ex.type, ptr(x), DTYPES.get(x.dtype, -1), T, H, ptr(logits), ex.E, top_k,
                           int(normalize), ptr(ex.gate), ptr(ex.up), ptr(ex.down), ex.expert_bytes, ex.I,
                           ptr(y), ptr(ids), ptr(w), ptr(ws), ws.numel(), stream())
    if not _lib.check(rc, "moe_swiglu"):
        return None
    return (y, ids, w) if return_routing else y
