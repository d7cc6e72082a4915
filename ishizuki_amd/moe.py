"""MoE expert-gathered quantized FFN on MI355X.

Mirrors MoEBlock.callAsFunction / ResidentExperts.swiglu (Sources/IshizukiKit/Text/MoEBlock.swift:
124-171) over libishizuki_hip, for GGML-block experts and for MLX affine stacked experts
(StackedExperts, :22-50; 4- or 8-bit packs): routing, gate+up with SwiGLU, down, weighted sum.
Only the routed experts' weights are read.
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


def _shared_ptrs(x, shared, shared_gate):
    """The shared expert's output [T, H] and gate logit [T] (x's dtype), or (None, None)."""
    if (shared is None) != (shared_gate is None):
        raise ValueError("the shared expert needs both its output and its gate")
    if shared is None:
        return None, None, ()
    T, H = x.shape
    shared = shared.to(x.dtype).contiguous().view(T, H)
    shared_gate = shared_gate.to(x.dtype).contiguous().view(T)
    return ptr(shared), ptr(shared_gate), (shared, shared_gate)


def swiglu(x, logits, experts, top_k=8, normalize=True, return_routing=False, shared=None, shared_gate=None):
    """y [T, H] = sum_k w_k * down_k(silu(gate_k(x)) * up_k(x)) (+ sigmoid(shared_gate) * shared,
    the shared expert, when given); None if declined."""
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
    sp, sgp, _keep = _shared_ptrs(x, shared, shared_gate)
    rc = L.ishz_moe_swiglu(ex.type, ptr(x), DTYPES.get(x.dtype, -1), T, H, ptr(logits), ex.E, top_k,
                           int(normalize), ptr(ex.gate), ptr(ex.up), ptr(ex.down), ex.expert_bytes, ex.I,
                           sp, sgp, ptr(y), ptr(ids), ptr(w), ptr(ws), ws.numel(), stream())
    if not _lib.check(rc, "moe_swiglu"):
        return None
    return (y, ids, w) if return_routing else y


class AffineExperts:
    """StackedExperts (Text/MoEBlock.swift:22-50) for gate, up ([E, I, H]) and down ([E, H, I]): each
    an MLX affine pack (codes int32 [E, rows, K * bits / 32], scales / biases fp16 or bf16
    [E, rows, K / group])."""

    def __init__(self, gate, up, down, bits, group, experts, hidden, intermediate):
        self.gate = tuple(t.contiguous() for t in gate)
        self.up = tuple(t.contiguous() for t in up)
        self.down = tuple(t.contiguous() for t in down)
        self.bits, self.group, self.E, self.H, self.I = bits, group, experts, hidden, intermediate


def swiglu_affine(x, logits, experts, top_k=8, normalize=True, return_routing=False, shared=None,
                  shared_gate=None):
    """The MoE FFN over affine stacked experts (shared expert as in swiglu); None if declined."""
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
    (gc, gs, gb), (uc, us, ub), (dc, ds, db) = ex.gate, ex.up, ex.down
    sp, sgp, _keep = _shared_ptrs(x, shared, shared_gate)
    rc = L.ishz_moe_swiglu_affine(ptr(x), DTYPES.get(x.dtype, -1), T, H, ptr(logits), ex.E, top_k, int(normalize),
                                  ptr(gc), ptr(gs), ptr(gb), ptr(uc), ptr(us), ptr(ub), ptr(dc), ptr(ds), ptr(db),
                                  DTYPES.get(gs.dtype, -1), ex.bits, ex.group, ex.I, sp, sgp, ptr(y), ptr(ids),
                                  ptr(w), ptr(ws), ws.numel(), stream())
    if not _lib.check(rc, "moe_swiglu_affine"):
        return None
    return (y, ids, w) if return_routing else y
