"""PackedLinear for MI355X: one projection, whatever its weights are held as.

Mirrors PackedLinear (Sources/IshizukiKit/Core/Hadamard.swift:25-252): the same four kinds of
weight and the same checks at construction (BonsaiError there, ValueError here), and a forward
that dispatches as `callAsFunction` (:180-231) does:

* GGUF blocks -> `ggml.apply` (ggmlApply, :145-178, with the MI355X row policy);
* EXL3 -> `exl3.apply` (EXL3Kernels.apply);
* dense fp16 -> `x @ W^T`;
* MLX affine pack (2, 4 or 8 bits), rotated by a blockwise Hadamard transform when `block` > 0
  -> `affine.linear` (rotation fused for blocks up to 128, then the quantized matmul), in calls
  of at most 16 rows.

The forward returns None where the reference's kernels return nil (a declined shape or dtype).
"""
import torch

from . import affine, exl3, ggml


class PackedLinear:
    def __init__(self, weight, scales, biases, signs=None, block=0, group_size=128, bits=2):
        """A quantized projection (Hadamard.swift:49-85): codes [N, K * bits / 32] (int32),
        scales / biases [N, K / group_size]; `signs` [K] required when `block` > 0."""
        self.weight, self.scales, self.biases = weight, scales, biases
        self.signs, self.block, self.group_size, self.bits = signs, block, group_size, bits
        self.is_dense, self.ggml, self.exl3 = False, None, None
        self.output_dim = weight.shape[0]
        self.input_dim = scales.shape[1] * group_size
        if block > 0:
            if signs is None:
                raise ValueError("rotated module is missing its sign vector")
            if signs.shape[0] != self.input_dim:
                raise ValueError(f"sign vector is {signs.shape[0]} wide, expected {self.input_dim}")
            if self.input_dim % block:
                raise ValueError(f"Hadamard block {block} does not divide input width {self.input_dim}")

    @classmethod
    def dense(cls, weight):
        """init(dense:) (:92-108): the real fp16 weight [N, K]."""
        self = cls.__new__(cls)
        self.weight, self.scales, self.biases, self.signs = weight, None, None, None
        self.block, self.group_size, self.bits = 0, weight.shape[1], 16
        self.is_dense, self.ggml, self.exl3 = True, None, None
        self.output_dim, self.input_dim = weight.shape
        return self

    @classmethod
    def from_ggml(cls, blocks):
        """init(ggml:) (:110-124): a GGUF tensor still in blocks (`gguf.GGUFBlocks`)."""
        self = cls.__new__(cls)
        self.weight, self.scales, self.biases, self.signs = blocks.bytes, None, None, None
        self.block, self.group_size, self.bits = 0, ggml.block_size(blocks.type), 0
        self.is_dense, self.ggml, self.exl3 = False, blocks, None
        self.output_dim, self.input_dim = blocks.shape[0], blocks.shape[-1]
        return self

    @classmethod
    def from_exl3(cls, tensor):
        """init(exl3:) (:126-140): a trellis-coded EXL3 tensor."""
        self = cls.__new__(cls)
        self.weight, self.scales, self.biases, self.signs = tensor.trellis, None, None, None
        self.block, self.group_size, self.bits = 0, 256, int(tensor.bits2) // 2
        self.is_dense, self.ggml, self.exl3 = False, None, tensor
        self.output_dim, self.input_dim = tensor.output_dim, tensor.input_dim
        return self

    def __call__(self, x):
        if self.ggml is not None:
            return ggml.apply(x, self.ggml.bytes, self.ggml.type, self.output_dim)
        if self.exl3 is not None:
            shape = x.shape
            rows = x.reshape(-1, shape[-1])
            parts = [exl3.apply(rows[r:r + 16], self.exl3) for r in range(0, rows.shape[0], 16)]
            if any(p is None for p in parts):
                return None
            return torch.cat(parts, 0).reshape(*shape[:-1], self.output_dim)
        if self.is_dense:
            return x @ self.weight.t().to(x.dtype)
        shape = x.shape
        rows = x.reshape(-1, shape[-1])
        signs = self.signs if self.block > 0 else None
        parts = [affine.linear(rows[r:r + 16], self.weight, self.scales, self.biases, signs=signs, block=self.block,
                               group_size=self.group_size, bits=self.bits) for r in range(0, rows.shape[0], 16)]
        if any(p is None for p in parts):
            return None
        return torch.cat(parts, 0).reshape(*shape[:-1], self.output_dim)
