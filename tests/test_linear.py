"""PackedLinear construction checks (Core/Hadamard.swift:49-85), no GPU needed."""
import pytest
import torch

from ishizuki_amd.linear import PackedLinear


def pack(N=8, K=256, group=64, bits=2):
    return (torch.zeros((N, K * bits // 32), dtype=torch.int32), torch.ones((N, K // group), dtype=torch.float16),
            torch.zeros((N, K // group), dtype=torch.float16))


def test_input_width_comes_from_the_groups():
    w, s, b = pack(K=512, group=128)
    lin = PackedLinear(w, s, b, group_size=128)
    assert (lin.output_dim, lin.input_dim) == (8, 512)


def test_rotated_module_needs_signs():
    w, s, b = pack()
    with pytest.raises(ValueError, match="missing its sign vector"):
        PackedLinear(w, s, b, block=128, group_size=64)


def test_sign_vector_width():
    w, s, b = pack()
    with pytest.raises(ValueError, match="wide"):
        PackedLinear(w, s, b, signs=torch.ones(128), block=128, group_size=64)


def test_block_divides_width():
    w, s, b = pack(K=384, group=64)
    with pytest.raises(ValueError, match="does not divide"):
        PackedLinear(w, s, b, signs=torch.ones(384), block=256, group_size=64)


def test_dense():
    lin = PackedLinear.dense(torch.zeros((6, 32), dtype=torch.float16))
    assert lin.is_dense and (lin.output_dim, lin.input_dim) == (6, 32)
