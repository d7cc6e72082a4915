"""PackedLinear forward on the GPU, every kind of weight, against the CPU oracle (max |y - ref| <=
1e-3 * max |ref|); more than 16 rows go through in 16-row calls."""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from ishizuki_amd import exl3, ggml, gguf, synth
from ishizuki_amd.linear import PackedLinear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
dev = lambda a: torch.from_numpy(a).to(DEV)


@pytest.mark.parametrize("rows", [1, 3, 20])
def test_rotated_affine_2bit(rows):
    N, K = 300, 1024
    codes, s, b = synth.affine_pack(N, K, group=64, seed=rows)
    signs = synth.hadamard_signs(K, seed=3)
    x = synth.fp16_normal((rows, K), seed=rows + 1)
    xr = oracle.hadamard(x.astype(np.float32), 128, signs).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, 2, 64)
    lin = PackedLinear(dev(codes.view(np.int32)), dev(s), dev(b), signs=torch.from_numpy(signs), block=128,
                       group_size=64, bits=2)
    y = lin(dev(x))
    assert y is not None and y.shape == (rows, N)
    assert_close(y.float().cpu().numpy(), ref, what=f"PackedLinear affine rows={rows}")


def test_affine_4bit_three_dim_input():
    N, K = 200, 512
    codes, s, b = synth.affine_pack_bits(N, K, 4, group=128, seed=9)
    x = synth.fp16_normal((2, 3, K), seed=10)
    ref = oracle.affine_matmul(x.reshape(6, K).astype(np.float32), codes, s.view(np.uint16), b.view(np.uint16), N, 4,
                               128).reshape(2, 3, N)
    lin = PackedLinear(dev(codes.view(np.int32)), dev(s), dev(b), group_size=128, bits=4)
    y = lin(dev(x))
    assert y is not None and y.shape == (2, 3, N)
    assert_close(y.float().cpu().numpy(), ref, what="PackedLinear affine 4-bit")


def test_ggml_blocks():
    N, K, rows = 96, 1024, 5
    blk = synth.ggml_blocks(ggml.Q6_K, N, K, seed=11)
    x = synth.fp16_normal((rows, K), seed=12)
    ref = oracle.ggml_matmul(ggml.Q6_K, x.astype(np.float32), blk, N)
    lin = PackedLinear.from_ggml(gguf.GGUFBlocks(dev(blk), ggml.Q6_K, (N, K)))
    y = lin(dev(x))
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, what="PackedLinear ggml")


def test_exl3_and_dense():
    K, N, rows = 512, 256, 3
    t, suh, svh = synth.exl3_pack(K, N, bits2=4, seed=13)
    ten = exl3.EXL3Tensor(dev(t), dev(suh), dev(svh))
    x = synth.fp16_normal((rows, K), seed=14)
    ref = oracle.exl3_apply(x.astype(np.float32), t, suh, svh, 4, 0)
    y = PackedLinear.from_exl3(ten)(dev(x))
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, what="PackedLinear exl3")
    w = synth.fp16_normal((N, K), seed=15)
    yd = PackedLinear.dense(dev(w))(dev(x))
    refd = x.astype(np.float32) @ w.astype(np.float32).T
    assert_close(yd.float().cpu().numpy(), refd, what="PackedLinear dense")
