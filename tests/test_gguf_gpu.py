"""GGUF load -> device upload -> fused matvec, checked against the CPU oracle.

The packed half of GGUFWeights.load (Sources/IshizukiKit/Core/GGUFWeights.swift:47-85): a
quantized tensor's blocks reach HBM exactly as they lie in the file, and the kernels run on them."""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from ishizuki_amd import ggml, gguf, synth
from tests import gguf_writer as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_upload_then_matvec(tmp_path):
    N, K = 96, 2048
    payloads = {f"blk.0.{n}.weight": synth.ggml_blocks(t, N, K, seed=t).tobytes()
                for n, t in (("q4k", ggml.Q4_K), ("q6k", ggml.Q6_K), ("iq2", ggml.IQ2_XS), ("q40", ggml.Q4_0))}
    types = {"q4k": ggml.Q4_K, "q6k": ggml.Q6_K, "iq2": ggml.IQ2_XS, "q40": ggml.Q4_0}
    tensors = [(f"blk.0.{n}.weight", [N, K], t) for n, t in types.items()] + [("norm.weight", [K], 0)]
    path = W.write(tmp_path / "w.gguf", tensors, [("general.architecture", W.STRING, W.string("t"))],
                   payloads=payloads)
    with gguf.GGUFFile(path) as f:
        blocks = gguf.load_blocks(f, DEV)
        assert set(blocks) == set(payloads)  # the F32 norm is not a packed tensor
        x = synth.fp16_normal((1, K), seed=3)
        for name, b in blocks.items():
            assert b.shape == (N, K)
            assert bytes(b.bytes.cpu().numpy()) == payloads[name]
            y = ggml.matvec(torch.from_numpy(x).to(DEV), b.bytes, b.type, N)
            ref = oracle.ggml_matmul(b.type, x.astype(np.float32), np.frombuffer(payloads[name], np.uint8), N)
            assert_close(y.float().cpu().numpy(), ref, what=name)


def test_upload_refuses_short_buffer(tmp_path):
    path = W.write(tmp_path / "s.gguf", [("w", [4, 256], ggml.Q4_K)])
    with gguf.GGUFFile(path) as f:
        small = torch.empty(10, dtype=torch.uint8, device=DEV)
        from ishizuki_amd import _lib
        from ishizuki_amd._torch import ptr, stream
        assert _lib.lib().ishz_gguf_tensor_upload(f._h, 0, ptr(small), 10, stream()) != _lib.OK
