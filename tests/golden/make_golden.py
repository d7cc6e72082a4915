"""Extracts the reference's own known-answer vectors into small fixtures under tests/golden/.

Sources (data files held by the reference's tests, read as bytes, nothing executed):
  Tests/IshizukiKitTests/Fixtures/ggml-reference.bin          (GGMLDequantTests.swift:20-58)
      format GGMLREF1: u32 count, then per case {u32 type, u32 nblocks, u32 nbytes,
      u32 nfloats, bytes, f32[nfloats]} written by llama.cpp's to_float.
  Tests/IshizukiKitTests/Fixtures/exl3-reference.safetensors  (EXL3Tests.swift:15-55)
      r{rate}{h5}c{codebook}.trellis int16 [2,3,16*bits] / .expected f32 [32,48]
      (exllamav3's reconstruction), qwen3/qwen38 trellis + suh/svh + fp16 weight.

Outputs:
  tests/golden/ggml_reference.bin  -- the GGMLREF1 records, copied verbatim (all 14 types)
  tests/golden/exl3_reference.npz  -- every array of the safetensors file, as numpy arrays

Run from the repo root:  python tests/golden/make_golden.py /root/reference
"""
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DT = {"F16": np.float16, "F32": np.float32, "I16": np.int16, "I32": np.int32}


def read_safetensors(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    body = raw[8 + n:]
    out = {}
    for key, meta in header.items():
        if key == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        out[key] = np.frombuffer(body[a:b], dtype=DT[meta["dtype"]]).reshape(meta["shape"]).copy()
    return out


def main(ref):
    fx = os.path.join(ref, "Tests/IshizukiKitTests/Fixtures")
    raw = open(os.path.join(fx, "ggml-reference.bin"), "rb").read()
    assert raw[:8] == b"GGMLREF1"
    open(os.path.join(HERE, "ggml_reference.bin"), "wb").write(raw)
    arrays = read_safetensors(os.path.join(fx, "exl3-reference.safetensors"))
    np.savez_compressed(os.path.join(HERE, "exl3_reference.npz"), **arrays)
    print("ggml records:", struct.unpack("<I", raw[8:12])[0], "exl3 arrays:", len(arrays))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
