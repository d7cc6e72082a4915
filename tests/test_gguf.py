"""GGUF container reader (C ABI in csrc/gguf.cpp, Python mirror in ishizuki_amd/gguf.py).

Cases follow the reference's suite (Tests/IshizukiKitTests/GGUFTests.swift:17-86: blockGeometry,
containerRoundTrip, refusesRaggedBlocks) plus the malformed-file refusals of
Sources/IshizukiKit/Config/GGUFFile.swift:205-300 (magic, version, truncation, alignment, data past
the end of the file, unknown types)."""
import struct

import pytest

from ishizuki_amd import gguf
from ishizuki_amd.gguf import GGUFError, GGUFFile
from tests import gguf_writer as W

F32, F16, Q4_0, Q2_K, Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M, BF16 = (
    0, 1, 2, 10, 12, 14, 16, 17, 18, 19, 20, 21, 22, 23, 29, 30)


def test_block_geometry():
    """GGUFTests.swift:17-35; the remaining types' geometry is the published ggml table."""
    expected = [(F32, 1, 4), (F16, 1, 2), (BF16, 1, 2), (Q2_K, 256, 84), (Q4_K, 256, 144), (Q6_K, 256, 210),
                (IQ1_S, 256, 50), (IQ1_M, 256, 56), (IQ2_XXS, 256, 66), (IQ2_XS, 256, 74), (IQ2_S, 256, 82),
                (IQ3_XXS, 256, 98), (IQ3_S, 256, 110), (IQ4_NL, 32, 18), (IQ4_XS, 256, 136),
                (Q4_0, 32, 18), (3, 32, 20), (6, 32, 22), (7, 32, 24), (8, 32, 34), (9, 32, 36),
                (11, 256, 110), (13, 256, 176), (15, 256, 292), (24, 1, 1), (25, 1, 2), (26, 1, 4),
                (27, 1, 8), (28, 1, 8)]
    for t, bs, ts in expected:
        assert gguf.geometry(t) == (bs, ts), gguf.GGML_TYPES[t]
    # 5120 x 248320 at IQ1_M is 278,118,400 bytes (the smallest published build's embedding).
    assert gguf.byte_count(IQ1_M, 5120 * 248320) == 278_118_400
    for t in (4, 5, 31, 39, 1000):
        with pytest.raises(GGUFError):
            gguf.geometry(t)


def _round_trip_file(tmp_path):
    meta = [("general.architecture", W.STRING, W.string("qwen35")),
            ("qwen35.block_count", W.U32, W.u32(2)),
            ("qwen35.rope.freq_base", W.F32, W.f32(10_000_000)),
            ("qwen35.rope.dimension_sections", W.ARRAY, W.int_array([11, 11, 10, 0])),
            ("tokenizer.ggml.tokens", W.ARRAY, W.string_array(["a", "b", "c"]))]
    tensors = [("token_embd.weight", [3, 256], IQ1_M), ("output_norm.weight", [256], F32),
               ("blk.0.attn_qkv.weight", [512, 256], IQ2_XS)]
    return W.write(tmp_path / "rt.gguf", tensors, meta)


def test_container_round_trip(tmp_path):
    """GGUFTests.swift:37-73."""
    with GGUFFile(_round_trip_file(tmp_path)) as f:
        assert f.version == 3
        assert f.architecture == "qwen35"
        assert f.architecture_value("block_count").int_value == 2
        assert f.architecture_value("rope.freq_base").float_value == 10_000_000
        assert f.architecture_value("rope.dimension_sections").int_array == [11, 11, 10, 0]
        assert f["tokenizer.ggml.tokens"].string_array == ["a", "b", "c"]
        assert len(f.tensors) == 3
        qkv = f.tensor("blk.0.attn_qkv.weight")
        assert qkv.shape == (512, 256) and qkv.type == IQ2_XS
        assert qkv.byte_count == 512 * 256 // 256 * 74
        emb = f.tensor("token_embd.weight")
        assert len(f.data(emb)) == emb.byte_count
        assert (F32, 1) in f.type_histogram
        assert f.data_offset % 32 == 0
        assert f.tensor("missing") is None and f["missing"] is None


def test_tensor_bytes_and_offsets(tmp_path):
    """Offsets are relative to the aligned data section; payloads come back byte for byte."""
    a, b = bytes(range(256)) * 72, bytes([7, 9]) * 512  # 18432 bytes = 512x64 Q4_0; 1024 bytes = 512 f16
    p = W.write(tmp_path / "p.gguf", [("a", [512, 64], Q4_0), ("b", [512], F16)],
                [("general.architecture", W.STRING, W.string("x"))], payloads={"a": a, "b": b})
    with GGUFFile(p) as f:
        assert f.data(f.tensor("a")) == a and f.data(f.tensor("b")) == b
        assert f.tensor("a").offset == 0 and f.tensor("b").offset == len(a)
        assert f.tensor("b").element_count == 512


def test_metadata_value_types(tmp_path):
    meta = [("u8", W.U8, b"\xfe"), ("i8", W.I8, b"\xfe"), ("u16", W.U16, struct.pack("<H", 65535)),
            ("i16", W.I16, struct.pack("<h", -3)), ("i32", W.I32, struct.pack("<i", -70000)),
            ("u64", W.U64, struct.pack("<Q", 1 << 40)), ("i64", W.I64, struct.pack("<q", -(1 << 40))),
            ("f64", W.F64, struct.pack("<d", 0.125)), ("b", W.BOOL, b"\x01"),
            ("neg", W.ARRAY, W.int_array([-1, 2])), ("nested", W.ARRAY, W.u32(W.ARRAY) + struct.pack("<Q", 1)
                                                    + W.u32(W.U8) + struct.pack("<Q", 2) + b"\x01\x02")]
    with GGUFFile(W.write(tmp_path / "m.gguf", [], meta)) as f:
        assert f["u8"].int_value == 254 and f["i8"].int_value == -2 and f["u16"].int_value == 65535
        assert f["i16"].int_value == -3 and f["i32"].int_value == -70000
        assert f["u64"].int_value == 1 << 40 and f["i64"].int_value == -(1 << 40)
        assert f["f64"].float_value == 0.125 and f["b"].bool_value is True
        assert f["u8"].string_value is None and f["b"].int_value == 1 and f["u8"].bool_value is True
        assert f["neg"].float_value is None and f["b"].float_value is None
        assert f["neg"].int_array == [-1, 2]
        assert f["nested"].array_value[0].int_array == [1, 2]
        assert f.architecture == ""


def test_refuses_ragged_blocks(tmp_path):
    """GGUFTests.swift:75-86."""
    p = W.write(tmp_path / "r.gguf", [("blk.0.ffn_up.weight", [4, 100], IQ2_XS)],
                [("general.architecture", W.STRING, W.string("qwen35"))])
    with pytest.raises(GGUFError):
        GGUFFile(p)


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "past_eof", "unknown_type", "alignment",
                                  "rank", "missing"])
def test_refuses_malformed(tmp_path, case):
    tensors = [("w", [4, 256], Q4_K)]
    meta = [("general.architecture", W.STRING, W.string("q"))]
    if case == "magic":
        data = W.build(tensors, meta, magic=0x46554746)
    elif case == "version":
        data = W.build(tensors, meta, version=1)
    elif case == "truncated":
        data = W.build(tensors, meta)[:40]
    elif case == "past_eof":
        data = W.build(tensors, meta)[:-1]
    elif case == "unknown_type":
        data = W.build([("w", [4, 256], 4)], meta)
    elif case == "alignment":
        data = W.build(tensors, meta + [("general.alignment", W.U32, W.u32(48))])
    elif case == "rank":
        data = W.build([("w", [1, 1, 1, 1, 256], F32)], meta)
    path = tmp_path / "bad.gguf"
    if case != "missing":
        path.write_bytes(data)
    with pytest.raises(GGUFError):
        f = GGUFFile(path)
        f.data(f.tensors[0])


def test_custom_alignment(tmp_path):
    tensors = [("a", [1, 256], Q4_K), ("b", [256], F32)]
    p = W.write(tmp_path / "al.gguf", tensors, [("general.alignment", W.U32, W.u32(64))], alignment=64)
    with GGUFFile(p) as f:
        assert f.data_offset % 64 == 0
        assert f.tensor("b").offset == 192 and len(f.data(f.tensor("b"))) == 1024
