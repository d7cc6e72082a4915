"""Seeded synthetic weights and activations in the reference's packed formats.

The generators follow the benchmark configurations: uniform random codes and sub-scales, fp16
super-scales |N(0,1)| * scale. Each returns raw packed bytes exactly as a GGUF / MLX / EXL3 file
would hold them (numpy arrays), so the same bytes feed the GPU kernels and the CPU oracle.
"""
import numpy as np

Q4_0, Q4_K, Q6_K, IQ2_XS = 2, 12, 14, 17
BLOCK = {Q4_0: (32, 18), Q4_K: (256, 144), Q6_K: (256, 210), IQ2_XS: (256, 74)}
# byte offsets of fp16 super-scales inside a block
SCALE_AT = {Q4_0: (0,), Q4_K: (0, 2), Q6_K: (208,), IQ2_XS: (0,)}


def rng(seed):
    return np.random.default_rng(seed)


def fp16_absnormal(r, n, scale):
    return (np.abs(r.standard_normal(n)) * scale).astype(np.float16)


def ggml_blocks(type_, N, K, seed=0, scale=0.01):
    """GGML blocks for W [N, K]: uniform random bytes with fp16 |N(0,1)|*scale super-scales."""
    bs, ts = BLOCK[type_]
    assert K % bs == 0
    r = rng(seed)
    nb = N * (K // bs)
    blk = r.integers(0, 256, size=(nb, ts), dtype=np.uint8)
    for off in SCALE_AT[type_]:
        blk[:, off:off + 2] = fp16_absnormal(r, nb, scale).view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def fp16_normal(shape, seed=0):
    return rng(seed).standard_normal(shape).astype(np.float16)


def affine_pack(N, K, group=64, bits=2, seed=0, scale=0.02, probs=(0.3, 0.4, 0.3)):
    """MLX affine pack (Quantize/WeightedAffineQuantizer.swift:142-153): codes u32 [N, K*bits/32]
    (value k at bits (k % (32/bits)) * bits of word k / (32/bits)), scales s = |N|*scale and
    biases -s as fp16 [N, K/group], so codes {0,1,2} are {-s, 0, +s}."""
    assert bits == 2
    r = rng(seed)
    q = r.choice(len(probs), size=(N, K), p=probs).astype(np.uint32)
    per = 32 // bits
    q = q.reshape(N, K // per, per)
    codes = np.zeros((N, K // per), np.uint32)
    for i in range(per):
        codes |= q[:, :, i] << np.uint32(bits * i)
    s = fp16_absnormal(r, N * (K // group), scale).reshape(N, K // group)
    b = (-s.astype(np.float32)).astype(np.float16)
    return codes, s, b


def exl3_pack(K, N, bits2=4, seed=0, scale=0.02):
    """EXL3 tensor: trellis int16 [K/16, N/16, 8*bits2] of uniform random bits, and suh/svh
    scales fp16 |N(0,1)|*scale."""
    r = rng(seed)
    t = r.integers(-32768, 32768, size=(K // 16, N // 16, 8 * bits2), dtype=np.int16)
    suh = fp16_absnormal(r, K, scale)
    svh = fp16_absnormal(r, N, scale)
    return t, suh, svh


def hadamard_signs(width, seed=None):
    """All +1, or a seeded +-1 vector."""
    if seed is None:
        return np.ones(width, np.float32)
    return np.where(rng(seed).integers(0, 2, width) == 1, 1.0, -1.0).astype(np.float32)
