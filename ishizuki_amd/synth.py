"""Seeded synthetic weights and activations in the reference's packed formats.

The generators follow the benchmark configurations: uniform random codes and sub-scales, fp16
super-scales |N(0,1)| * scale. Each returns raw packed bytes exactly as a GGUF / MLX / EXL3 file
would hold them (numpy arrays), so the same bytes feed the GPU kernels and the CPU oracle.
"""
import numpy as np

Q4_0, Q2_K, Q4_K, Q6_K = 2, 10, 12, 14
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 17, 18, 19, 21, 22, 23, 29
BLOCK = {Q4_0: (32, 18), Q2_K: (256, 84), Q4_K: (256, 144), Q6_K: (256, 210), IQ2_XXS: (256, 66),
         IQ2_XS: (256, 74), IQ3_XXS: (256, 98), IQ1_S: (256, 50), IQ3_S: (256, 110), IQ2_S: (256, 82),
         IQ4_XS: (256, 136), IQ1_M: (256, 56)}
# byte offsets of fp16 super-scales inside a block (IQ1_M spreads its d over the top nibbles of
# the four scale words at 48..55)
SCALE_AT = {Q4_0: (0,), Q2_K: (80, 82), Q4_K: (0, 2), Q6_K: (208,), IQ2_XXS: (0,), IQ2_XS: (0,),
            IQ3_XXS: (0,), IQ1_S: (0,), IQ3_S: (0,), IQ2_S: (0,), IQ4_XS: (0,), IQ1_M: ()}


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
    if type_ == IQ1_M:
        d = fp16_absnormal(r, nb, scale).view(np.uint16).astype(np.uint16)
        w = blk[:, 48:56].copy().view(np.uint16)  # [nb, 4]
        for i in range(4):
            w[:, i] = (w[:, i] & 0x0FFF) | (((d >> (4 * i)) & 0xF) << 12)
        blk[:, 48:56] = w.view(np.uint8)
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


def affine_pack_bits(N, K, bits, group=64, seed=0, scale=0.02, return_codes=False):
    """MLX affine pack of `bits` in 2..8: uniform random codes, code k at bit k * bits of the row's
    little-endian u32 stream (for bits dividing 32: bits (k % (32/bits)) * bits of word
    k / (32/bits)), scales |N|*scale and biases -s * 2^(bits-1) (fp16), so weights are centred
    on zero. return_codes: also the codes themselves [N, K]."""
    assert 2 <= bits <= 8 and (K * bits) % 32 == 0
    r = rng(seed)
    q = r.integers(0, 1 << bits, size=(N, K), dtype=np.uint64)
    pos = np.arange(K, dtype=np.uint64) * np.uint64(bits)
    word, off = (pos // np.uint64(32)).astype(np.int64), pos % np.uint64(32)
    acc = np.zeros((N, K * bits // 32 + 1), np.uint64)  # 64-bit words: a code may spill into the next
    np.add.at(acc, (slice(None), word), q << off)       # disjoint bits: the sum is the OR
    lo = acc & np.uint64(0xFFFFFFFF)
    codes = lo.copy()
    codes[:, 1:] += acc[:, :-1] >> np.uint64(32)         # the spill of word w lands in word w + 1
    codes = codes[:, :K * bits // 32].astype(np.uint32)
    s = fp16_absnormal(r, N * (K // group), scale).reshape(N, K // group)
    b = (-s.astype(np.float32) * (1 << (bits - 1))).astype(np.float16)
    if return_codes:
        return codes, s, b, q.astype(np.uint32)
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
