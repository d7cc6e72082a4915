"""The i-quant GEMV and verify decoders build fp16 sign-bit masks in registers by one multiply per
word (sign_words and iq2xs_sign_words in csrc/ggml_formats.h): the pattern shifted
left by 7 times a constant, both within 24 bits (v_mul_u32_u24). For every sign
pattern, the multiplied words must put sign bit j of the pattern on exactly the fp16 weight the
decoder pairs it with: natural order (w0,w1 | w2,w3 | ...) for sign_words, the GEMV's permuted
order (x0,x2 | x1,x3 | x4,x6 | x5,x7) for IQ2_XS. ksigns patterns carry their parity as bit 7
(ggml's ksigns_iq2xs table)."""
import os
import re

CSRC = os.path.join(os.path.dirname(__file__), "..", "ishizuki_amd", "csrc")


def _multipliers(fname, func):
    src = open(os.path.join(CSRC, fname)).read()
    body = src[src.index(func):]
    body = body[:body.index("}")]
    assert "<< 7" in body
    return [int(m, 16) for m in re.findall(r"mul24\(t, (0x[0-9A-Fa-f]+)u\)", body)]


def _masks(mults, s):
    t = s << 7
    assert t < 1 << 24
    out = []
    for m in mults:
        assert m < 1 << 24  # a 24-bit operand: the product is exact in 48 bits, low 32 kept
        out.append((t * m) & 0x80008000 & 0xFFFFFFFF)
    return out


def _expect(s, order):
    words = []
    for lo, hi in order:
        words.append((((s >> lo) & 1) << 15) | (((s >> hi) & 1) << 31))
    return words


def test_sign_words_natural_order_all_patterns():
    mults = _multipliers("ggml_formats.h", "DEV u4 sign_words(uint32_t s)")
    assert len(mults) == 4
    for s in range(256):
        assert _masks(mults, s) == _expect(s, [(0, 1), (2, 3), (4, 5), (6, 7)]), s


def test_iq2xs_sign_words_permuted_order_all_ksigns():
    mults = _multipliers("ggml_formats.h", "DEV u4 iq2xs_sign_words(uint32_t idx)")
    assert len(mults) == 4
    for idx in range(128):
        s = idx | (bin(idx).count("1") & 1) << 7
        assert bin(s).count("1") % 2 == 0  # ksigns patterns have even parity
        assert _masks(mults, s) == _expect(s, [(0, 2), (1, 3), (4, 6), (5, 7)]), idx
