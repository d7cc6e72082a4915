"""The CPU oracle against the reference's own known-answer vectors and closed forms.

ggml_reference.bin is llama.cpp's to_float output for 8 pseudo-random blocks per type
(the fixture of Tests/IshizukiKitTests/GGMLDequantTests.swift:60-85), NaN == NaN.
exl3_reference.npz holds exllamav3's reconstructions (EXL3Tests.swift:44-55).
"""
import numpy as np
import pytest

import oracle
from conftest import bits_equal

ALL_TYPES = [0, 1, 30, 10, 12, 14, 19, 29, 16, 17, 22, 18, 21, 23]


@pytest.mark.parametrize("t", ALL_TYPES)
def test_dequant_matches_llama_cpp(golden_ggml, t):
    b, e = golden_ggml[t]
    assert bits_equal(oracle.dequant(t, b, e.size), e)


def test_golden_covers_every_type(golden_ggml):
    assert sorted(golden_ggml) == sorted(ALL_TYPES)


def test_refusals():
    # GGMLDequantTests.refusesUnsupported / refusesShortBuffer (:87-105)
    with pytest.raises(ValueError):
        oracle.dequant(11, np.zeros(1024, np.uint8), 256)      # Q3_K: no dequantizer
    with pytest.raises(ValueError):
        oracle.dequant(17, np.zeros(73, np.uint8), 256)        # short buffer
    with pytest.raises(ValueError):
        oracle.dequant(17, np.zeros(1024, np.uint8), 100)      # not whole blocks


def test_q4_0_closed_form():
    # Q4_0 has no reference decoder: pinned by ggml's block definition, element j of a block is
    # (lo(qs[j]) - 8) * d and element j + 16 is (hi(qs[j]) - 8) * d.
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    y = oracle.dequant(2, blk, 32)
    assert np.array_equal(y[:16], (np.arange(16) - 8) * 0.5)
    assert np.array_equal(y[16:], (np.arange(16)[::-1] - 8) * 0.5)
    # every code once, with a subnormal and a negative scale
    for d in (np.float16(-3.25), np.float16(6e-8)):
        blk[0:2] = np.array([d], np.float16).view(np.uint8)
        y = oracle.dequant(2, blk, 32)
        assert np.array_equal(y[:16], ((np.arange(16) - 8) * np.float32(d)).astype(np.float32))


def test_q4_k_matches_brute_force_layout():
    # One Q4_K block built by hand: scale j = j+1, min j = 2j, nibble pattern known.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0.25], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.125], np.float16).view(np.uint8)
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    mn = [0, 2, 4, 6, 8, 10, 12, 14]
    q = blk[4:16]
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    codes = np.random.default_rng(1).integers(0, 16, 256)
    for jj in range(4):
        for l in range(32):
            blk[16 + 32 * jj + l] = codes[64 * jj + l] | (codes[64 * jj + 32 + l] << 4)
    y = oracle.dequant(12, blk, 256)
    want = np.array([0.25 * sc[k // 32] * codes[k] - 0.125 * mn[k // 32] for k in range(256)], np.float32)
    assert np.array_equal(y, want)


def test_half_conversions():
    vals = np.array([0, -0.0, 1, -2.5, 65504, 6e-8, 1e-5, 3.14159, 70000, -1e9], np.float32)
    for v in vals:
        assert oracle.lib().ishzo_float_to_half(float(v)) == int(np.float32(v).astype(np.float16).view(np.uint16))
    for h in range(0, 65536, 7):
        f = oracle.lib().ishzo_half_to_float(h)
        ref = float(np.uint16(h).view(np.float16))
        assert (np.isnan(f) and np.isnan(ref)) or f == ref


EXL3_CASES = [("r1c0", 0), ("r2c1", 1), ("r3c2", 2), ("r4c0", 0), ("r5c2", 2), ("r6c1", 1),
              ("r7c2", 2), ("r8c0", 0), ("r1h5c2", 2), ("r2h5c2", 2), ("r3h5c2", 2)]


@pytest.mark.parametrize("name,cb", EXL3_CASES)
def test_exl3_decode_matches_exllamav3(golden_exl3, name, cb):
    t = golden_exl3[name + ".trellis"]
    w = oracle.exl3_dequant(t, t.shape[2] // 8, cb)
    assert bits_equal(w, golden_exl3[name + ".expected"])


@pytest.mark.parametrize("name,cb", [("qwen3", 0), ("qwen38", 2)])
def test_exl3_projection_reproduces_checkpoint(golden_exl3, name, cb):
    # EXL3Tests.projectionMatchesCheckpoint (:74-98): rel-L2 < 0.12 vs the original fp16 weight.
    t = golden_exl3[name + ".trellis"]
    suh = golden_exl3[name + ".suh"].astype(np.float32)
    svh = golden_exl3[name + ".svh"].astype(np.float32)
    ref = golden_exl3[name + ".weight"].astype(np.float32)
    x = np.random.default_rng(3).standard_normal((12, 128)).astype(np.float16).astype(np.float32)
    y = oracle.exl3_apply(x, t, suh, svh, t.shape[2] // 8, cb)
    want = x @ ref
    err = np.sqrt(((y - want) ** 2).sum() / (want ** 2).sum())
    assert err < 0.12


def _f16_round_pinned(pre, err):
    """fp16(v) for v within err of pre, where that rounding is determined (no fp16 rounding boundary
    inside [pre - err, pre + err]); NaN where either neighbour may come out."""
    lo = (pre - err).astype(np.float16).astype(np.float64)
    hi = (pre + err).astype(np.float16).astype(np.float64)
    return np.where(lo == hi, lo, np.nan)


@pytest.mark.parametrize("name,cb", [("qwen3", 0), ("qwen38", 2)])
def test_exl3_apply_composition_pinned(golden_exl3, name, cb):
    """oracle.exl3_apply against a float64 numpy restatement of EXL3Kernels.apply
    (Core/EXL3.swift:82-100): xr = fp16(H(x * suh) / sqrt(128)), yh = xr @ W (W the golden-pinned
    decode), y = fp16(H(yh) / sqrt(128) * svh), H the Sylvester matrix from its closed form (not the
    oracle's butterflies). The oracle's fp32 sums of 128 products and its fp32 butterflies differ
    from float64 by far less than 2^-20 of each output's bound sum |xr||W| (sqrt(128) times fp32's
    2^-24 per level at most); every output whose final fp16 rounding that difference cannot flip
    (about half of them) must equal the restatement's exactly, and every output lies within half an
    fp16 ulp plus that difference. A missing fp16 rounding of xr (about half an fp16 ulp of y, since
    |y| is about bound / 128) or svh applied before the transform fails. The reference's own
    criterion for the product, 1e-5 of the bound (EXL3Tests.swift:57-72), is 10x looser."""
    t = golden_exl3[name + ".trellis"]
    bits2 = t.shape[2] // 8
    suh = golden_exl3[name + ".suh"].astype(np.float64)
    svh = golden_exl3[name + ".svh"].astype(np.float64)
    W = oracle.exl3_dequant(t, bits2, cb).astype(np.float64)
    K, N = W.shape
    i = np.arange(128)
    H = np.where(np.bitwise_count(i[:, None] & i[None, :]) % 2, -1.0, 1.0) / np.sqrt(128.0)
    x = np.random.default_rng(11).standard_normal((12, K)).astype(np.float16).astype(np.float64)
    xr = ((x * suh).reshape(12, K // 128, 128) @ H).reshape(12, K).astype(np.float16).astype(np.float64)
    yh = xr @ W
    pre = (yh.reshape(12, N // 128, 128) @ H).reshape(12, N) * svh
    bh = np.abs(xr) @ np.abs(W)
    bound = np.repeat(bh.reshape(12, N // 128, 128).sum(2), 128, 1) / np.sqrt(128.0) * np.abs(svh)
    err = 2.0 ** -20 * bound
    y = oracle.exl3_apply(x.astype(np.float32), t, suh.astype(np.float32), svh.astype(np.float32), bits2,
                          cb).astype(np.float64)
    assert np.array_equal(y, y.astype(np.float16).astype(np.float64)), "outputs are not fp16 values"
    want = _f16_round_pinned(pre, err)
    fixed = ~np.isnan(want)
    assert fixed.mean() > 0.3
    assert np.array_equal(y[fixed], want[fixed])
    assert np.all(np.abs(y - pre) <= err + np.abs(pre) * 2.0 ** -11)


@pytest.mark.parametrize("block", [2, 8, 128, 512])
def test_hadamard_closed_form(block):
    # Sylvester order: H[i][j] = (-1)^popcount(i & j) / sqrt(b); orthonormal and symmetric.
    eye = np.eye(block, dtype=np.float32)
    H = oracle.hadamard(eye, block)
    i = np.arange(block)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    want = np.where(pc % 2 == 0, 1.0, -1.0) / np.sqrt(block)
    assert np.allclose(H, want, atol=1e-6)
    x = np.random.default_rng(0).standard_normal((3, 4 * block)).astype(np.float32)
    s = np.where(np.random.default_rng(1).integers(0, 2, 4 * block) == 1, 1.0, -1.0).astype(np.float32)
    y = oracle.hadamard(x, block, s)
    back = oracle.hadamard(y, block, s, inverse=True)
    assert np.allclose(back, x, atol=1e-5)


def test_affine_closed_form():
    from ishizuki_amd import synth
    codes, s, b = synth.affine_pack(8, 256, group=64, seed=2)
    w = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), 8, 256, 2, 64)
    q = np.stack([(codes[:, k // 16] >> np.uint32(2 * (k % 16))) & 3 for k in range(256)], 1)
    sf = np.repeat(s.astype(np.float32), 64, 1)
    assert np.array_equal(w, (sf * q + np.repeat(b.astype(np.float32), 64, 1)).astype(np.float32))
    assert set(np.unique(q)) <= {0, 1, 2}
    # {0, 1, 2} -> {-s, 0, +s} exactly
    assert np.array_equal(np.abs(w[q != 1]), sf[q != 1]) and np.all(w[q == 1] == 0)


@pytest.mark.parametrize("bits", [4, 8])
def test_affine_closed_form_wide(bits):
    """4- and 8-bit packs: field k of the row's u32 stream, restated with numpy bit ops."""
    from ishizuki_amd import synth
    N, K, g = 5, 256, 128
    codes, s, b = synth.affine_pack_bits(N, K, bits, group=g, seed=bits)
    w = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, bits, g)
    per = 32 // bits
    q = np.stack([(codes[:, k // per] >> np.uint32(bits * (k % per))) & np.uint32((1 << bits) - 1)
                  for k in range(K)], 1).astype(np.float32)
    sf = np.repeat(s.astype(np.float32), g, 1)
    bf = np.repeat(b.astype(np.float32), g, 1)
    assert np.array_equal(w, (sf * q + bf).astype(np.float32))
    assert q.max() == (1 << bits) - 1 and q.min() == 0


@pytest.mark.parametrize("bits", [3, 5, 6, 7, 4])
def test_affine_closed_form_stream(bits):
    """Any width: codes packed by numpy into the little-endian u32 stream (code k at bit k * bits,
    spilling into the next word), read back by the oracle's C decoder, give s * q + b for the
    codes that were packed."""
    from ishizuki_amd import synth
    N, K, g = 4, 256, 64
    codes, s, b, q = synth.affine_pack_bits(N, K, bits, group=g, seed=bits, return_codes=True)
    assert codes.shape == (N, K * bits // 32)
    w = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, bits, g)
    sf = np.repeat(s.astype(np.float32), g, 1)
    bf = np.repeat(b.astype(np.float32), g, 1)
    assert np.array_equal(w, (sf * q.astype(np.float32) + bf).astype(np.float32))
    assert q.max() == (1 << bits) - 1 and q.min() == 0


def test_matmul_fused_agrees_with_expanded():
    from ishizuki_amd import synth
    for t, K in ((2, 512), (12, 512), (14, 512), (17, 512)):
        blk = synth.ggml_blocks(t, 33, K, seed=t)
        x = np.random.default_rng(0).standard_normal((3, K)).astype(np.float32)
        a = oracle.ggml_matmul(t, x, blk, 33)
        f = oracle.ggml_matmul(t, x, blk, 33, fused=True)
        w = oracle.dequant(t, blk, 33 * K).reshape(33, K)
        assert np.allclose(a, x @ w.T, rtol=1e-4, atol=1e-4 * np.abs(a).max())
        assert np.allclose(a, f, rtol=1e-5, atol=1e-5 * np.abs(a).max())


def test_moe_route_matches_numpy():
    logits = np.random.default_rng(5).standard_normal((6, 128)).astype(np.float32)
    ids, w = oracle.moe_route(logits, 8)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    order = np.argsort(-p, 1, kind="stable")[:, :8]
    assert np.array_equal(ids, order)
    sel = np.take_along_axis(p, order, 1)
    assert np.allclose(w, sel / sel.sum(1, keepdims=True), rtol=1e-6)


def _affine_dense(codes, s, b, K, bits, group):
    """W from an MLX affine pack with numpy bit operations alone (field k of the row's u32
    stream, Quantize/WeightedAffineQuantizer.swift:142-153), in float64."""
    per = 32 // bits
    k = np.arange(K)
    q = (codes[:, k // per] >> np.uint32(bits) * (k % per).astype(np.uint32)) & np.uint32((1 << bits) - 1)
    return (np.repeat(s.astype(np.float64), group, 1) * q + np.repeat(b.astype(np.float64), group, 1))


@pytest.mark.parametrize("bits,group", [(2, 64), (2, 128), (4, 64), (4, 128), (8, 64), (8, 128)])
def test_affine_matmul_pinned(bits, group):
    """oracle.affine_matmul against x @ W.T in float64 with W rebuilt from the codes by numpy: each
    element within 1e-5 of sum |x||w| (the reference's per-element criterion,
    GGMLKernelTests.swift:131-137). A transposed operand, a wrong group index or a dropped bias
    each fail it."""
    from ishizuki_amd import synth
    N, K, M = 37, 1024, 5
    if bits == 2:
        codes, s, b = synth.affine_pack(N, K, group=group, seed=bits + group)
    else:
        codes, s, b = synth.affine_pack_bits(N, K, bits, group=group, seed=bits + group)
    # distinct biases (not just -s) so scale and bias cannot be confused
    b = (b.astype(np.float32) + np.float32(0.003) * np.arange(b.size).reshape(b.shape) % 7).astype(np.float16)
    x = np.random.default_rng(bits).standard_normal((M, K)).astype(np.float16).astype(np.float32)
    y = oracle.affine_matmul(x, codes, s.view(np.uint16), b.view(np.uint16), N, bits, group)
    W = _affine_dense(codes, s, b, K, bits, group)
    want = x.astype(np.float64) @ W.T
    bound = np.abs(x).astype(np.float64) @ np.abs(W).T
    assert np.all(np.abs(y - want) <= 1e-5 * bound + 1e-30)
    # and the dense weight itself bit-for-bit
    w32 = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, bits, group)
    assert np.array_equal(w32, W.astype(np.float32))


def _moe_loop_reference(x, logits, gate, up, down, t_, E, H, I, k, shared=None, shared_gate=None):
    """MoEBlockTests.reference (Tests/IshizukiKitTests/MoEBlockTests.swift:94-126) written out per
    token with numpy: softmax, top-k by sorting (ties to the lower index), renormalised weights,
    one SwiGLU per chosen expert with the fp16 activations of an fp16 model (each projection's
    output, sigmoid, silu and the product rounded to fp16), the weighted sum in fp32 in slot order,
    narrowed once. Weights from the golden-pinned dequantizer; dots in float64."""
    r16 = lambda a: np.asarray(a, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)
    Wg = oracle.dequant_rows(t_, gate, E * I, H).reshape(E, I, H).astype(np.float64)
    Wu = oracle.dequant_rows(t_, up, E * I, H).reshape(E, I, H).astype(np.float64)
    Wd = oracle.dequant_rows(t_, down, E * H, I).reshape(E, H, I).astype(np.float64)
    T = x.shape[0]
    y = np.zeros((T, H))
    bound = np.zeros((T, H))
    for t in range(T):
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        p /= p.sum()
        order = np.argsort(-logits[t], kind="stable")[:k]
        w = p[order] / p[order].sum()
        acc = np.zeros(H, np.float32)
        for s, e in enumerate(order):
            g = r16(Wg[e] @ x[t])
            u = r16(Wu[e] @ x[t])
            h = r16(r16(g * r16(1.0 / (1.0 + np.exp(-g)))) * u)
            o = r16(Wd[e] @ h)
            acc = (acc + (o * w[s]).astype(np.float32)).astype(np.float32)
            bound[t] += w[s] * (np.abs(Wd[e]) @ np.abs(h))
        if shared is not None:  # Text/MoEBlock.swift:158-160: sigmoid(gate) * shared in x.dtype, added in fp32
            term = r16(r16(1.0 / (1.0 + np.exp(-np.float64(shared_gate[t])))) * shared[t].astype(np.float64))
            acc = (acc + term.astype(np.float32)).astype(np.float32)
        y[t] = r16(acc)
    return y, bound, order


def test_moe_swiglu_pinned():
    """oracle.moe_swiglu against the loop-per-token reference above. An fp16 intermediate may round
    the other way when the two dot orders straddle a rounding boundary, so each element is held to
    one fp16 ulp of its down-projection terms (2^-10 * sum_s w_s |W_d||h_s|) plus the final
    narrowing (2^-11 |y|). A dropped slot, a wrong weight, a skipped renormalisation, gate and up
    swapped or silu applied to up all exceed it by orders of magnitude."""
    from ishizuki_amd import synth
    E, H, I, k, T, t_ = 16, 512, 256, 4, 3, 12
    gate = synth.ggml_blocks(t_, E * I, H, seed=1, scale=4e-4)
    up = synth.ggml_blocks(t_, E * I, H, seed=2, scale=4e-4)
    down = synth.ggml_blocks(t_, E * H, I, seed=3, scale=4e-4)
    x = synth.fp16_normal((T, H), seed=4).astype(np.float32)
    logits = np.random.default_rng(5).standard_normal((T, E)).astype(np.float32)
    ids, w = oracle.moe_route(logits, k)
    y = oracle.moe_swiglu(t_, x, ids, w, gate, up, down, E, I)
    want, bound, _ = _moe_loop_reference(x, logits, gate, up, down, t_, E, H, I, k)
    assert np.isfinite(want).all() and np.abs(want).max() > 1e-3
    err = np.abs(y - want)
    assert np.all(err <= 2.0 ** -10 * bound + 2.0 ** -11 * np.abs(want) + 2.0 ** -24), err.max()
    # the check has teeth: dropping the last slot is caught
    w2 = w.copy()
    w2[:, -1] = 0
    y2 = oracle.moe_swiglu(t_, x, ids, w2, gate, up, down, E, I)
    assert not np.all(np.abs(y2 - want) <= 2.0 ** -10 * bound + 2.0 ** -11 * np.abs(want) + 2.0 ** -24)


def test_moe_swiglu_shared_expert_pinned():
    """The shared-expert term (sigmoid of its gate logit, times its output, both fp16, added in
    fp32 before the one narrowing) against the loop reference; dropping the term or taking the
    gate's sigmoid with the wrong sign is caught."""
    from ishizuki_amd import synth
    E, H, I, k, T, t_ = 16, 512, 256, 4, 2, 12
    gate = synth.ggml_blocks(t_, E * I, H, seed=11, scale=4e-4)
    up = synth.ggml_blocks(t_, E * I, H, seed=12, scale=4e-4)
    down = synth.ggml_blocks(t_, E * H, I, seed=13, scale=4e-4)
    x = synth.fp16_normal((T, H), seed=14).astype(np.float32)
    logits = np.random.default_rng(15).standard_normal((T, E)).astype(np.float32)
    sh = (synth.fp16_normal((T, H), seed=16).astype(np.float32) * 0.05).astype(np.float16).astype(np.float32)
    sg = synth.fp16_normal((T,), seed=17).astype(np.float32)
    ids, w = oracle.moe_route(logits, k)
    y = oracle.moe_swiglu(t_, x, ids, w, gate, up, down, E, I, shared=sh, shared_gate=sg)
    want, bound, _ = _moe_loop_reference(x, logits, gate, up, down, t_, E, H, I, k, shared=sh, shared_gate=sg)
    tol = 2.0 ** -10 * bound + 2.0 ** -11 * np.abs(want) + 2.0 ** -24
    assert np.all(np.abs(y - want) <= tol)
    assert not np.all(np.abs(oracle.moe_swiglu(t_, x, ids, w, gate, up, down, E, I) - want) <= tol)
    assert not np.all(np.abs(oracle.moe_swiglu(t_, x, ids, w, gate, up, down, E, I, shared=sh, shared_gate=-sg)
                             - want) <= tol)


def test_cpu_baseline_matches_the_oracle():
    """bench.py's cpu_baseline leg (ishzo_bench_affine_linear): the dequantize-then-dot variant is
    the oracle's rotate + affine_matmul bit for bit; the fused decode-dot differs only in
    summation order."""
    import ctypes

    from ishizuki_amd import synth
    N, K = 96, 1024
    codes, s, b = synth.affine_pack(N, K, group=64, seed=2)
    x = synth.fp16_normal((1, K), seed=3)
    sg = synth.hadamard_signs(K, seed=4)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    L = oracle.lib()
    ys = []
    for variant in (0, 1):
        y = np.zeros(N, np.float32)
        t = L.ishzo_bench_affine_linear(P(x.view(np.uint16)), K, P(sg), 128, P(codes.view(np.uint32)),
                                        P(s.view(np.uint16)), P(b.view(np.uint16)), N, 64, variant, 3, 2, P(y))
        assert t > 0
        ys.append(y)
    xr = oracle.hadamard(x.astype(np.float32), 128, sg).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, 2, 64)
    assert np.array_equal(ys[0], ref[0])
    bound = np.abs(xr[0]) @ np.abs(oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, 2, 64)).T
    assert np.all(np.abs(ys[1] - ref[0]) <= 1e-5 * bound + 1e-6)
