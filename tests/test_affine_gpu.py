"""Affine 2-bit matmul and Hadamard rotation on the GPU vs the CPU oracle (through the C ABI).

Rotation: fp32 output within 1e-5 of the oracle's fp32 WHT (summation order differs); fp16 output
equal to the oracle rounded to fp16 except for rare one-ulp rounding-boundary cases.
Matmul: max |y - ref| <= 1e-3 * max |ref| with ref = the oracle's dequantize-then-fp32-dot of the
fp16-rounded rotated x (the reference casts the rotation back to x.dtype).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close
from ishizuki_amd import affine, synth


def affine_bound(xf, codes, s, b, N, K, bits, group):
    """|x| @ |W|.T for the per-element criterion (W from the oracle's affine dequantizer)."""
    W = oracle.affine_dequant(codes, np.asarray(s).view(np.uint16), np.asarray(b).view(np.uint16), N, K, bits, group)
    return np.abs(np.asarray(xf, np.float32)) @ np.abs(W).T


pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("block", [2, 8, 32, 64, 128, 512, 4096])
@pytest.mark.parametrize("inverse", [False, True])
def test_hadamard_fp32(block, inverse):
    x = np.random.default_rng(block).standard_normal((3, 8192)).astype(np.float32)
    s = synth.hadamard_signs(8192, seed=4)
    ref = oracle.hadamard(x, block, s, inverse=inverse)
    y = affine.hadamard_rotate(torch.from_numpy(x).to(DEV), block, torch.from_numpy(s), inverse).cpu().numpy()
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_hadamard_fp16_roundtrip():
    x = synth.fp16_normal((4, 5120), seed=1)
    xt = torch.from_numpy(x).to(DEV)
    y = affine.hadamard_rotate(xt, 128)
    ref = oracle.hadamard(x.astype(np.float32), 128).astype(np.float16)
    diff = np.abs(y.cpu().numpy().astype(np.float32) - ref.astype(np.float32))
    ulp = np.abs(ref.astype(np.float32)) * 2.0 ** -10 + 1e-7
    assert np.all(diff <= ulp)
    back = affine.hadamard_rotate(y, 128).cpu().numpy().astype(np.float32)  # H.H = I
    assert np.abs(back - x.astype(np.float32)).max() < 4e-3 * np.abs(x).max()


def affine_case(N, K, M, group, seed, block=0, signs_seed=None):
    codes, s, b = synth.affine_pack(N, K, group=group, seed=seed)
    x = synth.fp16_normal((M, K), seed=seed + 1)
    xf = x.astype(np.float32)
    signs = synth.hadamard_signs(K, seed=signs_seed) if block else None
    if block:
        xf = oracle.hadamard(xf, block, signs).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xf, codes, s.view(np.uint16), b.view(np.uint16), N, 2, group)
    dev = lambda a: torch.from_numpy(a).to(DEV)
    args = (dev(x), dev(codes.view(np.int32)), dev(s), dev(b))
    return args, signs, (ref, affine_bound(xf, codes, s, b, N, K, 2, group))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("group", [64, 128])
def test_affine_matmul(M, group):
    N, K = 1000, 2048
    (x, w, s, b), _, (ref, bd) = affine_case(N, K, M, group, seed=M)
    y = affine.quantized_matmul(x, w, s, b, group_size=group)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"affine M={M} g={group}")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("bits,group", [(2, 32), (4, 32), (8, 32), (3, 96), (2, 96)])
def test_affine_other_groups(bits, group, M, dt):
    """Groups other than 64 and 128 (applyAny accepts any multiple of 32 dividing K,
    Core/VerifyMatmul.swift:84): the exact-weight kernel, x in its own dtype, against the oracle."""
    N, K = 300, 3072
    codes, s, b = synth.affine_pack_bits(N, K, bits, group=group, seed=bits + group + M)
    x = torch.from_numpy(synth.fp16_normal((M, K), seed=M + 3)).to(dt)
    xf = x.float().numpy()
    print(f"affine group={group} bits={bits} M={M} {dt}", flush=True)
    y = affine.quantized_matmul(x.to(DEV), torch.from_numpy(codes.view(np.int32)).to(DEV), torch.from_numpy(s).to(DEV),
                                torch.from_numpy(b).to(DEV), group_size=group, bits=bits)
    assert y is not None and y.dtype == dt
    ref = oracle.affine_matmul(xf, codes, s.view(np.uint16), b.view(np.uint16), N, bits, group)
    bd = affine_bound(xf, codes, s, b, N, K, bits, group)
    # fp32 sums of exact weights: 1e-5 of the bound, plus the output's one rounding to x's dtype
    yv = y.float().cpu().numpy().astype(np.float64)
    lim = 1e-5 * bd + 2.0 ** (-11 if dt == torch.float16 else -8) * np.abs(ref)
    assert np.all(np.abs(yv - ref) <= lim), f"worst {np.max(np.abs(yv - ref) / lim):.3g}x"


@pytest.mark.parametrize("M", [1, 4])
def test_affine_group32_rotated_linear(M):
    """PackedLinear's rotated forward with group 32: x rotated once into the workspace (fp16, the
    reference's rounding), then the exact-weight kernel."""
    N, K, bits = 256, 2048, 2
    codes, s, b = synth.affine_pack(N, K, group=32, seed=M + 40)
    signs = synth.hadamard_signs(K, seed=41)
    x = synth.fp16_normal((M, K), seed=M + 42)
    y = affine.linear(torch.from_numpy(x).to(DEV), torch.from_numpy(codes.view(np.int32)).to(DEV),
                      torch.from_numpy(s).to(DEV), torch.from_numpy(b).to(DEV), signs=torch.from_numpy(signs),
                      block=128, group_size=32, bits=bits)
    assert y is not None
    xr = oracle.hadamard(x.astype(np.float32), 128, signs).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, bits, 32)
    assert_close(y.float().cpu().numpy(), ref, bound=affine_bound(xr, codes, s, b, N, K, bits, 32),
                 what=f"affine g32 rotated M={M}")


@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("block", [0, 128])
def test_affine_long_k_gemv(group, block):
    """K = 25600, M = 1: 400 units per row take 64 lanes per row and 1024-thread workgroups,
    whose sixteen waves stage (and rotate) x."""
    N, K = 200, 25600
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, 1, group, seed=41 + block, block=block, signs_seed=3)
    if block:
        y = affine.linear(x, w, s, b, signs=torch.from_numpy(signs), block=block, group_size=group)
    else:
        y = affine.quantized_matmul(x, w, s, b, group_size=group)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"affine long K g={group} block={block}")


@pytest.mark.parametrize("bits", [4, 3])
def test_affine_wide_bits_long_k_gemv(bits):
    N, K = 96, 25600
    codes, s, b = synth.affine_pack_bits(N, K, bits, group=64, seed=bits + 50)
    x = synth.fp16_normal((1, K), seed=bits + 51)
    xf = x.astype(np.float32)
    ref = oracle.affine_matmul(xf, codes, s.view(np.uint16), b.view(np.uint16), N, bits, 64)
    bd = affine_bound(xf, codes, s, b, N, K, bits, 64)
    dev = lambda a: torch.from_numpy(a).to(DEV)
    y = affine.quantized_matmul(dev(x), dev(codes.view(np.int32)), dev(s), dev(b), group_size=64, bits=bits)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"affine {bits}-bit long K")


@pytest.mark.parametrize("bits", [3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("M", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("group,bf16", [(64, False), (128, True)])
def test_affine_wide_bits(bits, M, group, bf16):
    """3- to 8-bit packs (VerifyMatmul.applyAny's 4- and 8-bit fast paths and its generic one for
    the other widths, Core/VerifyMatmul.swift:83-89, 273-290): the GEMV at M = 1, the streaming
    MFMA kernel above."""
    N, K = 1000, 1024
    codes, s, b = synth.affine_pack_bits(N, K, bits, group=group, seed=bits + M)
    x = synth.fp16_normal((M, K), seed=M + 40)
    ref = oracle.affine_matmul(x.astype(np.float32), codes, s.view(np.uint16), b.view(np.uint16), N, bits, group)
    bound = affine_bound(x, codes, s, b, N, K, bits, group)
    sd, bd = torch.from_numpy(s).to(DEV), torch.from_numpy(b).to(DEV)
    if bf16:  # bf16 scales and biases (the values rounded to bf16; the reference uses them as given)
        sd, bd = sd.to(torch.bfloat16), bd.to(torch.bfloat16)
        ref = _ref_bf16(x, codes, sd, bd, N, K, bits, group)
    y = affine.quantized_matmul(torch.from_numpy(x).to(DEV), torch.from_numpy(codes.view(np.int32)).to(DEV), sd, bd,
                                group_size=group, bits=bits)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bound, what=f"affine bits={bits} M={M} g={group} bf16={bf16}")


def _ref_bf16(x, codes, sd, bd, N, K, bits, group):
    """Reference with bf16 scales: dequantize through the oracle with unit scale / zero bias, then
    apply the bf16 values (exact in fp32)."""
    one = np.full((N, K // group), 0x3C00, np.uint16)  # the codes themselves: scale 1, bias 0
    q = oracle.affine_dequant(codes, one, np.zeros_like(one), N, K, bits, group)
    s = np.repeat(sd.float().cpu().numpy(), group, 1)
    b = np.repeat(bd.float().cpu().numpy(), group, 1)
    w = (s * q + b).astype(np.float32)
    return x.astype(np.float32) @ w.T


@pytest.mark.parametrize("bits,M", [(4, 1), (4, 8), (8, 3), (3, 1), (5, 8), (6, 2)])
def test_affine_wide_bits_rotated_linear(bits, M):
    """PackedLinear's rotated forward with a 3- to 8-bit pack: x rotated once, then the matmul."""
    N, K = 300, 1024
    codes, s, b = synth.affine_pack_bits(N, K, bits, group=64, seed=bits * 3 + M)
    x = synth.fp16_normal((M, K), seed=M + 50)
    signs = synth.hadamard_signs(K, seed=7)
    xr = oracle.hadamard(x.astype(np.float32), 128, signs).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, bits, 64)
    bound = affine_bound(xr, codes, s, b, N, K, bits, 64)
    y = affine.linear(torch.from_numpy(x).to(DEV), torch.from_numpy(codes.view(np.int32)).to(DEV),
                      torch.from_numpy(s).to(DEV), torch.from_numpy(b).to(DEV), signs=torch.from_numpy(signs),
                      block=128, group_size=64, bits=bits)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bound, what=f"affine linear bits={bits} M={M}")


@pytest.mark.parametrize("M", [5, 8, 16])
def test_affine_verify_very_wide_output(M):
    """40000 output rows (2500 tiles, more than 16 / NQ per CU): the verify kernel runs in several
    rounds of workgroups rather than declining (the vocabulary-head shape)."""
    N, K = 40000, 256
    (x, w, s, b), _, (ref, bd) = affine_case(N, K, M, 64, seed=M + 100)
    y = affine.quantized_matmul(x, w, s, b, group_size=64)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"affine wide N={N} M={M}")


@pytest.mark.parametrize("M", [1, 2, 8])
@pytest.mark.parametrize("signs_seed", [None, 7])
def test_affine_rotated_linear(M, signs_seed):
    N, K = 1088, 5120
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, M, 64, seed=20 + M, block=128, signs_seed=signs_seed)
    y = affine.linear(x, w, s, b, signs=torch.from_numpy(signs), block=128, group_size=64)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"rotated M={M}")


def _random_affine_cases(n, seed):
    """Seeded 2-bit shapes: N from 1 to 2499, K any multiple of 128 up to 8192, M from 1 to 8,
    groups of 64 and 128, unrotated or rotated in blocks of 64 or 128."""
    r = np.random.default_rng(seed)
    return [(int(r.integers(1, 2500)), 128 * int(r.integers(1, 65)), int(r.integers(1, 9)), (64, 128)[i % 2],
             (0, 64, 128)[i % 3]) for i in range(n)]


@pytest.mark.parametrize("N,K,M,group,block", _random_affine_cases(24, 2025))
def test_affine_random_shapes(N, K, M, group, block):
    print(f"affine random N={N} K={K} M={M} g={group} block={block}", flush=True)
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, M, group, seed=N + K, block=block, signs_seed=K)
    if block:
        y = affine.linear(x, w, s, b, signs=torch.from_numpy(signs), block=block, group_size=group)
    else:
        y = affine.quantized_matmul(x, w, s, b, group_size=group)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"affine random N={N} K={K} M={M} g={group} b={block}")


@pytest.mark.parametrize("block,K", [(b, K) for K in (1152, 5120) for b in (2, 32, 64, 128, 512) if K % b == 0])
@pytest.mark.parametrize("prestage", [True, False])
def test_affine_rotated_gemv_staging(block, prestage, K):
    """M = 1 with x staged by the prestage kernel or inside every workgroup; K = 1152 leaves a
    partial 512-value pass (rotation blocks that divide K only)."""
    N = 700
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, 1, 64, seed=block + K, block=block, signs_seed=3)
    y = affine.linear(x, w, s, b, signs=torch.from_numpy(signs), block=block, group_size=64, _prestage=prestage)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"gemv block={block} prestage={prestage} K={K}")


@pytest.mark.parametrize("M", [2, 5, 16])
@pytest.mark.parametrize("block", [2, 32, 128])
@pytest.mark.parametrize("K,prestage", [(1152, True), (5120, True), (5120, False)])
def test_affine_rotated_verify(M, block, K, prestage):
    """2..16 rows: x rotated and staged once by the prestage kernel, or the rotation fused into
    the verify kernel's staging (K % 256 == 0, block <= 128), else the rotation kernel into the
    workspace and the general verify kernel (K = 1152). M = 16 at K = 5120 stages x in two K
    chunks."""
    N = 530
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, M, 64, seed=M + block + K, block=block, signs_seed=5)
    y = affine.linear(x, w, s, b, signs=torch.from_numpy(signs), block=block, group_size=64, _prestage=prestage)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"verify M={M} block={block} K={K} prestage={prestage}")


@pytest.mark.parametrize("N,K,M,group", [(4352, 5120, 8, 64), (4352, 1024, 4, 64), (8320, 2304, 3, 128),
                                         (8320, 5120, 16, 64), (4100, 5120, 8, 64)])
def test_affine_verify_leftover_tiles(N, K, M, group):
    """More 16-row tiles than CUs but not a whole number per CU (4352 rows: 272 tiles on 256 CUs;
    4100 rows: a last tile of 4 rows), with x prestaged: several tiles per workgroup, uneven
    counts, group 128, and (M = 16 at K = 5120) x staged in K chunks. Two calls in a row give the
    same bits."""
    print(f"affine leftover N={N} K={K} M={M} g={group}", flush=True)
    (x, w, s, b), signs, (ref, bd) = affine_case(N, K, M, group, seed=N + K + M, block=128, signs_seed=9)
    sg = torch.from_numpy(signs)
    y1 = affine.linear(x, w, s, b, signs=sg, block=128, group_size=group)
    y2 = affine.linear(x, w, s, b, signs=sg, block=128, group_size=group)
    assert y1 is not None and y2 is not None
    assert_close(y1.float().cpu().numpy(), ref, bound=bd, what=f"leftover N={N} K={K} M={M}")
    assert torch.equal(y1, y2)


def test_affine_bf16_scales():
    N, K = 300, 1024
    codes, s, b = synth.affine_pack(N, K, group=64, seed=3)
    sb = torch.from_numpy(s.astype(np.float32)).to(torch.bfloat16)
    bb = torch.from_numpy(b.astype(np.float32)).to(torch.bfloat16)
    sf = sb.float().numpy().astype(np.float16)  # bf16 values are exact in fp32; oracle takes fp16
    x = synth.fp16_normal((1, K), seed=4)
    w = oracle.affine_dequant(codes, np.zeros_like(s).view(np.uint16), np.zeros_like(b).view(np.uint16), N, K, 2, 64)
    q = w  # all-zero scales/biases give zeros: rebuild from codes directly
    qv = np.stack([(codes[:, k // 16] >> np.uint32(2 * (k % 16))) & 3 for k in range(K)], 1).astype(np.float32)
    wf = np.repeat(sb.float().numpy(), 64, 1) * qv + np.repeat(bb.float().numpy(), 64, 1)
    ref = x.astype(np.float32) @ wf.T
    for M in (1, 4):
        xx = np.repeat(x, M, 0)
        y = affine.quantized_matmul(torch.from_numpy(xx).to(DEV), torch.from_numpy(codes.view(np.int32)).to(DEV),
                                    sb.to(DEV), bb.to(DEV), group_size=64)
        assert_close(y.float().cpu().numpy(), np.repeat(ref, M, 0), what=f"bf16 scales M={M}")


def test_affine_declines():
    x = torch.zeros((1, 256), dtype=torch.float16, device=DEV)
    w = torch.zeros((4, 16), dtype=torch.int32, device=DEV)
    s = torch.zeros((4, 8), dtype=torch.float16, device=DEV)
    assert affine.quantized_matmul(x, w, s, s, group_size=48) is None        # group not a multiple of 32
    assert affine.quantized_matmul(x.to(torch.int16), w, s, s, group_size=64) is None  # integer x
    assert affine.verify_apply(torch.zeros((1, 256), dtype=torch.float16, device=DEV), w, s, s) is None
