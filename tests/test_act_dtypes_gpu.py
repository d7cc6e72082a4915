"""bf16 and fp32 activations (the reference's matmuls are templated on the activation type,
Core/GGMLKernels.swift:196, Core/VerifyMatmul.swift:95-120, EXL3Kernels.apply rotating `to:
x.dtype`, Core/EXL3.swift:85-99): outputs in x's dtype, against the oracle fed the same values.

bf16 calls run the fp16 kernels on an fp16 image of x with a power-of-two factor per row. bf16
values land in it exactly (their 8 significant bits fit fp16's 11 at any scale within 2^-17 of
the row's largest), so a bf16 call is held to the fp16 call's per-element bound plus the bf16
output rounding (2^-9 relative, 2^-8 allowed). fp32 calls take the fp32 path (exact fp32
weights, fp32 FMAs) and are held to the reference's own fp32 criterion, 1e-5 of sum |x||w| per
element (Tests/IshizukiKitTests/GGMLKernelTests.swift:131-137). Rows far above fp16's range (1e6)
and far below it (1e-7) check the scaling."""
import numpy as np
import pytest
import torch

import oracle
from conftest import ggml_reference
from ishizuki_amd import affine, exl3, ggml, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bf16_round(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def activations(M, K, seed, dt):
    """M rows: N(0,1) values; with M >= 3, row 1 scaled to ~1e6 (beyond fp16) and row 2 to ~1e-7
    (below fp16's normal range), in dtype dt; returns (torch tensor on the GPU, fp32 values)."""
    x = np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)
    if M >= 3:
        x[1] *= 1.0e6
        x[2] *= 1.0e-7
    t = torch.from_numpy(x).to(dt)
    return t.to(DEV), t.float().numpy()


def check(y, ref, bound, dt, what):
    y = y.float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(y)), f"{what}: non-finite"
    if dt == torch.bfloat16:
        lim = 1e-4 * bound + 2.0 ** -8 * np.abs(ref) + 1e-30
    else:
        lim = 1e-5 * bound + 1e-30
    bad = np.abs(y - ref) > lim
    assert not bad.any(), f"{what}: {int(bad.sum())} outside; worst {np.max(np.abs(y - ref) / lim):.3g}x the bound"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("t", [ggml.Q4_0, ggml.Q4_K, ggml.IQ2_XS, ggml.IQ3_S])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_ggml_matvec_act_dtypes(dt, t, M):
    N, K = 300, 2048
    blocks = synth.ggml_blocks(t, N, K, seed=t + M)
    x, xf = activations(M, K, seed=M + 5, dt=dt)
    print(f"ggml act dtype={dt} t={t} M={M}", flush=True)
    y = ggml.matvec(x, torch.from_numpy(blocks).to(DEV), t, N)
    assert y is not None and y.dtype == dt
    ref, bd = ggml_reference(t, xf, blocks, N)
    check(y, ref, bd, dt, f"ggml t={t} M={M} {dt}")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits,M", [(2, 1), (2, 5), (4, 1), (4, 8), (3, 3)])
def test_affine_matmul_act_dtypes(dt, bits, M):
    N, K = 400, 1024
    if bits == 2:
        codes, s, b = synth.affine_pack(N, K, group=64, seed=bits + M)
    else:
        codes, s, b = synth.affine_pack_bits(N, K, bits, group=64, seed=bits + M)
    x, xf = activations(M, K, seed=M + 6, dt=dt)
    print(f"affine act dtype={dt} bits={bits} M={M}", flush=True)
    y = affine.quantized_matmul(x, torch.from_numpy(codes.view(np.int32)).to(DEV), torch.from_numpy(s).to(DEV),
                                torch.from_numpy(b).to(DEV), group_size=64, bits=bits)
    assert y is not None and y.dtype == dt
    ref = oracle.affine_matmul(xf, codes, s.view(np.uint16), b.view(np.uint16), N, bits, 64)
    W = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, bits, 64)
    check(y, ref, np.abs(xf) @ np.abs(W).T, dt, f"affine bits={bits} M={M} {dt}")


@pytest.mark.parametrize("M", [1, 4])
def test_affine_rotated_linear_bf16(M):
    """PackedLinear's rotated forward with bf16 activations: hadamardRotate in bf16 (the rotated
    activation the reference multiplies is x.dtype), then the product."""
    N, K = 300, 1024
    codes, s, b = synth.affine_pack(N, K, group=64, seed=M + 60)
    signs = synth.hadamard_signs(K, seed=9)
    x, xf = activations(M, K, seed=M + 61, dt=torch.bfloat16)
    y = affine.linear(x, torch.from_numpy(codes.view(np.int32)).to(DEV), torch.from_numpy(s).to(DEV),
                      torch.from_numpy(b).to(DEV), signs=torch.from_numpy(signs), block=128, group_size=64, bits=2)
    assert y is not None and y.dtype == torch.bfloat16
    xr = bf16_round(oracle.hadamard(xf, 128, signs))
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, 2, 64)
    W = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, 2, 64)
    # one bf16 rounding of a rotated value may go the other way (fp32 butterfly order): 2^-8 of it
    check(y, ref, (np.abs(xr) @ np.abs(W).T) * 40, torch.bfloat16, f"affine linear bf16 M={M}")


@pytest.mark.parametrize("M", [1, 3])
def test_exl3_apply_bf16(M):
    """EXL3Kernels.apply with bf16 x: rotated into bf16, the product in fp32, the output rotated
    into bf16 (Core/EXL3.swift:82-100)."""
    K, N, bits2 = 1024, 512, 4
    tr, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=M + 70)
    tt = exl3.EXL3Tensor(torch.from_numpy(tr).to(DEV), torch.from_numpy(suh).to(DEV), torch.from_numpy(svh).to(DEV))
    x, xf = activations(M, K, seed=M + 71, dt=torch.bfloat16)
    y = exl3.apply(x, tt)
    assert y is not None and y.dtype == torch.bfloat16
    W = oracle.exl3_dequant(tr, bits2, 0)
    xr = bf16_round(oracle.hadamard(xf * suh.astype(np.float32), 128))
    yh = xr.astype(np.float64) @ W
    ref = oracle.hadamard(yh.astype(np.float32), 128) * svh.astype(np.float32)
    # an output of the output rotation is +-1/sqrt(128) times each of its block's 128 products,
    # times svh: bound it by the magnitudes forming those products
    bh = np.abs(xr).astype(np.float64) @ np.abs(W)
    blk = np.repeat(bh.reshape(M, N // 128, 128).sum(2), 128, 1)
    bound = blk / np.sqrt(128.0) * np.abs(svh.astype(np.float64))
    check(y, ref, bound * 40, torch.bfloat16, f"exl3 bf16 M={M}")


def test_bf16_row_near_float_max():
    """A bf16 row whose largest value lies just below FLT_MAX (beyond 2^127): the image's row
    factor stays a finite 2^127, so finite inputs give finite outputs."""
    N, K, t = 256, 1024, ggml.Q4_K
    blocks = synth.ggml_blocks(t, N, K, seed=80, scale=1e-6)
    x = np.random.default_rng(81).standard_normal((2, K)).astype(np.float32)
    x[1] *= 1e-3
    x[1, 7] = 3.3e38  # bf16 rounds this to 3.3e38 (2^127 < 3.3e38 < FLT_MAX)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    xf = xb.float().numpy()
    y = ggml.matvec(xb.to(DEV), torch.from_numpy(blocks).to(DEV), t, N)
    assert y is not None
    ref, bd = ggml_reference(t, xf.astype(np.float64), blocks, N)
    yf = y.float().cpu().numpy()
    fin = np.isfinite(ref.astype(np.float32)) & (np.abs(ref) < 3.0e38)
    assert np.all(np.isfinite(yf[fin])), "finite inputs gave non-finite outputs"
    check(torch.from_numpy(yf[fin]), ref[fin], bd[fin], torch.bfloat16, "bf16 row near FLT_MAX")


@pytest.mark.parametrize("bits2,cb", [(4, 0), (2, 0), (3, 2), (8, 1)])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_exl3_matvec_fp32(bits2, cb, M):
    """EXL3Kernels.matvec with fp32 x against the expanded weight, within 1e-5 of the largest
    sum |x||w| (Tests/IshizukiKitTests/EXL3Tests.swift:57-72)."""
    K, N = 1024, 512
    tr, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=M + 90 + bits2)
    tt = exl3.EXL3Tensor(torch.from_numpy(tr).to(DEV), torch.from_numpy(suh).to(DEV), torch.from_numpy(svh).to(DEV),
                         codebook=cb)
    x = np.random.default_rng(M + 91).standard_normal((M, K)).astype(np.float32)
    print(f"exl3 matvec fp32 bits2={bits2} cb={cb} M={M}", flush=True)
    y = exl3.matvec(torch.from_numpy(x).to(DEV), tt)
    assert y is not None
    W = oracle.exl3_dequant(tr, bits2, cb).astype(np.float64)
    ref = x.astype(np.float64) @ W
    bound = (np.abs(x).astype(np.float64) @ np.abs(W)).max()
    worst = np.abs(y.cpu().numpy().astype(np.float64) - ref).max() / bound
    assert worst < 1e-5, f"worst {worst}"


@pytest.mark.parametrize("M", [1, 3])
def test_exl3_apply_fp32(M):
    """EXL3Kernels.apply with fp32 x: rotated in fp32, the fp32 product, the output rotated in
    fp32 (Core/EXL3.swift:82-100), per element within 1e-5 of its bound."""
    K, N, bits2 = 1024, 512, 4
    tr, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=M + 72)
    tt = exl3.EXL3Tensor(torch.from_numpy(tr).to(DEV), torch.from_numpy(suh).to(DEV), torch.from_numpy(svh).to(DEV))
    x, xf = activations(M, K, seed=M + 73, dt=torch.float32)
    y = exl3.apply(x, tt)
    assert y is not None and y.dtype == torch.float32
    W = oracle.exl3_dequant(tr, bits2, 0).astype(np.float64)
    xr = oracle.hadamard(xf * suh.astype(np.float32), 128).astype(np.float64)
    yh = xr @ W
    ref = oracle.hadamard(yh.astype(np.float32), 128).astype(np.float64) * svh.astype(np.float64)
    bh = np.abs(xr) @ np.abs(W)
    blk = np.repeat(bh.reshape(M, N // 128, 128).sum(2), 128, 1)
    bound = blk / np.sqrt(128.0) * np.abs(svh.astype(np.float64))
    check(y, ref, bound, torch.float32, f"exl3 fp32 M={M}")


@pytest.mark.parametrize("bits,M", [(2, 1), (2, 4), (4, 3)])
def test_affine_rotated_linear_fp32(bits, M):
    """PackedLinear's rotated forward with fp32 x: hadamardRotate in fp32, then the fp32 product."""
    N, K = 300, 1024
    if bits == 2:
        codes, s, b = synth.affine_pack(N, K, group=64, seed=M + 62)
    else:
        codes, s, b = synth.affine_pack_bits(N, K, bits, group=64, seed=M + 62)
    signs = synth.hadamard_signs(K, seed=10)
    x, xf = activations(M, K, seed=M + 63, dt=torch.float32)
    y = affine.linear(x, torch.from_numpy(codes.view(np.int32)).to(DEV), torch.from_numpy(s).to(DEV),
                      torch.from_numpy(b).to(DEV), signs=torch.from_numpy(signs), block=128, group_size=64, bits=bits)
    assert y is not None and y.dtype == torch.float32
    xr = oracle.hadamard(xf, 128, signs)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, bits, 64)
    W = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, bits, 64)
    check(y, ref, np.abs(xr) @ np.abs(W).T, torch.float32, f"affine linear fp32 bits={bits} M={M}")
