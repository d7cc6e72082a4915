"""Every BASELINE configuration at its full shape on the GPU against the oracle, through the C ABI.

Each output is held to both criteria of `assert_close`: max |y - ref| <= 1e-3 * max |ref|
(BASELINE's bar on fp16 outputs) and, per element, |y - ref| <= 1e-4 * sum|x||w| plus half an fp16
ulp (the reference's own per-element yardstick, Tests/IshizukiKitTests/GGMLKernelTests.swift:131-137).
The shapes are the ones the bench times, so every timed kernel instantiation is also checked:
  configs[0]  Q4_0 4096x4096, M = 1 (and 8)
  configs[1]  affine 2-bit g64 + 128-point rotation, 17408x5120, M in {1, 2, 4, 8}
  configs[2]  Q4_K / Q6_K / IQ2_XS at 25600x5120 (gate/up) and 5120x25600 (down), M in {1, 8};
              the down projection's M = 1 GEMV has 400 units per row (64 lanes per row, ragged)
  configs[3]  EXL3 2 bpw 5120 -> 17408, M in {1, 2, 4, 8}
  north-star  Q4_0 / Q4_K / Q6_K / IQ2_XS at 17408x5120, M in {1, 8}
(configs[4], the MoE FFN at T = 1, 8 and 64, is in test_moe_gpu.py.)
Synthetic data follow the configs' distributions (ishizuki_amd.synth).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close, ggml_reference
from ishizuki_amd import affine, exl3, ggml, synth
from test_exl3_gpu import APPLY_ELEM, apply_reference

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ggml_case(t, N, K, Ms, seed):
    blk = synth.ggml_blocks(t, N, K, seed=seed)
    wb = torch.from_numpy(blk).to(DEV)
    x = synth.fp16_normal((max(Ms), K), seed=seed + 1)
    ref, bound = ggml_reference(t, x, blk, N)
    for M in Ms:
        print(f"config ggml type={t} N={N} K={K} M={M}", flush=True)
        y = ggml.matvec(torch.from_numpy(x[:M]).to(DEV), wb, t, N)
        assert y is not None, "declined"
        assert_close(y.float().cpu().numpy(), ref[:M], bound=bound[:M], what=f"type={t} {N}x{K} M={M}")


def test_config0_q4_0_4096():
    _ggml_case(ggml.Q4_0, 4096, 4096, (1, 8), seed=0x15A12)


@pytest.mark.parametrize("t", [ggml.Q4_K, ggml.Q6_K, ggml.IQ2_XS])
@pytest.mark.parametrize("N,K", [(25600, 5120), (5120, 25600)])
def test_config2_qwen_mlp(t, N, K):
    _ggml_case(t, N, K, (1, 8), seed=0x15A14 + t + K)


@pytest.mark.parametrize("t", [ggml.Q4_0, ggml.Q4_K, ggml.Q6_K, ggml.IQ2_XS])
def test_north_star_17408x5120(t):
    _ggml_case(t, 17408, 5120, (1, 8), seed=0x15A20 + t)


def test_config1_affine_rotated():
    N, K, g = 17408, 5120, 64
    codes, s, b = synth.affine_pack(N, K, group=g, seed=0x15A13)
    signs = synth.hadamard_signs(K, seed=0x15A13)
    x = synth.fp16_normal((8, K), seed=0x15A13 + 1)
    xr = oracle.hadamard(x.astype(np.float32), 128, signs).astype(np.float16).astype(np.float32)
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, 2, g)
    W = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, 2, g)
    np.abs(W, out=W)
    bound = np.abs(xr) @ W.T
    del W
    wd = torch.from_numpy(codes.view(np.int32)).to(DEV)
    sd, bd = torch.from_numpy(s).to(DEV), torch.from_numpy(b).to(DEV)
    for M in (1, 2, 4, 8):
        print(f"config affine M={M}", flush=True)
        y = affine.linear(torch.from_numpy(x[:M]).to(DEV), wd, sd, bd, signs=torch.from_numpy(signs), block=128,
                          group_size=g)
        assert y is not None
        assert_close(y.float().cpu().numpy(), ref[:M], bound=bound[:M], what=f"affine 17408x5120 M={M}")


def test_config3_exl3_2bpw():
    K, N = 5120, 17408
    t, suh, svh = synth.exl3_pack(K, N, bits2=4, seed=0x15A15)
    ten = exl3.EXL3Tensor(torch.from_numpy(t).to(DEV), torch.from_numpy(suh).to(DEV), torch.from_numpy(svh).to(DEV),
                          codebook=exl3.THREE_INST)
    x = synth.fp16_normal((8, K), seed=0x15A15 + 1)
    ref, bound = apply_reference(x, t, suh, svh, 4, 0)
    for M in (1, 2, 4, 8):
        print(f"config exl3 M={M}", flush=True)
        y = exl3.apply(torch.from_numpy(x[:M]).to(DEV), ten)
        assert y is not None
        assert_close(y.float().cpu().numpy(), ref[:M], bound=bound[:M], elem=APPLY_ELEM, what=f"exl3 5120->17408 M={M}")



def _properties(f, x1, x2, bound_of, rel, what, exact_scale=True):
    """Size-independent checks of a linear map at full size, no oracle product needed: doubling x
    doubles y, and y(x1 + x2) = y(x1) + y(x2) within rel of the two products' per-element bounds
    plus the fp16 roundings of the three outputs. exact_scale: scaling by 2 is exact through every
    fp16 rounding and fp32 sum on the path (2^-22 absolute slack for subnormals); otherwise the
    doubling is held to the same tolerance as the sum."""
    y1, y2 = f(x1).float(), f(x2).float()
    yd = f(x1 * 2).float()
    y1n, y2n = y1.cpu().numpy(), y2.cpu().numpy()
    if exact_scale:
        assert (yd - 2 * y1).abs().max().item() <= 2.0 ** -22, f"{what}: y(2x) != 2 y(x)"
    else:
        err2 = np.abs(yd.cpu().numpy() - 2 * y1n)
        assert np.all(err2 <= rel * 2 * bound_of(x1) + 2.0 ** -9 * 2 * np.abs(y1n) + 1e-6), f"{what}: y(2x) != 2 y(x)"
    ys = f(x1 + x2).float()
    err = np.abs(ys.cpu().numpy() - (y1n + y2n))
    tol = rel * (bound_of(x1) + bound_of(x2)) + 2.0 ** -9 * (np.abs(y1n) + np.abs(y2n)) + 1e-6
    assert np.all(err <= tol), f"{what}: not additive (worst {np.max(err / tol):.2f} of the tolerance)"


@pytest.mark.parametrize("t", [ggml.Q4_K, ggml.IQ2_XS])
@pytest.mark.parametrize("M", [1, 8])
def test_north_star_linearity(t, M):
    N, K = 17408, 5120
    blk = synth.ggml_blocks(t, N, K, seed=77)
    wb = torch.from_numpy(blk).to(DEV)
    w_abs_t = np.abs(oracle.dequant_rows(t, blk, N, K)).T.copy()
    x1 = torch.from_numpy(synth.fp16_normal((M, K), seed=78)).to(DEV)
    x2 = torch.from_numpy(synth.fp16_normal((M, K), seed=79)).to(DEV)
    bound_of = lambda x: np.abs(x.float().cpu().numpy()) @ w_abs_t
    print(f"linearity ggml type={t} M={M}", flush=True)
    # fp32 sums in another order and the fp16 output: 2e-4 of sum |x||w|
    _properties(lambda x: ggml.matvec(x, wb, t, N), x1, x2, bound_of, 2e-4, f"type={t} M={M}")


@pytest.mark.parametrize("M", [1, 8])
def test_config1_affine_linearity(M):
    N, K = 17408, 5120
    codes, sc, bi = synth.affine_pack(N, K, group=64, seed=80)
    signs = synth.hadamard_signs(K, seed=81)
    w_abs_t = np.abs(oracle.affine_dequant(codes, sc.view(np.uint16), bi.view(np.uint16), N, K, 2, 64)).T.copy()
    wd, sd, bd = (torch.from_numpy(a).to(DEV) for a in (codes.view(np.int32), sc, bi))
    x1 = torch.from_numpy(synth.fp16_normal((M, K), seed=82)).to(DEV)
    x2 = torch.from_numpy(synth.fp16_normal((M, K), seed=83)).to(DEV)
    rot = lambda x: oracle.hadamard(x.float().cpu().numpy(), 128, signs)
    bound_of = lambda x: np.abs(rot(x)) @ w_abs_t
    print(f"linearity affine M={M}", flush=True)
    # each rotated x is rounded to fp16 on its own (three roundings of up to 2^-11): 2e-3 of the
    # bound; the image holds x / 4^i (i < 5), subnormal for the smallest x, so doubling is exact
    # only to that tolerance
    _properties(lambda x: affine.linear(x, wd, sd, bd, signs=torch.from_numpy(signs), block=128, group_size=64),
                x1, x2, bound_of, 2e-3, f"affine M={M}", exact_scale=False)


@pytest.mark.parametrize("t", [ggml.Q4_K, ggml.Q6_K])
def test_north_star_fp32(t):
    """fp32 activations at the north-star shape: the exact-weight fp32 path against the oracle's
    dequantize-then-fp32-dot, per element within 1e-5 of sum |x||w| (the reference's fp32
    criterion, GGMLKernelTests.swift:131-137), M = 1 and 8."""
    N, K = 17408, 5120
    blk = synth.ggml_blocks(t, N, K, seed=90 + t)
    x = np.random.default_rng(91).standard_normal((8, K)).astype(np.float32)
    ref, bound = ggml_reference(t, x, blk, N)
    wb = torch.from_numpy(blk).to(DEV)
    for M in (1, 8):
        print(f"north-star fp32 type={t} M={M}", flush=True)
        y = ggml.matvec(torch.from_numpy(x[:M]).to(DEV), wb, t, N)
        assert y is not None and y.dtype == torch.float32
        err = np.abs(y.cpu().numpy().astype(np.float64) - ref[:M])
        assert np.all(err <= 1e-5 * bound[:M]), f"worst {np.max(err / (1e-5 * bound[:M])):.3g}x"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_config1_affine_rotated_act_dtypes(dt):
    """BASELINE configs[1] (17408x5120, g64, 128-point rotation) with bf16 and fp32 activations,
    M = 1 and 8: rotated in x's dtype, then the product (fp32: exact weights, 1e-5 of the bound;
    bf16: the fp16 kernels' bound plus bf16's own roundings of x, the rotation and y)."""
    N, K = 17408, 5120
    codes, s, b = synth.affine_pack(N, K, group=64, seed=0xA1)
    signs = synth.hadamard_signs(K, seed=0xA2)
    xt = torch.from_numpy(np.random.default_rng(0xA3).standard_normal((8, K)).astype(np.float32)).to(dt)
    xf = xt.float().numpy()
    xr = oracle.hadamard(xf, 128, signs)
    if dt == torch.bfloat16:
        xr = torch.from_numpy(xr).to(torch.bfloat16).float().numpy()
    ref = oracle.affine_matmul(xr, codes, s.view(np.uint16), b.view(np.uint16), N, 2, 64)
    W = oracle.affine_dequant(codes, s.view(np.uint16), b.view(np.uint16), N, K, 2, 64)
    bound = np.abs(xr) @ np.abs(W).T
    args = [torch.from_numpy(a).to(DEV) for a in (codes.view(np.int32), s, b)]
    for M in (1, 8):
        print(f"config1 {dt} M={M}", flush=True)
        y = affine.linear(xt[:M].to(DEV), *args, signs=torch.from_numpy(signs), block=128, group_size=64, bits=2)
        assert y is not None and y.dtype == dt
        yv = y.float().cpu().numpy().astype(np.float64)
        if dt == torch.float32:
            lim = 1e-5 * bound[:M]
        else:  # a rotated value's bf16 rounding may go the other way (fp32 butterfly order): 40x slack
            lim = 40 * 1e-4 * bound[:M] + 2.0 ** -8 * np.abs(ref[:M])
        assert np.all(np.abs(yv - ref[:M]) <= lim), f"{dt} M={M}: worst {np.max(np.abs(yv - ref[:M]) / lim):.3g}x"
