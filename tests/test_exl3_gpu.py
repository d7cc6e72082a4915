"""EXL3 on the GPU vs the oracle and exllamav3's golden reconstructions (through the C ABI).

Dequant: bit-exact against exl3_reference.npz (11 rate/codebook cases, EXL3Tests.swift:44-55).
Matvec: max |y - ref| <= 1e-3 * max|ref| against the oracle's fp32 product with the decoded W
(the reference's own check is 1e-5 of the |x||W| bound in fp32, EXL3Tests.swift:57-72; ours are
fp16 activations with fp32 accumulation in a different order).
Apply: the full rotate -> matvec -> rotate path vs the oracle restatement, 1e-3 of max|ref|.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close, bits_equal
from ishizuki_amd import _lib, exl3, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
# apply: the rotated x is fp16, and a value on a rounding boundary may land one ulp apart between
# two fp32 butterfly orders, which moves an output by at most 2^-11 of its bound
APPLY_ELEM = 1e-4 + 2.0 ** -11


def apply_reference(x, t, suh, svh, bits2, cb):
    """(ref, bound) for EXL3Kernels.apply: the oracle's rotate -> product -> rotate, and the
    per-element bound carried through both rotations: |xh| @ |W| for yh, then each output takes
    1/sqrt(128) of its 128-block's yh bounds times |svh|."""
    x = np.asarray(x, np.float32)
    suh = np.asarray(suh, np.float32)
    svh = np.asarray(svh, np.float32)
    ref = oracle.exl3_apply(x, t, suh, svh, bits2, cb)
    xh = oracle.hadamard(x, 128, suh).astype(np.float16).astype(np.float32)
    bh = np.abs(xh) @ np.abs(oracle.exl3_dequant(t, bits2, cb))
    M, N = bh.shape
    blk = bh.reshape(M, N // 128, 128).sum(2, keepdims=True) / np.sqrt(128.0)
    bound = np.broadcast_to(blk, (M, N // 128, 128)).reshape(M, N) * np.abs(svh)
    return ref, bound
CASES = [("r1c0", 0), ("r2c1", 1), ("r3c2", 2), ("r4c0", 0), ("r5c2", 2), ("r6c1", 1),
         ("r7c2", 2), ("r8c0", 0), ("r1h5c2", 2), ("r2h5c2", 2), ("r3h5c2", 2)]


@pytest.mark.parametrize("name,cb", CASES)
def test_dequant_matches_exllamav3(golden_exl3, name, cb):
    t = golden_exl3[name + ".trellis"]
    K, N = t.shape[0] * 16, t.shape[1] * 16
    out = torch.empty((K, N), dtype=torch.float32, device=DEV)
    from ishizuki_amd._torch import ptr
    rc = _lib.lib().ishz_exl3_dequant(ptr(torch.from_numpy(t).to(DEV)), K, N, t.shape[2] // 8, cb, ptr(out),
                                      _lib.DT_F32, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert bits_equal(out.cpu().numpy(), golden_exl3[name + ".expected"])


def make(K, N, bits2, cb, seed):
    t, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=seed)
    ten = exl3.EXL3Tensor(torch.from_numpy(t).to(DEV), torch.from_numpy(suh).to(DEV),
                          torch.from_numpy(svh).to(DEV), codebook=cb)
    return t, suh, svh, ten


@pytest.mark.parametrize("bits2,cb", [(4, 0), (4, 1), (4, 2), (2, 0), (3, 2), (8, 0), (16, 1), (7, 2)])
def test_dequant_random_rates(bits2, cb):
    t, _, _, ten = make(256, 384, bits2, cb, seed=bits2 * 3 + cb)
    w = exl3.dequantize(ten, torch.float32).cpu().numpy()
    assert bits_equal(w, oracle.exl3_dequant(t, bits2, cb))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 8, 16])
@pytest.mark.parametrize("bits2,cb", [(4, 0), (4, 2), (3, 2), (6, 1), (2, 0), (2, 2), (8, 1), (10, 0)])
def test_matvec(M, bits2, cb):
    K, N = 1024, 512
    t, _, _, ten = make(K, N, bits2, cb, seed=M + bits2)
    w = oracle.exl3_dequant(t, bits2, cb)
    xh = synth.fp16_normal((M, K), seed=M)
    ref = xh.astype(np.float32) @ w
    bd = np.abs(xh.astype(np.float32)) @ np.abs(w)
    y = exl3.matvec(torch.from_numpy(xh).to(DEV), ten)
    assert y is not None
    assert_close(y.cpu().numpy(), ref, bound=bd, what=f"exl3 matvec M={M} bits2={bits2} cb={cb}")


@pytest.mark.parametrize("M", [1, 5])
def test_matvec_is_deterministic(M):
    """K split over many workgroups (K = 5120, N = 1024: dozens of parts): the parts are summed in
    split order, so repeated calls give the same bits; the result matches the oracle."""
    K, N = 5120, 1024
    t, _, _, ten = make(K, N, 4, 0, seed=70 + M)
    xh = torch.from_numpy(synth.fp16_normal((M, K), seed=71 + M)).to(DEV)
    ys = [exl3.matvec(xh, ten) for _ in range(3)]
    for y in ys[1:]:
        assert torch.equal(y.view(torch.int32), ys[0].view(torch.int32))
    w = oracle.exl3_dequant(t, 4, 0)
    xf = xh.float().cpu().numpy()
    assert_close(ys[0].cpu().numpy(), xf @ w, bound=np.abs(xf) @ np.abs(w), what=f"exl3 deterministic M={M}")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 5])
def test_matvec_workspace_matches_temporaries(M, dt):
    """ishz_exl3_matvec_ws (caller workspace, no allocation) gives the bits of ishz_exl3_matvec
    (stream-ordered temporaries); a workspace one byte short is refused."""
    K, N = 5120, 1024
    t, _, _, ten = make(K, N, 4, 0, seed=80 + M)
    xh = torch.from_numpy(synth.fp16_normal((M, K), seed=81 + M)).to(DEV).to(dt)
    nb = exl3.matvec_workspace_size(M, ten)
    ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
    y0 = exl3.matvec(xh, ten)
    y1 = exl3.matvec(xh, ten, workspace=ws)
    assert y0 is not None and y1 is not None
    assert torch.equal(y0.view(torch.int32), y1.view(torch.int32))
    with pytest.raises(_lib.IshzError):
        exl3.matvec(xh, ten, workspace=ws[: nb - 1])


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("bits2,N", [(2, 384), (4, 384), (2, 640), (8, 128)])
def test_matvec_n_not_a_multiple_of_the_wide_step(M, bits2, N):
    """The wide-step kernel covers 32 / bits column tiles per step (512 columns at 1 bpw, 256 at
    2 bpw): other N take the general kernel, and every column is computed."""
    K = 512
    t, _, _, ten = make(K, N, bits2, 0, seed=N + bits2 + M)
    xh = synth.fp16_normal((M, K), seed=M)
    w = oracle.exl3_dequant(t, bits2, 0)
    ref = xh.astype(np.float32) @ w
    bd = np.abs(xh.astype(np.float32)) @ np.abs(w)
    y = exl3.matvec(torch.from_numpy(xh).to(DEV), ten)
    assert y is not None
    assert_close(y.cpu().numpy(), ref, bound=bd, what=f"exl3 matvec bits2={bits2} N={N} M={M}")


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("bits2,N", [(2, 640), (4, 1024)])
def test_apply_split_partials(M, bits2, N):
    """apply sums the matvec's K-split partial slices in the output rotation; K = 5120 gives
    several splits."""
    K = 5120
    t, suh, svh, ten = make(K, N, bits2, 0, seed=M + N)
    x = synth.fp16_normal((M, K), seed=M + 3)
    ref, bd = apply_reference(x, t, suh, svh, bits2, 0)
    y = exl3.apply(torch.from_numpy(x).to(DEV), ten)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=APPLY_ELEM, what=f"exl3 apply split bits2={bits2} N={N} M={M}")


@pytest.mark.parametrize("M", [1, 4, 8])
def test_apply_matches_oracle(M):
    K, N = 5120, 1024
    t, suh, svh, ten = make(K, N, 4, 0, seed=40 + M)
    x = synth.fp16_normal((M, K), seed=M + 100)
    ref, bd = apply_reference(x, t, suh, svh, 4, 0)
    y = exl3.apply(torch.from_numpy(x).to(DEV), ten)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=APPLY_ELEM, what=f"exl3 apply M={M}")


def _random_apply_cases(n, seed):
    """Seeded shapes for the full apply: K and N any multiple of 128 up to 3072 (both sides are
    rotated in 128-blocks), M from 1 to 8, bits2 (twice the rate) 2 to 8 over the three codebooks
    (half-integer rates take the MUL1 codebook, the only one defined for them)."""
    r = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        K, N, M = 128 * int(r.integers(1, 25)), 128 * int(r.integers(1, 25)), int(r.integers(1, 9))
        bits2 = (2, 3, 4, 5, 6, 8)[int(r.integers(0, 6))]
        cases.append((K, N, M, bits2, 2 if bits2 % 2 else i % 3))
    return cases


@pytest.mark.parametrize("K,N,M,bits2,cb", _random_apply_cases(24, 2026))
def test_apply_random_shapes(K, N, M, bits2, cb):
    print(f"exl3 random apply K={K} N={N} M={M} bits2={bits2} cb={cb}", flush=True)
    t, suh, svh, ten = make(K, N, bits2, cb, seed=K + N + M)
    x = synth.fp16_normal((M, K), seed=K + M)
    ref, bd = apply_reference(x, t, suh, svh, bits2, cb)
    y = exl3.apply(torch.from_numpy(x).to(DEV), ten)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=APPLY_ELEM,
                 what=f"exl3 random apply K={K} N={N} M={M} bits2={bits2} cb={cb}")


@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("K", [128, 1152, 5120])
@pytest.mark.parametrize("bits2,cb", [(2, 0), (4, 1), (8, 2), (4, 0)])
def test_apply_fused_input_rotation(M, K, bits2, cb):
    """N a whole number of wide steps: at M = 1 the matvec rotates x itself (every workgroup the
    128-blocks of its K range; K ranges that start and end inside a block at K = 1152), no
    rotation launch; M = 3 and 16 take the rotation kernel into the workspace at the same shapes."""
    N = 512
    t, suh, svh, ten = make(K, N, bits2, cb, seed=K + bits2 + cb)
    x = synth.fp16_normal((M, K), seed=K + 7 + M)
    ref, bd = apply_reference(x, t, suh, svh, bits2, cb)
    y = exl3.apply(torch.from_numpy(x).to(DEV), ten)
    assert y is not None
    assert_close(y.float().cpu().numpy(), ref, bound=bd, elem=APPLY_ELEM, what=f"exl3 apply fused rotation M={M} K={K} bits2={bits2} cb={cb}")


@pytest.mark.parametrize("name,cb", [("qwen3", 0), ("qwen38", 2)])
def test_projection_reproduces_checkpoint(golden_exl3, name, cb):
    # EXL3Tests.projectionMatchesCheckpoint (:74-98): rel-L2 < 0.12 against the fp16 checkpoint.
    t = torch.from_numpy(golden_exl3[name + ".trellis"]).to(DEV)
    ten = exl3.EXL3Tensor(t, torch.from_numpy(golden_exl3[name + ".suh"]).to(DEV),
                          torch.from_numpy(golden_exl3[name + ".svh"]).to(DEV), codebook=cb)
    ref_w = golden_exl3[name + ".weight"].astype(np.float32)
    x = np.random.default_rng(3).standard_normal((16, 128)).astype(np.float16)
    prev = None
    for rows in (1, 5, 12, 16):
        y = exl3.apply(torch.from_numpy(x[:rows]).to(DEV), ten).float().cpu().numpy()
        want = x[:rows].astype(np.float32) @ ref_w
        err = np.sqrt(((y - want) ** 2).sum() / (want ** 2).sum())
        assert err < 0.12, (rows, err)
        if prev is not None:
            assert np.abs(y[0] - prev[0]).max() < 2e-2
        prev = y


def test_tensor_validation():
    z = torch.zeros((8, 8, 24), dtype=torch.int16)
    with pytest.raises(ValueError):
        exl3.EXL3Tensor(z, torch.ones(128), torch.ones(128), codebook=0)   # 1.5 bits needs mul1
    with pytest.raises(ValueError):
        exl3.EXL3Tensor(torch.zeros((8, 8, 20), dtype=torch.int16), torch.ones(128), torch.ones(128))
