"""GGML kernels on the GPU vs the CPU oracle, through the C ABI.

Dequant/gather: bit-exact (fp32 bits; fp16/bf16 = the oracle's fp32 rounded once).
Matmul (GEMV M=1 and MFMA verify M=2..16): max |y - ref| <= 1e-3 * max |ref| on fp16 outputs,
ref = the oracle's dequantize-then-fp32-dot.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import assert_close, bits_equal, ggml_reference
from ishizuki_amd import ggml, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TYPES = list(ggml.SUPPORTED)  # the four headline formats and the quarter-block ones
QUARTER = [ggml.Q2_K, ggml.IQ4_XS, ggml.IQ2_XXS, ggml.IQ2_S, ggml.IQ3_XXS, ggml.IQ3_S, ggml.IQ1_S, ggml.IQ1_M]


def to_bf16_bits(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


@pytest.mark.parametrize("t", [10, 12, 14, 16, 17, 18, 19, 21, 22, 23, 29])
def test_dequant_golden_bit_exact(golden_ggml, t):
    """The reference's own vectors (ggml-reference.bin) for every type it decodes."""
    b, e = golden_ggml[t]
    out = ggml.dequantize(torch.from_numpy(b).to(DEV), t, (e.size,), dtype=torch.float32)
    assert bits_equal(out.cpu().numpy(), e)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_dequant_synthetic(t, dt):
    N, K = 37, 1024
    blk = synth.ggml_blocks(t, N, K, seed=7 + t)
    ref = oracle.dequant(t, blk, N * K)
    out = ggml.dequantize(torch.from_numpy(blk).to(DEV), t, (N, K), dtype=dt).cpu()
    if dt == torch.float32:
        assert bits_equal(out.numpy().reshape(-1), ref)
    elif dt == torch.float16:
        assert np.array_equal(out.numpy().reshape(-1).view(np.uint16), ref.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(out.view(torch.int16).numpy().reshape(-1).view(np.uint16), to_bf16_bits(ref))


@pytest.mark.parametrize("t", TYPES)
def test_gather_exact_and_out_of_range_is_zero(t):
    N, K = 50, 512
    blk = synth.ggml_blocks(t, N, K, seed=3)
    ref = oracle.dequant(t, blk, N * K).reshape(N, K)
    ids = np.array([3, 49, 0, 3, 17, -1, 50], np.int32)
    out = ggml.gather(torch.from_numpy(ids).to(DEV), torch.from_numpy(blk).to(DEV), t, K,
                      dtype=torch.float32).cpu().numpy()
    assert bits_equal(out[:5], ref[ids[:5]])
    assert np.all(out[5:] == 0)


def run_matvec(t, M, N, K, seed=0, few=False):
    blk = synth.ggml_blocks(t, N, K, seed=seed)
    x = synth.fp16_normal((M, K), seed=seed + 1)
    ref, bound = ggml_reference(t, x, blk, N)
    xb = torch.from_numpy(x).to(DEV)
    wb = torch.from_numpy(blk).to(DEV)
    y = (ggml.matmul_few if few else ggml.matvec)(xb, wb, t, N)
    assert y is not None, "kernel declined"
    return y.float().cpu().numpy(), ref, bound


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("N,K", [(64, 4096), (17, 5120), (1000, 768 * 4), (40, 256 * 3)])
def test_gemv_m1(t, N, K):
    if K % synth.BLOCK[t][0]:
        pytest.skip("K not whole blocks")
    print(f"gemv type={t} N={N} K={K}", flush=True)
    y, ref, bd = run_matvec(t, 1, N, K, seed=N + t)
    assert_close(y, ref, bound=bd, what=f"gemv t={t} N={N} K={K}")


def _random_cases(n, seed):
    """Seeded shapes across every format: N from 1 to 2499 (ragged tiles, single rows), K any
    whole number of blocks up to about 12K, M from 1 to 8 (GEMV, verify, per-block paths)."""
    r = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        t = TYPES[i % len(TYPES)]
        bk = synth.BLOCK[t][0]
        cases.append((t, int(r.integers(1, 2500)), bk * int(r.integers(1, 12288 // bk + 1)), int(r.integers(1, 9))))
    return cases


@pytest.mark.parametrize("t,N,K,M", _random_cases(48, 2024))
def test_random_shapes(t, N, K, M):
    print(f"random shape type={t} N={N} K={K} M={M}", flush=True)
    y, ref, bd = run_matvec(t, M, N, K, seed=N + K + M)
    assert_close(y, ref, bound=bd, what=f"random t={t} N={N} K={K} M={M}")


def test_gemv_wide_lanes():
    # units >= 1024 per row: the 32-lanes-per-row variant
    y, ref, bd = run_matvec(ggml.Q4_0, 1, 48, 32768, seed=5)
    assert_close(y, ref, bound=bd)


@pytest.mark.parametrize("t", TYPES)
def test_gemv_long_k(t):
    """K = 25600, M = 1: 400 units per row, so 64 lanes per row (ragged) and 1024-thread
    workgroups; N not a multiple of the workgroup's rows."""
    N, K = 130, 25600
    print(f"gemv long K type={t}", flush=True)
    y, ref, bd = run_matvec(t, 1, N, K, seed=31 + t)
    assert_close(y, ref, bound=bd, what=f"gemv long K t={t}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [2, 3, 5, 8, 16])
def test_verify_rows(t, M):
    N, K = 4100, 1024   # N >= 4096: two tiles per workgroup, ragged last tile
    print(f"verify type={t} M={M}", flush=True)
    y, ref, bd = run_matvec(t, M, N, K, seed=M + 10 * t)
    assert_close(y, ref, bound=bd, what=f"verify t={t} M={M}")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [8, 16])
def test_verify_long_k_chunks(t, M):
    """K = 25600 (the down projection): x is staged in several K chunks per workgroup."""
    N, K = 300, 25600
    print(f"verify long K type={t} M={M}", flush=True)
    y, ref, bd = run_matvec(t, M, N, K, seed=M + t)
    assert_close(y, ref, bound=bd, what=f"verify long K t={t} M={M}")


@pytest.mark.parametrize("M", [2, 7])
def test_verify_q4_0_k_not_multiple_of_256(M):
    """K % 256 != 0 takes the per-block verify kernel."""
    y, ref, bd = run_matvec(ggml.Q4_0, M, 130, 32 * 13, seed=M)
    assert_close(y, ref, bound=bd, what=f"q4_0 K=416 M={M}")


@pytest.mark.parametrize("t", [ggml.Q4_K, ggml.Q6_K, ggml.IQ2_XS] + QUARTER)
def test_matmul_few_ragged(t):
    # GGMLKernelTests.matmulFew (:145-175): N = 17, a ragged tile
    for M in range(2, 9):
        y, ref, bd = run_matvec(t, M, 17, 512, seed=M, few=True)
        assert_close(y, ref, bound=bd, what=f"few t={t} M={M}")


def test_matvec_rows_agree_with_single_row():
    # a row's result does not depend on how many rows ride along
    t, N, K = ggml.Q4_K, 300, 2048
    blk = torch.from_numpy(synth.ggml_blocks(t, N, K, seed=9)).to(DEV)
    x = torch.from_numpy(synth.fp16_normal((8, K), seed=10)).to(DEV)
    y8 = ggml.matvec(x, blk, t, N).float()
    for m in range(8):
        y1 = ggml.matvec(x[m:m + 1], blk, t, N).float()
        assert torch.allclose(y1[0], y8[m], rtol=2e-3, atol=2e-3 * y8[m].abs().max().item())


def test_declines_return_none():
    blk = torch.zeros(144 * 4, dtype=torch.uint8, device=DEV)
    x = torch.zeros((17, 256), dtype=torch.float16, device=DEV)
    assert ggml.matvec(x, blk, ggml.Q4_K, 4) is None
    assert ggml.matvec(x[:1].to(torch.int16), blk, ggml.Q4_K, 4) is None  # integer x
    assert ggml.matvec(x[:1], blk, ggml.Q4_K, 5) is None   # short buffer


@pytest.mark.parametrize("rows", [3, 16, 20, 40])
def test_apply_row_policy(rows):
    """PackedLinear.ggmlApply's row policy: one call to 16 rows, 16-row calls, then dequantize +
    GEMM (40 rows of a small matrix). Same tolerance as the matvec."""
    N, K = 256, 1024
    blk = synth.ggml_blocks(ggml.Q4_K, N, K, seed=rows)
    x = synth.fp16_normal((rows, K), seed=rows + 1)
    ref, bd = ggml_reference(ggml.Q4_K, x, blk, N)
    y = ggml.apply(torch.from_numpy(x).to(DEV), torch.from_numpy(blk).to(DEV), ggml.Q4_K, N)
    assert y is not None and y.shape == (rows, N)
    assert_close(y.float().cpu().numpy(), ref, bound=bd, what=f"ggml apply rows={rows}")


@pytest.mark.parametrize("t", [ggml.Q4_0, ggml.Q4_K, ggml.Q6_K, ggml.IQ2_XS, ggml.IQ3_S])
@pytest.mark.parametrize("M", [2, 9])
def test_verify_k_split_matches_unsplit(t, M):
    """A narrow output (33 tiles) with a workspace takes the K split (fp32 parts summed in part
    order); without one, the unsplit kernel. Both against the oracle, per element."""
    from ishizuki_amd import _lib
    from ishizuki_amd._torch import ptr, stream
    N, K = 520, 8192
    L = _lib.lib()
    image = lambda m: (m * K * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256  # bf16 / fp32 x's fp16 image
    wsb = L.ishz_ggml_workspace_size(t, M, K, N)
    assert wsb > image(M), "this shape should be split"
    assert L.ishz_ggml_workspace_size(t, M, K, 17408) == image(M)  # wide outputs are not
    assert L.ishz_ggml_workspace_size(t, 1, K, N) == image(1)      # nor the GEMV
    blocks = synth.ggml_blocks(t, N, K, seed=M + 3 * t)
    x = synth.fp16_normal((M, K), seed=M + 7)
    wb, xd = torch.from_numpy(blocks).to(DEV), torch.from_numpy(x).to(DEV)
    ys = []
    for ws_bytes in (wsb, 0):
        y = torch.empty((M, N), dtype=torch.float16, device=DEV)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        print(f"k-split t={t} M={M} ws={ws_bytes}", flush=True)
        assert L.ishz_ggml_matvec_ws(t, ptr(xd), _lib.DT_F16, M, K, ptr(wb), blocks.nbytes, N, ptr(y),
                                     ptr(ws) if ws_bytes else None, ws_bytes, stream()) == _lib.OK
        ys.append(y.float().cpu().numpy())
    ref, bd = ggml_reference(t, x.astype(np.float32), blocks, N)
    for y, what in zip(ys, ("split", "unsplit")):
        assert_close(y, ref, bound=bd, what=f"{what} t={t} M={M}")
