import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


FP16_SUBNORMAL_STEP = 2.0 ** -24
# Per-element criterion: |y - ref| <= ELEM_TOL * sum_k |x_k||w_k| + half an fp16 ulp of the output.
# The reference judges each element against the sum of the magnitudes that formed it
# (Tests/IshizukiKitTests/GGMLKernelTests.swift:131-137, 1e-5 with fp32 outputs). The kernels add
# the format's magic offset (fp16 1024 + q) before the fp32 dot and take it back out through the
# sum of x, so their fp32 partials carry about 1024/|q| times the magnitude of the plain dot's:
# 1e-4 of the bound covers that at K = 25600, and the fp16 output rounding is added on top.
ELEM_TOL = 1e-4


def assert_close(y, ref, rel=1e-3, what="", bound=None, elem=ELEM_TOL):
    """Two checks on fp16 outputs against the oracle's fp32 result:
    * normwise: max |y - ref| <= rel * max |ref| (BASELINE's max relative error 1e-3), plus the
      fp16 subnormal spacing 2^-24 (an fp16 output cannot resolve finer than that);
    * per element, when `bound` (= |x| @ |W|.T, the sum of the magnitudes forming each output) is
      given: |y_i - ref_i| <= elem * bound_i + 2^-11 |ref_i| + 2^-24, so a wrong small-magnitude
      element fails even when the largest outputs are right.
    Returns the normwise relative error."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    scale = np.abs(ref).max()
    d = np.abs(y - ref)
    err = d.max()
    assert err <= rel * scale + FP16_SUBNORMAL_STEP, f"{what}: max err {err:.3e} > {rel} * {scale:.3e} (rel {err / scale:.3e})"
    if bound is not None:
        bound = np.asarray(bound, np.float64)
        assert bound.shape == ref.shape
        lim = elem * bound + 2.0 ** -11 * np.abs(ref) + FP16_SUBNORMAL_STEP
        bad = d > lim
        if bad.any():
            i = np.unravel_index(np.argmax(d / lim), d.shape)
            raise AssertionError(f"{what}: {int(bad.sum())} elements outside the per-element bound; worst at {i}: "
                                 f"|y-ref| {d[i]:.3e}, bound {bound[i]:.3e}, ref {ref[i]:.3e}")
    return err / scale


def ggml_reference(type_, x, blocks, N):
    """(ref, bound) for y = x @ W.T with W the GGML blocks [N][K]: ref is the oracle's
    dequantize-then-fp32-dot, bound = |x| @ |W|.T."""
    import oracle
    x = np.asarray(x, np.float32)
    ref = oracle.ggml_matmul(type_, x, blocks, N)
    W = oracle.dequant_rows(type_, blocks, N, x.shape[1])
    np.abs(W, out=W)
    bound = np.abs(x) @ W.T
    return ref, bound


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    same = a.view(np.uint32) == b.view(np.uint32)
    return bool(np.all(same | (np.isnan(a) & np.isnan(b))))


@pytest.fixture(scope="session")
def golden_ggml():
    import struct
    raw = open(os.path.join(ROOT, "tests", "golden", "ggml_reference.bin"), "rb").read()
    assert raw[:8] == b"GGMLREF1"
    (count,) = struct.unpack("<I", raw[8:12])
    p, out = 12, {}
    for _ in range(count):
        t, nb, nby, nf = struct.unpack("<4I", raw[p:p + 16])
        p += 16
        b = np.frombuffer(raw[p:p + nby], np.uint8).copy()
        p += nby
        e = np.frombuffer(raw[p:p + 4 * nf], np.float32).copy()
        p += 4 * nf
        out[t] = (b, e)
    return out


@pytest.fixture(scope="session")
def golden_exl3():
    return dict(np.load(os.path.join(ROOT, "tests", "golden", "exl3_reference.npz")))


MOE_ELEM = 2.0 ** -9


def moe_reference(type_, x, ids, weights, gate, up, down, E, I, shared=None, shared_gate=None):
    """(ref, bound) for the expert-gathered SwiGLU FFN: ref is the oracle's loop-per-token
    restatement; bound_t = sum_s w_s |W_down[e_s]| @ |h_s|, the magnitudes forming each output.
    Check with elem=MOE_ELEM: an fp16 intermediate (a projection output, silu, h) computed in
    another summation order may round one ulp the other way, which moves the output by about 2^-10
    of its bound; 2^-9 leaves room for two such flips and nothing more."""
    import oracle
    x = np.asarray(x, np.float32)
    T, H = x.shape
    ref = oracle.moe_swiglu(type_, x, ids, weights, gate, up, down, E, I, shared=shared, shared_gate=shared_gate)
    bs, ts = oracle.block_size(type_), oracle.type_size(type_)
    gb = I * (H // bs) * ts
    db = H * (I // bs) * ts
    cache = {}

    def expert(e):
        if e not in cache:
            g = oracle.dequant_rows(type_, gate[e * gb:(e + 1) * gb], I, H)
            u = oracle.dequant_rows(type_, up[e * gb:(e + 1) * gb], I, H)
            d = oracle.dequant_rows(type_, down[e * db:(e + 1) * db], H, I)
            cache[e] = (g, u, np.abs(d))
        return cache[e]

    bound = np.zeros((T, H), np.float64)
    for t in range(T):
        for s in range(ids.shape[1]):
            g, u, ad = expert(int(ids[t, s]))
            gv = g @ x[t]
            h = gv / (1.0 + np.exp(-gv.astype(np.float64))) * (u @ x[t])
            bound[t] += float(weights[t, s]) * (ad @ np.abs(h))
    if shared is not None:
        bound += np.abs(np.asarray(shared, np.float64))
    return ref, bound
