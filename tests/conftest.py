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


def assert_close(y, ref, rel=1e-3, what=""):
    """max |y - ref| <= rel * max |ref| (fp16 outputs vs the oracle's fp32 result), plus the fp16
    subnormal spacing 2^-24: an fp16 output cannot resolve finer than that, so outputs that land
    in fp16's subnormal range (|y| < 6.1e-5) are held to one subnormal step."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    scale = np.abs(ref).max()
    err = np.abs(y - ref).max()
    assert err <= rel * scale + FP16_SUBNORMAL_STEP, f"{what}: max err {err:.3e} > {rel} * {scale:.3e} (rel {err / scale:.3e})"
    return err / scale


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
