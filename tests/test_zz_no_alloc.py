"""ishz_exl3_apply_static (the no-allocation EXL3 apply) against ishz_exl3_apply, through the C ABI.

Both run the same kernels on the same inputs, one with a caller workspace and one with the
library's static device scratch, so the outputs must be bit-identical. Two calls in a row, the
second smaller, show that what the first left in the scratch does not leak into the second; a
shape whose workspace exceeds the scratch is refused with ISHZ_EINVAL.
"""
import numpy as np
import pytest
import torch

from ishizuki_amd import _lib, synth
from ishizuki_amd._torch import ptr, stream

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _both(M, K, N, bits2, cb, seed):
    t, suh, svh = synth.exl3_pack(K, N, bits2=bits2, seed=seed)
    x = torch.from_numpy(synth.fp16_normal((M, K), seed=seed + 1)).to(DEV)
    td, sd, vd = (torch.from_numpy(a).to(DEV) for a in (t, suh, svh))
    L = _lib.lib()
    ws = torch.empty(L.ishz_exl3_workspace_size(M, K, N), dtype=torch.uint8, device=DEV)
    y_ws = torch.empty((M, N), dtype=torch.float16, device=DEV)
    y_st = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    rc = L.ishz_exl3_apply(ptr(x), _lib.DT_F16, M, K, ptr(td), ptr(sd), ptr(vd), N, bits2, cb, ptr(y_ws), ptr(ws),
                           ws.numel(), stream())
    assert rc == _lib.OK, _lib.last_error()
    rc = L.ishz_exl3_apply_static(ptr(x), _lib.DT_F16, M, K, ptr(td), ptr(sd), ptr(vd), N, bits2, cb, ptr(y_st),
                                  stream())
    assert rc == _lib.OK, _lib.last_error()
    torch.cuda.synchronize()
    a, b = y_ws.cpu().numpy(), y_st.cpu().numpy()
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"M={M} K={K} N={N}"


def test_static_matches_workspace_twice_then_smaller():
    print("no-alloc exl3 apply: M=8 K=5120 N=4096, then M=2 K=1024 N=512", flush=True)
    _both(8, 5120, 4096, 4, 0, seed=11)   # K-split partials + rotated x in the scratch
    _both(2, 1024, 512, 2, 1, seed=12)    # smaller: the first call's contents are left behind
    _both(1, 1024, 1024, 4, 2, seed=13)   # one row: the fused input rotation path


def test_static_rejects_oversized():
    L = _lib.lib()
    M, K, N = 16, 1 << 20, 128  # the rotated x alone is 32 MiB
    assert L.ishz_exl3_workspace_size(M, K, N) > (32 << 20)
    rc = L.ishz_exl3_apply_static(None, _lib.DT_F16, M, K, None, None, None, N, 4, 0, None, stream())
    assert rc == _lib.EINVAL and "scratch" in _lib.last_error()
