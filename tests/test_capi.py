"""The C-ABI library loads and exports every symbol include/ishizuki_hip.h declares (no GPU)."""
import ctypes
import os

from ishizuki_amd import _lib


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in _lib.header_symbols() if not hasattr(L, s)]
    assert not missing, missing


def test_version_and_geometry():
    L = _lib.lib()
    assert L.ishz_version() >= 100
    assert [L.ishz_ggml_block_size(t) for t in (2, 12, 14, 17)] == [32, 256, 256, 256]
    assert [L.ishz_ggml_type_size(t) for t in (2, 12, 14, 17)] == [18, 144, 210, 74]
    assert L.ishz_ggml_block_size(11) == 0


def test_declines_without_touching_the_gpu():
    # GGMLKernelTests (:204-213): too many rows, ragged K, short buffer, unsupported type.
    L = _lib.lib()
    dummy = ctypes.c_void_p(16)
    assert L.ishz_ggml_matvec(12, dummy, _lib.DT_F16, 17, 256, dummy, 1 << 20, 4, dummy, None) == _lib.DECLINED
    assert L.ishz_ggml_matvec(12, dummy, _lib.DT_F16, 1, 100, dummy, 1 << 20, 4, dummy, None) == _lib.DECLINED
    assert L.ishz_ggml_matvec(12, dummy, _lib.DT_F16, 1, 256, dummy, 143, 1, dummy, None) == _lib.DECLINED
    assert L.ishz_ggml_matvec(11, dummy, _lib.DT_F16, 1, 256, dummy, 1 << 20, 1, dummy, None) == _lib.DECLINED
    assert L.ishz_ggml_matmul_few(2, dummy, _lib.DT_F16, 4, 256, dummy, 1 << 20, 4, 2, dummy, None) == _lib.DECLINED
    assert L.ishz_ggml_matmul_few(12, dummy, _lib.DT_F16, 1, 256, dummy, 1 << 20, 4, 2, dummy, None) == _lib.DECLINED
    assert "declined" in _lib.last_error()


def test_modulemap_names_the_header():
    here = os.path.dirname(_lib.HEADER)
    text = open(os.path.join(here, "module.modulemap")).read()
    assert 'header "ishizuki_hip.h"' in text and 'link "ishizuki_hip"' in text
