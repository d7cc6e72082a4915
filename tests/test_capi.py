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


def test_header_compiles_as_c11_and_links(tmp_path):
    """A C caller (what the Swift module map imports) compiles against the header with gcc
    -std=c11 -Wall -Werror, links against the library, and gets the library's answers back: the
    version, the block geometry and a decline that never reaches the GPU."""
    import subprocess
    src = tmp_path / "caller.c"
    src.write_text(r'''
#include "ishizuki_hip.h"
#include <stdio.h>
#include <string.h>
int main(void) {
  char dummy[16] = {0};
  int rc = ishz_ggml_matvec(12, dummy, ISHZ_DT_F16, 17, 256, dummy, 1u << 20, 4, dummy, NULL);
  printf("%d %d %d %d %d\n", ishz_version() >= 100, ishz_ggml_block_size(12), ishz_ggml_type_size(14),
         rc == ISHZ_DECLINED, strstr(ishz_last_error(), "declined") != NULL);
  return 0;
}
''')
    exe = tmp_path / "caller"
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.dirname(_lib.HEADER),
                    str(src), "-L", libdir, "-lishizuki_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    assert out == ["1", "256", "210", "1", "1"]
