"""GGUF container reader and packed-weight loader over the C ABI (host-side C++ in csrc/gguf.cpp).

Mirrors GGUFFile (Sources/IshizukiKit/Config/GGUFFile.swift:179-397), GGUFValue (:125-168), the
GGMLType geometry (:13-121) and the packed half of GGUFWeights.load
(Sources/IshizukiKit/Core/GGUFWeights.swift:47-85): names, shapes (row-major), errors on malformed
files (GGUFError here, BonsaiError there) and the tensor bytes read from the data section.
"""
import ctypes
from collections import Counter, namedtuple

from . import _lib

# GGMLType raw values (GGUFFile.swift:13-43) and names (:90-116)
GGML_TYPES = {
    0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1", 10: "Q2_K",
    11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS",
    19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32",
    27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16",
}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file (the reference throws BonsaiError)."""


def geometry(type_):
    """(blockSize, typeSize) of a GGMLType raw value."""
    bs, ts = ctypes.c_int(), ctypes.c_int()
    if _lib.lib().ishz_ggml_geometry(type_, ctypes.byref(bs), ctypes.byref(ts)) != _lib.OK:
        raise GGUFError(f"unknown GGML type {type_}")
    return bs.value, ts.value


def byte_count(type_, elements):
    """GGMLType.byteCount(elements:) (GGUFFile.swift:118-120)."""
    bs, ts = geometry(type_)
    return elements // bs * ts


def is_quantized(type_):
    return geometry(type_)[0] > 1


class TensorInfo(namedtuple("TensorInfo", "name shape type offset byte_count")):
    @property
    def element_count(self):
        n = 1
        for d in self.shape:
            n *= d
        return n


class GGUFValue:
    """One metadata value (GGUFValue): read through the reference's accessors."""

    def __init__(self, file, ptr):
        self._file, self._p = file, ptr  # the file keeps the storage alive

    @property
    def type(self):
        return _lib.lib().ishz_gguf_value_type(self._p)

    def _get(self, fn, ctype):
        v = ctype()
        return v.value if fn(self._p, ctypes.byref(v)) == _lib.OK else None

    @property
    def int_value(self):
        return self._get(_lib.lib().ishz_gguf_value_int, ctypes.c_int64)

    @property
    def float_value(self):
        return self._get(_lib.lib().ishz_gguf_value_float, ctypes.c_double)

    @property
    def bool_value(self):
        v = self._get(_lib.lib().ishz_gguf_value_bool, ctypes.c_int)
        return None if v is None else bool(v)

    @property
    def string_value(self):
        s, n = ctypes.c_void_p(), ctypes.c_size_t()
        if _lib.lib().ishz_gguf_value_string(self._p, ctypes.byref(s), ctypes.byref(n)) != _lib.OK:
            return None
        return ctypes.string_at(s, n.value).decode("utf-8", errors="replace")

    @property
    def array_value(self):
        L = _lib.lib()
        n = L.ishz_gguf_value_len(self._p)
        if n < 0:
            return None
        return [GGUFValue(self._file, L.ishz_gguf_value_elem(self._p, j)) for j in range(n)]

    @property
    def int_array(self):
        a = self.array_value
        return None if a is None else [v.int_value for v in a if v.int_value is not None]

    @property
    def string_array(self):
        a = self.array_value
        return None if a is None else [v.string_value for v in a if v.string_value is not None]


class GGUFFile:
    MAGIC = 0x46554747

    def __init__(self, path):
        L = _lib.lib()
        h = ctypes.c_void_p()
        rc = L.ishz_gguf_open(str(path).encode(), ctypes.byref(h))
        if rc != _lib.OK:
            raise GGUFError(L.ishz_last_error().decode())
        self._h = h
        self.path = str(path)
        self.version = L.ishz_gguf_version(h)
        self.data_offset = L.ishz_gguf_data_offset(h)
        self.metadata = {}
        for i in range(L.ishz_gguf_kv_count(h)):
            self.metadata[L.ishz_gguf_kv_key(h, i).decode("utf-8", errors="replace")] = GGUFValue(
                self, L.ishz_gguf_kv_value(h, i))
        self.tensors = []
        self._index = {}
        for i in range(L.ishz_gguf_tensor_count(h)):
            name, rank = ctypes.c_char_p(), ctypes.c_int()
            shape = (ctypes.c_int64 * 4)()
            t, off, nb = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
            L.ishz_gguf_tensor_info(h, i, ctypes.byref(name), ctypes.byref(rank), shape, ctypes.byref(t),
                                    ctypes.byref(off), ctypes.byref(nb))
            info = TensorInfo(name.value.decode("utf-8", errors="replace"), tuple(shape[:rank.value]), t.value,
                              off.value, nb.value)
            self._index[info.name] = i
            self.tensors.append(info)

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().ishz_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __getitem__(self, key):
        return self.metadata.get(key)

    def tensor(self, name):
        i = self._index.get(name)
        return None if i is None else self.tensors[i]

    @property
    def architecture(self):
        v = self.metadata.get("general.architecture")
        return (v.string_value if v else None) or ""

    def architecture_value(self, suffix):
        return self.metadata.get(f"{self.architecture}.{suffix}")

    def _i(self, tensor):
        return self._index[tensor.name if isinstance(tensor, TensorInfo) else tensor]

    def data(self, tensor):
        """The tensor's bytes from the data section (GGUFFile.data(for:))."""
        L = _lib.lib()
        i = self._i(tensor)
        p = L.ishz_gguf_tensor_data(self._h, i)
        if not p:
            raise GGUFError(L.ishz_last_error().decode())
        return ctypes.string_at(p, self.tensors[i].byte_count)

    @property
    def type_histogram(self):
        """Every storage type with how many tensors use it, most used first."""
        return Counter(t.type for t in self.tensors).most_common()


GGUFBlocks = namedtuple("GGUFBlocks", "bytes type shape")  # GGUFWeights.swift:11-25


def load_blocks(file, device="cuda:0", names=None):
    """The packed half of GGUFWeights.load: every quantized tensor's blocks, as they lie on disk,
    in a device uint8 tensor (torch is the allocator here)."""
    import torch
    from ._torch import ptr, stream
    L = _lib.lib()
    out = {}
    for t in file.tensors:
        if (names is not None and t.name not in names) or not is_quantized(t.type):
            continue
        buf = torch.empty(t.byte_count, dtype=torch.uint8, device=device)
        rc = L.ishz_gguf_tensor_upload(file._h, file._i(t), ptr(buf), t.byte_count, stream())
        if rc != _lib.OK:
            raise GGUFError(L.ishz_last_error().decode())
        out[t.name] = GGUFBlocks(buf, t.type, t.shape)
    return out
