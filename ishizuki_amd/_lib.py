"""Loads libishizuki_hip.so and declares the C ABI of include/ishizuki_hip.h for ctypes.

The product path has no fallback: if the library is missing, importing a kernel module raises.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libishizuki_hip.so")
HEADER = os.path.join(HERE, "..", "include", "ishizuki_hip.h")

OK, DECLINED, EINVAL, EHIP = 0, 1, 2, 3
DT_F32, DT_F16, DT_BF16 = 0, 1, 2

P, I, U32, SZ, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_float
_SIGS = {
    "ishz_last_error": (ctypes.c_char_p, []),
    "ishz_version": (I, []),
    "ishz_stream_read": (I, [P, SZ, P, P]),
    "ishz_ggml_block_size": (I, [U32]),
    "ishz_ggml_type_size": (I, [U32]),
    "ishz_ggml_matvec": (I, [U32, P, I, I, I, P, SZ, I, P, P]),
    "ishz_ggml_workspace_size": (SZ, [U32, I, I, I]),
    "ishz_ggml_matvec_ws": (I, [U32, P, I, I, I, P, SZ, I, P, P, SZ, P]),
    "ishz_ggml_matmul_few": (I, [U32, P, I, I, I, P, SZ, I, I, P, P]),
    "ishz_ggml_dequant": (I, [U32, P, SZ, SZ, P, I, P]),
    "ishz_ggml_gather": (I, [U32, P, I, P, SZ, I, I, P, I, P]),
    "ishz_hadamard": (I, [P, I, I, I, I, P, I, P, P]),
    "ishz_affine_matmul": (I, [P, I, I, I, P, P, P, I, I, I, I, P, P]),
    "ishz_affine_workspace_size": (SZ, [I, I]),
    "ishz_affine_linear": (I, [P, I, I, I, P, I, P, P, P, I, I, I, I, P, P, SZ, P]),
    "ishz_exl3_dequant": (I, [P, I, I, I, I, P, I, P]),
    "ishz_exl3_rotate": (I, [P, I, I, I, P, I, P, I, P]),
    "ishz_exl3_matvec": (I, [P, I, I, I, P, I, I, I, P, P]),
    "ishz_exl3_matvec_workspace_size": (SZ, [I, I, I]),
    "ishz_exl3_matvec_ws": (I, [P, I, I, I, P, I, I, I, P, P, SZ, P]),
    "ishz_exl3_workspace_size": (SZ, [I, I, I]),
    "ishz_exl3_apply": (I, [P, I, I, I, P, P, P, I, I, I, P, P, SZ, P]),
    "ishz_exl3_apply_static": (I, [P, I, I, I, P, P, P, I, I, I, P, P]),
    "ishz_moe_route": (I, [P, I, I, I, I, P, P, P]),
    "ishz_moe_workspace_size": (SZ, [I, I, I, I, I]),
    "ishz_moe_swiglu": (I, [U32, P, I, I, I, P, I, I, I, P, P, P, SZ, I, P, P, P, P, P, P, SZ, P]),
    "ishz_moe_swiglu_affine": (I, [P, I, I, I, P, I, I, I, P, P, P, P, P, P, P, P, P, I, I, I, I, P, P, P, P, P, P, SZ,
                                   P]),
    "ishz_ggml_type_known": (I, [U32]),
    "ishz_ggml_geometry": (I, [U32, ctypes.POINTER(I), ctypes.POINTER(I)]),
    "ishz_gguf_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "ishz_gguf_close": (None, [P]),
    "ishz_gguf_version": (U32, [P]),
    "ishz_gguf_data_offset": (ctypes.c_uint64, [P]),
    "ishz_gguf_tensor_count": (ctypes.c_int64, [P]),
    "ishz_gguf_find_tensor": (ctypes.c_int64, [P, ctypes.c_char_p]),
    "ishz_gguf_tensor_info": (I, [P, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(I),
                                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(U32),
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "ishz_gguf_tensor_data": (P, [P, ctypes.c_int64]),
    "ishz_gguf_tensor_upload": (I, [P, ctypes.c_int64, P, SZ, P]),
    "ishz_gguf_kv_count": (ctypes.c_int64, [P]),
    "ishz_gguf_kv_key": (ctypes.c_char_p, [P, ctypes.c_int64]),
    "ishz_gguf_find_kv": (ctypes.c_int64, [P, ctypes.c_char_p]),
    "ishz_gguf_kv_value": (P, [P, ctypes.c_int64]),
    "ishz_gguf_value_type": (I, [P]),
    "ishz_gguf_value_len": (ctypes.c_int64, [P]),
    "ishz_gguf_value_elem": (P, [P, ctypes.c_int64]),
    "ishz_gguf_value_int": (I, [P, ctypes.POINTER(ctypes.c_int64)]),
    "ishz_gguf_value_float": (I, [P, ctypes.POINTER(ctypes.c_double)]),
    "ishz_gguf_value_bool": (I, [P, ctypes.POINTER(I)]),
    "ishz_gguf_value_string": (I, [P, ctypes.POINTER(P), ctypes.POINTER(SZ)]),
    "ishz_gguf_value_raw": (I, [P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int64),
                                ctypes.POINTER(ctypes.c_double)]),
}

_lib = None


class IshzError(RuntimeError):
    pass


def header_symbols():
    """Function names declared by include/ishizuki_hip.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(ishz_\w+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise IshzError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().ishz_last_error().decode()


def check(rc, what):
    """OK -> True, DECLINED -> False (the reference's nil), anything else raises."""
    if rc == OK:
        return True
    if rc == DECLINED:
        return False
    raise IshzError(f"{what}: status {rc}: {last_error()}")
