"""CPU oracle for the quantized-weight matmul path — TEST INFRASTRUCTURE ONLY.

A ctypes view of oracle/liboracle.so (built from ishz_oracle.c by oracle/Makefile). Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
product (ishizuki_amd) never does. Each function names the reference function it restates
in ishz_oracle.c; what pins it is listed in ishz_oracle.h.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4_0, Q2_K, Q4_K, Q6_K, IQ2_XS = 2, 10, 12, 14, 17
F32, F16, BF16 = 0, 1, 30
IQ2_XXS, IQ3_XXS, IQ1_S, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 18, 19, 21, 22, 23, 29

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, U, F, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_float, ctypes.c_size_t
        sig = {
            "ishzo_block_size": (I, [U]),
            "ishzo_type_size": (I, [U]),
            "ishzo_half_to_float": (F, [ctypes.c_uint16]),
            "ishzo_float_to_half": (ctypes.c_uint16, [F]),
            "ishzo_dequant": (I, [U, P, SZ, SZ, P]),
            "ishzo_dequant_rows": (I, [U, P, I, I, P, I]),
            "ishzo_ggml_matmul": (I, [U, P, I, I, P, I, P, I]),
            "ishzo_ggml_matmul_fused": (I, [U, P, I, I, P, I, P, I]),
            "ishzo_affine_dequant": (I, [P, P, P, I, I, I, I, P]),
            "ishzo_affine_matmul": (I, [P, I, I, P, P, P, I, I, I, P, I]),
            "ishzo_hadamard": (None, [P, I, I, I, P, I, P]),
            "ishzo_exl3_dequant": (I, [P, I, I, I, I, P]),
            "ishzo_exl3_decode": (F, [U, I]),
            "ishzo_exl3_apply": (I, [P, I, I, P, P, P, I, I, I, P, I]),
            "ishzo_moe_route": (None, [P, I, I, I, I, P, P]),
            "ishzo_moe_swiglu": (I, [U, P, I, I, P, P, I, P, P, P, I, I, P, P, P, I]),
            "ishzo_bench_affine_linear": (ctypes.c_double, [P, I, P, I, P, P, P, I, I, I, I, I, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def block_size(t):
    return lib().ishzo_block_size(t)


def type_size(t):
    return lib().ishzo_type_size(t)


def dequant(type_, blocks, count):
    """GGMLDequant.dequantize (Core/GGMLDequant.swift:25). Raises on refusal like the reference."""
    b = _c(np.frombuffer(bytes(blocks), np.uint8) if isinstance(blocks, (bytes, bytearray)) else blocks, np.uint8)
    out = np.empty(count, np.float32)
    rc = lib().ishzo_dequant(type_, _p(b), b.size, count, _p(out))
    if rc:
        raise ValueError({-1: "unsupported type", -2: "count is not whole blocks", -3: "short buffer"}[rc])
    return out


def dequant_rows(type_, blocks, N, K, threads=0):
    """W [N][K] from its GGML blocks, rows decoded in parallel (ishzo_dequant per row)."""
    b = _c(blocks, np.uint8)
    out = np.empty((N, K), np.float32)
    rc = lib().ishzo_dequant_rows(type_, _p(b), N, K, _p(out), threads)
    if rc:
        raise ValueError(f"oracle dequant failed {rc}")
    return out


def ggml_matmul(type_, x, blocks, N, threads=0, fused=False):
    x = _c(np.atleast_2d(x), np.float32)
    M, K = x.shape
    b = _c(blocks, np.uint8)
    y = np.empty((M, N), np.float32)
    fn = lib().ishzo_ggml_matmul_fused if fused else lib().ishzo_ggml_matmul
    rc = fn(type_, _p(x), M, K, _p(b), N, _p(y), threads)
    if rc:
        raise ValueError(f"oracle matmul failed {rc}")
    return y


def affine_dequant(codes, scales, biases, N, K, bits, group):
    out = np.empty((N, K), np.float32)
    rc = lib().ishzo_affine_dequant(_p(_c(codes, np.uint32)), _p(_c(scales, np.uint16)),
                                    _p(_c(biases, np.uint16)), N, K, bits, group, _p(out))
    if rc:
        raise ValueError("bad affine geometry")
    return out


def affine_matmul(x, codes, scales, biases, N, bits, group, threads=0):
    x = _c(np.atleast_2d(x), np.float32)
    M, K = x.shape
    y = np.empty((M, N), np.float32)
    rc = lib().ishzo_affine_matmul(_p(x), M, K, _p(_c(codes, np.uint32)), _p(_c(scales, np.uint16)),
                                   _p(_c(biases, np.uint16)), N, bits, group, _p(y), threads)
    if rc:
        raise ValueError("bad affine geometry")
    return y


def hadamard(x, block, signs=None, inverse=False):
    x = _c(np.atleast_2d(x), np.float32)
    rows, width = x.shape
    y = np.empty_like(x)
    s = None if signs is None else _c(signs, np.float32)
    lib().ishzo_hadamard(_p(x), rows, width, block, None if s is None else _p(s), int(inverse), _p(y))
    return y


def exl3_decode(state, codebook):
    return lib().ishzo_exl3_decode(state, codebook)


def exl3_dequant(trellis, bits2, codebook):
    t = _c(trellis, np.int16)
    K, N = t.shape[0] * 16, t.shape[1] * 16
    out = np.empty((K, N), np.float32)
    if lib().ishzo_exl3_dequant(_p(t), K, N, bits2, codebook, _p(out)):
        raise ValueError("bad EXL3 rate/codebook")
    return out


def exl3_apply(x, trellis, suh, svh, bits2, codebook, threads=0):
    x = _c(np.atleast_2d(x), np.float32)
    M, K = x.shape
    t = _c(trellis, np.int16)
    N = t.shape[1] * 16
    y = np.empty((M, N), np.float32)
    rc = lib().ishzo_exl3_apply(_p(x), M, K, _p(t), _p(_c(suh, np.float32)), _p(_c(svh, np.float32)),
                                N, bits2, codebook, _p(y), threads)
    if rc:
        raise ValueError("bad EXL3 rate/codebook")
    return y


def moe_route(logits, topk, normalize=True):
    l = _c(logits, np.float32)
    T, E = l.shape
    ids = np.empty((T, topk), np.int32)
    w = np.empty((T, topk), np.float32)
    lib().ishzo_moe_route(_p(l), T, E, topk, int(normalize), _p(ids), _p(w))
    return ids, w


def moe_swiglu(type_, x, ids, weights, gate, up, down, E, I, threads=0, shared=None, shared_gate=None):
    """shared [T][H] / shared_gate [T]: the shared expert's output and gate logit (fp16 values)."""
    x = _c(np.atleast_2d(x), np.float32)
    T, H = x.shape
    ids = _c(ids, np.int32)
    topk = ids.shape[1]
    y = np.empty((T, H), np.float32)
    sh = None if shared is None else _c(np.reshape(shared, (T, H)), np.float32)
    sg = None if shared_gate is None else _c(np.reshape(shared_gate, (T,)), np.float32)
    rc = lib().ishzo_moe_swiglu(type_, _p(x), T, H, _p(ids), _p(_c(weights, np.float32)), topk,
                                _p(_c(gate, np.uint8)), _p(_c(up, np.uint8)), _p(_c(down, np.uint8)),
                                E, I, None if sh is None else _p(sh), None if sg is None else _p(sg), _p(y), threads)
    if rc:
        raise ValueError(f"moe oracle failed {rc}")
    return y
