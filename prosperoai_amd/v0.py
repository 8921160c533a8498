"""Bindings of the v0 per-group entry points of libpai_hip.so (tests and
benchmarks): the [K][N] int8 / nibble GEMMs and the flat quantizer."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib

WORKSPACE_BYTES = 4 << 20  # PAI_HIP_WQ_WORKSPACE_BYTES


class Scheme(C.Structure):
    """pai_hip_quant_scheme_t."""
    _fields_ = [("bit_width", C.c_uint8), ("is_signed", C.c_uint8), ("group_size", C.c_uint16)]


def value_bytes(n: int, bits: int) -> int:
    return (n + 1) // 2 if bits == 4 else n


def num_groups(n: int, group_size: int) -> int:
    gs = n if group_size == 0 else group_size
    return -(-n // gs)


def gemm(bits: int, a: np.ndarray, w_q: np.ndarray, scales: np.ndarray, n: int,
         group_size: int) -> np.ndarray:
    """c = a * dequant(W) through pai_hip_gemm_w8_f32 / _w4_f32 (host
    pointers, synchronous)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    m, k = a.shape
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    c = np.empty((m, n), np.float32)
    fn = lib().pai_hip_gemm_w8_f32 if bits == 8 else lib().pai_hip_gemm_w4_f32
    check(fn(m, n, k, a.ctypes.data, w_q.ctypes.data, scales.ctypes.data, group_size,
             c.ctypes.data), "pai_hip_gemm_w%d_f32" % bits)
    return c


def gemm_async(bits: int, m: int, n: int, k: int, a_ptr: int, w_ptr: int, s_ptr: int,
               group_size: int, c_ptr: int, ws_ptr: int | None, ws_bytes: int,
               stream: int | None) -> None:
    check(lib().pai_hip_gemm_wq_f32_async(bits, m, n, k, a_ptr, w_ptr, s_ptr, group_size, c_ptr,
                                          ws_ptr, ws_bytes, stream), "pai_hip_gemm_wq_f32_async")


def quantize(x: np.ndarray, bits: int, group_size: int):
    """(codes int8, scales f32) through pai_hip_quantize_f32."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    q = np.empty(value_bytes(x.size, bits), np.int8)
    s = np.empty(max(num_groups(x.size, group_size), 1), np.float32)
    ng = C.c_uint64(0)
    sch = Scheme(bits, 1, group_size)
    check(lib().pai_hip_quantize_f32(x.ctypes.data, x.size, C.byref(sch), q.ctypes.data,
                                     s.ctypes.data, C.byref(ng)), "pai_hip_quantize_f32")
    return q, s[:ng.value]


def dequantize(q: np.ndarray, scales: np.ndarray, n: int, bits: int,
               group_size: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.empty(n, np.float32)
    sch = Scheme(bits, 1, group_size)
    check(lib().pai_hip_dequantize_f32(q.ctypes.data, scales.ctypes.data, n, C.byref(sch),
                                       out.ctypes.data), "pai_hip_dequantize_f32")
    return out
