"""Python view of the C-ABI for tests and benchmarks.

Mirrors the reference's operator contract: the C entry points return
pai_status_t and never allocate the caller's buffers; here a non-zero status
raises PaiError carrying the status name and the library's message.
Device buffers, streams and graphs for the device-pointer entry points come
from hipmem (the HIP runtime libpai_hip.so links); every kernel runs
through libpai_hip.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import HipDescriptor, check, lib

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
QTYPES = {"q4_0": Q4_0, "q8_0": Q8_0, "q4_k": Q4_K, "q6_k": Q6_K}
BLOCK_ELEMS = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}

FLAG_DEVICE_PTRS = 1 << 0
FLAG_MFMA_BF16 = 1 << 1
FLAG_FP32 = 1 << 2
MFMA_MIN_M = 8


def qtype_bytes(qtype: int, numel: int) -> int:
    return int(lib().pai_qtype_bytes(qtype, numel))


def normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().paiq_normal_f32(seed & 0xFFFFFFFFFFFFFFFF, mean, std, out.ctypes.data, n)
    return out


def quantize(qtype: int, w: np.ndarray, threads: int = 0) -> np.ndarray:
    """Encode f32 rows [N][K] into native GGUF blocks (uint8 [N][row_bytes])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    rb = qtype_bytes(qtype, k)
    out = np.empty((n, rb), dtype=np.uint8)
    check(lib().paiq_quantize(qtype, w.ctypes.data, n, k, out.ctypes.data, out.nbytes, threads),
          "paiq_quantize")
    return out


def init() -> None:
    check(lib().pai_hip_init(), "pai_hip_init")


# pai_hip_set_tuning knobs (include/pai_hip.h)
TUNE = {"gemm_splits": 1, "gemm_no_x16": 2, "gemm_atomic_splits": 3, "gemv_wgs": 4,
        "gemv_rows": 5, "gemv_nw": 6, "gemv_no_mx": 7, "mfma_min_m": 8, "gemm_tile": 9,
        "v0_sequential": 10}


def set_tuning(name: str, value: int) -> None:
    """Launch-shape override for measurements and tests (0 = shipped dispatch)."""
    check(lib().pai_hip_set_tuning(TUNE[name], int(value)), "pai_hip_set_tuning")


class tuning:
    """Context manager: knobs set on entry, back to 0 on exit."""

    def __init__(self, **knobs):
        self.knobs = knobs

    def __enter__(self):
        for k, v in self.knobs.items():
            set_tuning(k, v)
        return self

    def __exit__(self, *exc):
        for k in self.knobs:
            set_tuning(k, 0)
        return False


def descriptors() -> list[HipDescriptor]:
    count = C.c_uint32(0)
    ptr = lib().pai_hip_op_descriptors(C.byref(count))
    arr = C.cast(ptr, C.POINTER(HipDescriptor))
    return [arr[i] for i in range(count.value)]


class QMat:
    """A packed W[N][K] resident in device memory (pai_qmat_t)."""

    def __init__(self, qtype: int, n: int, k: int, blocks, *, device_ptr: int | None = None,
                 stream: int = 0):
        self.qtype, self.n, self.k = qtype, n, k
        self._h = C.c_void_p()
        if device_ptr is not None:
            nbytes = n * qtype_bytes(qtype, k)
            check(lib().pai_qmat_upload_device(C.byref(self._h), qtype, n, k, device_ptr, nbytes,
                                               stream or None), "pai_qmat_upload_device")
        else:
            b = np.ascontiguousarray(blocks, dtype=np.uint8)
            check(lib().pai_qmat_upload(C.byref(self._h), qtype, n, k, b.ctypes.data, b.nbytes),
                  "pai_qmat_upload")

    @classmethod
    def adopt(cls, handle: C.c_void_p) -> "QMat":
        """Wrap a handle made by another upload entry point (it is freed with the object)."""
        self = cls.__new__(cls)
        self._h = handle
        t, n, k = C.c_uint32(), C.c_uint64(), C.c_uint64()
        check(lib().pai_qmat_shape(handle, C.byref(t), C.byref(n), C.byref(k)), "pai_qmat_shape")
        self.qtype, self.n, self.k = t.value, n.value, k.value
        return self

    @property
    def handle(self) -> int:
        return self._h.value

    @property
    def nbytes(self) -> int:
        return int(lib().pai_qmat_bytes(self._h))

    def free(self) -> None:
        if self._h.value:
            check(lib().pai_qmat_free(self._h), "pai_qmat_free")
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    # ---- host-pointer entry points (synchronous) ----
    def gemm(self, x: np.ndarray, flags: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = x.shape[0] if x.ndim == 2 else 1
        y = np.empty((m, self.n), dtype=np.float32)
        check(lib().pai_qgemm_f32(self._h, m, x.ctypes.data, y.ctypes.data, flags),
              "pai_qgemm_f32")
        return y

    def dequant(self) -> np.ndarray:
        out = np.empty((self.n, self.k), dtype=np.float32)
        check(lib().pai_qdequant_f32(self._h, out.ctypes.data, 0), "pai_qdequant_f32")
        return out

    # ---- device-pointer entry points (raw device addresses, hipStream_t) ----
    def gemm_async(self, x_ptr: int, y_ptr: int, m: int, flags: int = 0, stream: int = 0) -> None:
        check(lib().pai_qgemm_f32_async(self._h, m, x_ptr, y_ptr, flags | FLAG_DEVICE_PTRS,
                                        stream or None), "pai_qgemm_f32_async")


def _shape(dims) -> tuple:
    dims = [int(d) for d in dims]
    return len(dims), (C.c_uint64 * max(len(dims), 1))(*dims)


def gemm_shape_check(is_gemv: bool, a_shape, b_shape, c_shape, w_n: int, w_k: int) -> int:
    """run_gemm's shape rules (scheduler/scheduler.c:280-338) against a
    weight of w_n rows of w_k columns (pai_qgemm_shape_check); returns the
    number of activation rows (tokens), raises PaiError(MISMATCH) where
    run_gemm rejects the shapes."""
    (ar, a), (br, b), (cr, c) = _shape(a_shape), _shape(b_shape), _shape(c_shape)
    m = C.c_uint64(0)
    check(lib().pai_qgemm_shape_check(int(is_gemv), ar, a, br, b, cr, c, w_n, w_k, C.byref(m)),
          "pai_qgemm_shape_check")
    return m.value


def gemm_run(w: QMat, is_gemv: bool, a_shape, b_shape, c_shape, act: np.ndarray) -> np.ndarray:
    """The executor's GEMM/GEMV op on a GGUF weight (pai_qgemm_run, host
    pointers): `act` is the operand that is not the weight; the result has
    the shape of c."""
    (ar, a), (br, b), (cr, c) = _shape(a_shape), _shape(b_shape), _shape(c_shape)
    act = np.ascontiguousarray(act, dtype=np.float32)
    out = np.empty(tuple(int(d) for d in c_shape), dtype=np.float32)
    check(lib().pai_qgemm_run(w.handle, int(is_gemv), ar, a, br, b, cr, c, act.ctypes.data,
                              out.ctypes.data, 0), "pai_qgemm_run")
    return out


def gemm_multi_async(mats: list, x_ptr: int, y_ptrs: list, m: int, flags: int = 0,
                     stream: int = 0) -> None:
    """y_i = x * W_i^T for matrices sharing x, in one fused launch
    (pai_qgemm_f32_multi_async; device pointers)."""
    n = len(mats)
    hs = (C.c_void_p * n)(*[w.handle for w in mats])
    ys = (C.c_void_p * n)(*y_ptrs)
    check(lib().pai_qgemm_f32_multi_async(hs, n, m, x_ptr, ys, flags | FLAG_DEVICE_PTRS,
                                          stream or None), "pai_qgemm_f32_multi_async")


def gate_up_async(w_gate: QMat, w_up: QMat, x_ptr: int, h_ptr: int, m: int, flags: int = 0,
                  stream: int = 0) -> None:
    """h = silu(x W_gate^T) * (x W_up^T) (pai_qgemm_f32_gate_up_async; device pointers)."""
    check(lib().pai_qgemm_f32_gate_up_async(w_gate.handle, w_up.handle, m, x_ptr, h_ptr,
                                            flags | FLAG_DEVICE_PTRS, stream or None),
          "pai_qgemm_f32_gate_up_async")
