"""prosperoai_amd — MI355X (gfx950) quantized-weights matmul behind
ProsperoAI's C operator interface.

The product is the C-ABI library prosperoai_amd/lib/libpai_hip.so
(include/pai_hip.h, include/paiq.h). This package only binds it for tests
and benchmarks.
"""
from ._lib import LIB_PATH, PaiError, check, lib
from .gguf import GGUFDir, TensorInfo
from . import v0
from .qmat import (BLOCK_BYTES, BLOCK_ELEMS, FLAG_DEVICE_PTRS, FLAG_FP32, FLAG_MFMA_BF16,
                   MFMA_MIN_M, Q4_0, Q4_K, Q6_K, Q8_0, QTYPES, QMat, descriptors,
                   gate_up_async, gemm_multi_async, gemm_run, gemm_shape_check, init,
                   normal_f32, qtype_bytes, quantize, set_tuning, tuning)

__all__ = [
    "LIB_PATH", "PaiError", "check", "lib", "BLOCK_BYTES", "BLOCK_ELEMS", "FLAG_DEVICE_PTRS",
    "FLAG_FP32", "FLAG_MFMA_BF16", "MFMA_MIN_M", "Q4_0", "Q4_K", "Q6_K", "Q8_0", "QTYPES",
    "QMat", "GGUFDir", "TensorInfo", "descriptors", "gate_up_async", "gemm_multi_async", "gemm_run",
    "gemm_shape_check", "init",
    "normal_f32", "qtype_bytes", "quantize", "set_tuning", "tuning", "v0",
]
