"""ctypes binding of libpai_hip.so (the C-ABI declared in include/pai_hip.h
and include/paiq.h). Loading never falls back to anything: a missing or
unloadable library raises."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libpai_hip.so"

# sdk/include/pai/error.h:13-23
STATUS_NAMES = {
    0: "PAI_OK", -1: "PAI_ERR_INVALID_ARG", -2: "PAI_ERR_NOMEM",
    -3: "PAI_ERR_UNSUPPORTED", -4: "PAI_ERR_CAPABILITY", -5: "PAI_ERR_TIMEOUT",
    -6: "PAI_ERR_MISMATCH", -7: "PAI_ERR_IO", -8: "PAI_ERR_INIT",
    -9: "PAI_ERR_INTERNAL", -10: "PAI_ERR_PROTOCOL",
}

# Every symbol the headers declare, with its ctypes signature.
_u8p, _f32p, _vp = C.c_void_p, C.POINTER(C.c_float), C.c_void_p
SIGNATURES = {
    # pai_hip.h
    "pai_hip_init": (C.c_int32, []),
    "pai_hip_shutdown": (C.c_int32, []),
    "pai_hip_last_error": (C.c_char_p, []),
    "pai_hip_set_tuning": (C.c_int32, [C.c_uint32, C.c_int32]),
    "pai_qtype_bytes": (C.c_uint64, [C.c_uint32, C.c_uint64]),
    "pai_qmat_upload": (C.c_int32, [C.POINTER(C.c_void_p), C.c_uint32, C.c_uint64,
                                    C.c_uint64, _vp, C.c_uint64]),
    "pai_qmat_upload_device": (C.c_int32, [C.POINTER(C.c_void_p), C.c_uint32, C.c_uint64,
                                           C.c_uint64, _vp, C.c_uint64, _vp]),
    "pai_qmat_free": (C.c_int32, [_vp]),
    "pai_qmat_shape": (C.c_int32, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                   C.POINTER(C.c_uint64)]),
    "pai_qmat_bytes": (C.c_uint64, [_vp]),
    "pai_qgemm_f32": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, C.c_uint32]),
    "pai_qgemm_f32_async": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, C.c_uint32, _vp]),
    "pai_qgemm_f32_noalloc_async": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, C.c_uint32, _vp]),
    "pai_qgemm_f32_multi_async": (C.c_int32, [C.POINTER(C.c_void_p), C.c_uint32, C.c_uint64, _vp,
                                              C.POINTER(C.c_void_p), C.c_uint32, _vp]),
    "pai_qgemm_f32_gate_up_async": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, _vp, C.c_uint32,
                                                _vp]),
    "pai_qdequant_f32": (C.c_int32, [_vp, _vp, C.c_uint32]),
    "pai_gguf_dir_open": (C.c_int32, [_vp, C.c_uint64, C.POINTER(C.c_void_p)]),
    "pai_gguf_dir_close": (None, [_vp]),
    "pai_gguf_dir_count": (C.c_uint64, [_vp]),
    "pai_gguf_dir_layout": (C.c_int32, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                        C.POINTER(C.c_uint64)]),
    "pai_gguf_dir_tensor": (C.c_int32, [_vp, C.c_uint64, C.POINTER(C.c_char_p),
                                        C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                        C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "pai_gguf_dir_find": (C.c_int32, [_vp, C.c_char_p, C.POINTER(C.c_uint64)]),
    "pai_gguf_dir_blocks": (C.c_int32, [_vp, C.c_uint64, C.POINTER(C.c_void_p),
                                        C.POINTER(C.c_uint64)]),
    "pai_qmat_upload_gguf": (C.c_int32, [C.POINTER(C.c_void_p), _vp, C.c_char_p]),
    "pai_qgemm_ref_f32": (C.c_int32, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64, _vp, _vp,
                                      _vp]),
    "pai_hip_gemm_w8_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_hip_gemm_w4_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_hip_gemm_wq_f32_async": (C.c_int32, [C.c_uint32] + [C.c_uint64] * 3 + [_vp] * 3 +
                                  [C.c_uint64, _vp, _vp, C.c_uint64, _vp]),
    "pai_hip_quantize_f32": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, _vp, _vp]),
    "pai_hip_dequantize_f32": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, _vp]),
    "pai_hip_quantize_f32_async": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, _vp, _vp, _vp]),
    "pai_hip_dequantize_f32_async": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, _vp, _vp]),
    "pai_gemm_w8_ref_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_gemm_w4_ref_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    # pai_pai64.h
    "pai64_crc32": (C.c_uint32, [C.c_uint32, _vp, C.c_uint64]),
    "pai64_write_file": (C.c_int32, [C.c_char_p, _vp, C.c_uint32, C.POINTER(C.c_uint64)]),
    "pai64_open": (C.c_int32, [_vp, C.c_uint64, _vp]),
    "pai64_section": (C.c_void_p, [_vp, C.c_uint32, C.POINTER(C.c_uint64)]),
    "pai64_verify_section": (C.c_int32, [_vp, C.c_uint32]),
    "pai64_map_file": (C.c_int32, [C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
    "pai64_unmap_file": (C.c_int32, [_vp, C.c_uint64]),
    "pai64_manifest_bytes": (C.c_uint64, [_vp, C.c_uint32]),
    "pai64_manifest_encode": (C.c_int32, [_vp, C.c_uint32, _vp, C.c_uint64,
                                          C.POINTER(C.c_uint64)]),
    "pai64_manifest_decode": (C.c_int32, [_vp, C.c_uint64, _vp, C.c_uint32,
                                          C.POINTER(C.c_uint32)]),
    "pai64_qmat_upload": (C.c_int32, [_vp, _vp, C.POINTER(C.c_void_p)]),
    "pai64_tok_bytes": (C.c_uint64, [_vp, C.c_uint32, C.c_uint32]),
    "pai64_tok_encode": (C.c_int32, [_vp, _vp, C.c_uint32, _vp, C.c_uint32, _vp, C.c_uint64,
                                     C.POINTER(C.c_uint64)]),
    "pai64_tok_index": (C.c_int32, [_vp, C.c_uint64, C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint32), _vp, C.c_uint32,
                                    C.POINTER(C.c_uint64)]),
    "pai_qgemm_shape_check": (C.c_int32, [C.c_int, C.c_uint32, _vp, C.c_uint32, _vp,
                                          C.c_uint32, _vp, C.c_uint64, C.c_uint64,
                                          C.POINTER(C.c_uint64)]),
    "pai_qgemm_run": (C.c_int32, [_vp, C.c_int, C.c_uint32, _vp, C.c_uint32, _vp, C.c_uint32,
                                  _vp, _vp, _vp, C.c_uint32]),
    "pai_hip_quant_tag": (C.c_int32, [C.c_uint32, _vp]),
    "pai_hip_quant_type": (C.c_uint32, [_vp]),
    "pai_hip_op_descriptors": (C.c_void_p, [C.POINTER(C.c_uint32)]),
    "pai_hip_op_name": (C.c_char_p, [C.c_uint32]),
    # pai_llama.h
    "pai_rmsnorm_f32_async": (C.c_int32, [_vp, _vp, _vp, _vp, C.c_uint64, C.c_float, _vp]),
    "pai_qgemv_rmsnorm_f32_async": (C.c_int32, [_vp, C.c_uint32, _vp, _vp, C.c_float, _vp, _vp]),
    "pai_qgemv_rmsnorm_gate_up_async": (C.c_int32, [_vp, _vp, _vp, _vp, C.c_float, _vp, _vp]),
    "pai_qgemv_add_f32_async": (C.c_int32, [_vp, _vp, _vp, _vp]),
    "pai_rope_kv_append_async": (C.c_int32, [_vp] * 8 + [C.c_uint32] * 6 + [_vp]),
    "pai_attention_workspace_bytes": (C.c_uint64, [C.c_uint32] * 3),
    "pai_attention_decode_async": (C.c_int32, [_vp] * 5 + [C.c_uint32] * 5 + [_vp]),
    "pai_attention_decode_rope_async": (C.c_int32, [_vp] * 5 + [C.c_uint32] + [_vp] * 4
                                        + [C.c_uint32] * 5 + [_vp]),
    "pai_argmax_workspace_bytes": (C.c_uint64, []),
    "pai_argmax_f32_async": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, _vp]),
    "pai_llama_create": (C.c_int32, [C.POINTER(C.c_void_p), _vp]),
    "pai_llama_free": (None, [_vp]),
    "pai_llama_set_layer": (C.c_int32, [_vp, C.c_uint32] + [_vp] * 9),
    "pai_llama_set_output": (C.c_int32, [_vp] * 4),
    "pai_llama_kv_write": (C.c_int32, [_vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp]),
    "pai_llama_decode": (C.c_int32, [_vp, C.c_uint32, C.c_uint32, _vp, _vp]),
    "pai_llama_decode_async": (C.c_int32, [_vp, _vp, C.c_uint32, _vp, _vp]),
    "pai_llama_logits": (C.c_void_p, [_vp]),
    "pai_llama_kv_cache": (C.c_int32, [_vp, C.c_uint32, C.POINTER(C.c_void_p),
                                       C.POINTER(C.c_void_p)]),
    # paiq.h
    "paiq_quantize": (C.c_int32, [C.c_uint32, _vp, C.c_uint64, C.c_uint64, _vp, C.c_uint64,
                                  C.c_int]),
    "paiq_f32_to_f16": (C.c_uint16, [C.c_float]),
    "paiq_f16_to_f32": (C.c_float, [C.c_uint16]),
    "paiq_normal_f32": (None, [C.c_uint64, C.c_float, C.c_float, _vp, C.c_uint64]),
}


class PaiError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str = ""):
        self.status = status
        name = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{where}: {name}" + (f" ({detail})" if detail else ""))


class HipDescriptor(C.Structure):
    """Field-for-field mirror of pai_hip_op_descriptor_t / pai_op_descriptor_t."""
    _fields_ = [("name", C.c_char_p), ("version", C.c_uint32), ("num_inputs", C.c_uint32),
                ("num_outputs", C.c_uint32), ("in_dtype", C.c_int32),
                ("out_dtype", C.c_int32), ("caps", C.c_uint32), ("ref_fn", C.c_void_p),
                ("kernel_id", C.c_int32), ("reserved", C.c_uint32 * 2)]


_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run python -m prosperoai_amd.build")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int, where: str) -> None:
    if status != 0:
        detail = lib().pai_hip_last_error().decode(errors="replace")
        raise PaiError(status, where, detail)
