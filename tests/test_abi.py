"""C-ABI surface checks that need no GPU: the library loads, exports every
function include/*.h declares, validates arguments before touching a
device, and its registry descriptors plug into the reference's registry."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import prosperoai_amd as pa
from prosperoai_amd._lib import SIGNATURES, HipDescriptor

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(pai\w+|paiq\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = pa.lib()
    declared = declared_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    # and the Python binding covers exactly the declared set
    assert declared == set(SIGNATURES)


def test_status_codes_match_reference_values():
    text = (ROOT / "include" / "pai_hip.h").read_text()
    want = {"PAI_OK": 0, "PAI_ERR_INVALID_ARG": -1, "PAI_ERR_NOMEM": -2,
            "PAI_ERR_UNSUPPORTED": -3, "PAI_ERR_CAPABILITY": -4, "PAI_ERR_TIMEOUT": -5,
            "PAI_ERR_MISMATCH": -6, "PAI_ERR_IO": -7, "PAI_ERR_INIT": -8,
            "PAI_ERR_INTERNAL": -9, "PAI_ERR_PROTOCOL": -10}
    for name, v in want.items():
        assert re.search(rf"#define {name} {v}\b", text), name


def test_qtype_bytes_matches_oracle(orc):
    o = orc.oracle()
    for t in (2, 8, 12, 14, 0, 1, 13, 15):
        for numel in (0, 1, 31, 32, 96, 256, 4096, 14336, 1 << 33):
            assert pa.qtype_bytes(t, numel) == o.orc_type_bytes(t, numel)


def test_argument_errors_before_device():
    lib = pa.lib()
    h = C.c_void_p()
    blocks = np.zeros(18 * 4, np.uint8)
    # NULL out / NULL blocks
    assert lib.pai_qmat_upload(None, 2, 4, 32, blocks.ctypes.data, blocks.nbytes) == -1
    assert lib.pai_qmat_upload(C.byref(h), 2, 4, 32, None, blocks.nbytes) == -1
    # zero dims, unsupported type, ragged K, size mismatch
    assert lib.pai_qmat_upload(C.byref(h), 2, 0, 32, blocks.ctypes.data, 0) == -1
    assert lib.pai_qmat_upload(C.byref(h), 3, 4, 32, blocks.ctypes.data, blocks.nbytes) == -3
    assert lib.pai_qmat_upload(C.byref(h), 12, 4, 32, blocks.ctypes.data, blocks.nbytes) == -3
    assert lib.pai_qmat_upload(C.byref(h), 2, 4, 32, blocks.ctypes.data, 71) == -6
    assert h.value is None
    # compute entry points on NULL handles
    x = np.zeros(32, np.float32)
    assert lib.pai_qgemm_f32(None, 1, x.ctypes.data, x.ctypes.data, 0) == -1
    assert lib.pai_qgemm_f32_async(None, 1, x.ctypes.data, x.ctypes.data, 0, None) == -1
    assert lib.pai_qdequant_f32(None, x.ctypes.data, 0) == -1
    assert lib.pai_qmat_free(None) == 0
    hs = (C.c_void_p * 1)(None)
    ys = (C.c_void_p * 1)(x.ctypes.data)
    assert lib.pai_qgemm_f32_multi_async(None, 1, 1, x.ctypes.data, ys, 1, None) == -1
    assert lib.pai_qgemm_f32_multi_async(hs, 1, 1, x.ctypes.data, ys, 1, None) == -1
    assert lib.pai_qgemm_f32_multi_async(hs, 0, 1, x.ctypes.data, ys, 1, None) == -1
    assert lib.pai_qgemm_f32_multi_async(hs, 5, 1, x.ctypes.data, ys, 1, None) == -1
    assert lib.pai_qmat_bytes(None) == 0
    assert b"NULL" in lib.pai_hip_last_error() or lib.pai_hip_last_error() != b""


def test_descriptors_layout_and_names():
    ds = pa.descriptors()
    assert [d.name.decode() for d in ds] == ["qgemm_q4_0_f32", "qgemm_q8_0_f32",
                                             "qgemm_q4_k_f32", "qgemm_q6_k_f32",
                                             "qgemm_w8_f32", "qgemm_w4_f32"]
    twins = [pa.lib().pai_qgemm_ref_f32] * 4 + [pa.lib().pai_gemm_w8_ref_f32,
                                                pa.lib().pai_gemm_w4_ref_f32]
    for d, twin in zip(ds, twins):
        assert d.caps == (1 << 0) | (1 << 3) and d.num_outputs == 1
        assert d.num_inputs == (3 if d.name.startswith(b"qgemm_w") else 2)
        # each descriptor's reference function is its CPU twin
        assert d.ref_fn == C.cast(twin, C.c_void_p).value
        assert d.kernel_id == 0 and d.in_dtype == 0
    # pai_op_descriptor_t is 56 bytes on LP64 (sdk/include/pai/op.h:71-82)
    assert C.sizeof(HipDescriptor) == 56
    assert HipDescriptor.ref_fn.offset == 32 and HipDescriptor.kernel_id.offset == 40
    for t, name in ((2, b"qgemm_q4_0_f32"), (8, b"qgemm_q8_0_f32"), (12, b"qgemm_q4_k_f32"),
                    (14, b"qgemm_q6_k_f32"), (3, None)):
        assert pa.lib().pai_hip_op_name(t) == name


def test_descriptors_register_into_reference_registry(ref_lib):
    """Our descriptors, passed by pointer to the reference's own
    pai_op_registry_register, resolve by name and advertise the HIP and
    CPU-reference caps (the executor's plan check requires the latter)."""
    reg = C.create_string_buffer(8 + 8 * 64)  # pai_op_registry_t
    assert ref_lib.pai_op_registry_builtin(reg) == 0
    base = ref_lib.pai_op_registry_count(reg)
    count = C.c_uint32()
    ptr = pa.lib().pai_hip_op_descriptors(C.byref(count))
    for i in range(count.value):
        assert ref_lib.pai_op_registry_register(reg, ptr + i * C.sizeof(HipDescriptor)) == 0
    assert ref_lib.pai_op_registry_count(reg) == base + count.value
    for name in (b"qgemm_q4_0_f32", b"qgemm_q8_0_f32", b"qgemm_q4_k_f32", b"qgemm_q6_k_f32",
                 b"qgemm_w8_f32", b"qgemm_w4_f32"):
        d = ref_lib.pai_op_registry_lookup(reg, name)
        assert d is not None
        assert ref_lib.pai_op_supports(d, 1 << 3) == 1
        assert ref_lib.pai_op_supports(d, 1 << 0) == 1
    assert ref_lib.pai_op_registry_lookup(reg, b"matmul_f32") is not None


def test_init_without_gpu_reports_init_error():
    """On a host without a gfx950 device, init fails cleanly (no abort)."""
    import torch
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    assert pa.lib().pai_hip_init() == -8
    x = np.zeros((1, 32), np.float32)
    h = C.c_void_p()
    blocks = np.zeros(18, np.uint8)
    assert pa.lib().pai_qmat_upload(C.byref(h), 2, 1, 32, blocks.ctypes.data, 18) == -8


def test_decode_entry_points_reject_bad_arguments_before_device():
    """pai_llama.h: shape and argument errors come back before any device
    work (these run without a GPU)."""
    from prosperoai_amd.llama import LlamaConfig
    lib = pa.lib()
    fake = C.c_void_p(0x1000)  # never dereferenced: validation fails first
    h = C.c_void_p()
    base = dict(n_layer=1, n_embd=256, n_head=4, n_head_kv=2, n_ff=512, vocab=100, ctx=8, n_rot=0,
                rope_theta=0.0, norm_eps=0.0)
    for change, want in (({"n_head_kv": 3}, -1), ({"n_embd": 384, "n_head": 4}, -3),
                         ({"n_head": 16, "n_head_kv": 1, "n_embd": 1024}, -3), ({"ctx": 0}, -1),
                         ({"n_embd": 20480, "n_head": 160, "n_head_kv": 20}, -3)):
        cfg = LlamaConfig(**{**base, **change})
        assert lib.pai_llama_create(C.byref(h), C.byref(cfg)) == want, change
    assert lib.pai_llama_create(None, None) == -1
    # attention: head size, GQA ratio, length
    assert lib.pai_attention_decode_async(fake, fake, fake, fake, fake, 8, 2, 100, 64, 8, None) == -3
    assert lib.pai_attention_decode_async(fake, fake, fake, fake, fake, 8, 3, 64, 64, 8, None) == -1
    assert lib.pai_attention_decode_async(fake, fake, fake, fake, fake, 32, 2, 64, 64, 8, None) == -3
    assert lib.pai_attention_decode_async(fake, fake, fake, fake, fake, 8, 2, 64, 64, 65, None) == -1
    assert lib.pai_attention_decode_async(fake, fake, fake, fake, fake, 8, 2, 64, 64, 0, None) == -1
    # rope: position outside the cache, rotation wider than the head
    args = [fake] * 8
    assert lib.pai_rope_kv_append_async(*args, 4, 2, 64, 32, 16, 16, None) == -1
    assert lib.pai_rope_kv_append_async(*args, 4, 2, 64, 40, 16, 0, None) == -3
    assert lib.pai_rope_kv_append_async(*args, 4, 2, 512, 32, 16, 0, None) == -3
    # fused norm / residual projections: NULL arguments and matrix counts
    assert lib.pai_qgemv_rmsnorm_f32_async(None, 1, fake, fake, 0.0, fake, None) == -1
    assert lib.pai_qgemv_rmsnorm_f32_async(fake, 0, fake, fake, 0.0, fake, None) == -1
    assert lib.pai_qgemv_rmsnorm_f32_async(fake, 4, fake, fake, 0.0, fake, None) == -1
    assert lib.pai_qgemv_rmsnorm_gate_up_async(None, fake, fake, fake, 0.0, fake, None) == -1
    assert lib.pai_qgemv_add_f32_async(None, fake, fake, None) == -1
    assert lib.pai_qgemv_add_f32_async(fake, None, fake, None) == -1
    # norm and argmax sizes
    assert lib.pai_rmsnorm_f32_async(fake, None, fake, fake, 0, 0.0, None) == -1
    assert lib.pai_rmsnorm_f32_async(fake, None, fake, fake, 16385, 0.0, None) == -3
    assert lib.pai_argmax_f32_async(fake, 0, fake, fake, None) == -1
    assert lib.pai_attention_workspace_bytes(32, 128, 2048) == 32 * 32 * 130 * 4
    # the fused RoPE + append + attention: position outside the cache, long contexts
    args = [fake] * 5 + [64] + [fake] * 4
    assert lib.pai_attention_decode_rope_async(*args, 8, 2, 128, 64, 64, None) == -1
    assert lib.pai_attention_decode_rope_async(*args, 8, 2, 128, 40000, 39999, None) == -3
