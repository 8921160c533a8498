"""ctypes bindings of the CPU checkers (test infrastructure only).

  oracle/liboracle.so        this repository's C restatement of the reference
  oracle/_ref/libpairef.so   the reference's own C sources, compiled from the
                             reference tree by oracle/Makefile (optional: only
                             where that tree was present at build time)
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_PATH = ROOT / "oracle" / "liboracle.so"
REF_PATH = ROOT / "oracle" / "_ref" / "libpairef.so"

_vp = C.c_void_p
_ORACLE_SIGS = {
    "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_f16_to_f32_bits": (None, [_vp, _vp, C.c_uint64]),
    "orc_scale_min_k4": (None, [C.c_int, _vp, _vp, _vp]),
    "orc_type_bytes": (C.c_uint64, [C.c_uint32, C.c_uint64]),
    "orc_dequant": (C.c_int32, [C.c_uint32, _vp, _vp, C.c_uint64]),
    "orc_gemm_seq_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3),
    "orc_qgemm_seq_f32": (C.c_int32, [C.c_uint32, C.c_uint64, C.c_uint64, _vp, C.c_uint64, _vp,
                                      _vp]),
    "orc_qgemm_f64": (C.c_int32, [C.c_uint32, C.c_uint64, C.c_uint64, _vp, C.c_uint64, _vp,
                                  _vp]),
    "orc_compare_f32": (C.c_int32, [_vp, _vp, C.c_uint64, C.c_float, C.c_float, _vp]),
    "orc_silu_mul_f32": (C.c_int32, [_vp, _vp, _vp, C.c_uint64]),
    "orc_opt_gemv_avx2": (C.c_int32, [C.c_uint64, C.c_uint64, _vp, _vp, _vp]),
    "orc_opt_gemv_avx2_mt": (C.c_int32, [C.c_uint64, C.c_uint64, _vp, _vp, _vp, C.c_int]),
    "orc_opt_gemm_avx2": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3),
    "orc_opt_gemm_w8_avx2": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "orc_q8_0_encode_ref": (None, [_vp, _vp, C.c_uint64]),
    "orc_q4_0_encode_ref": (None, [_vp, _vp, C.c_uint64]),
}

_REF_SIGS = {
    "pai_gguf_open": (C.c_int32, [_vp, C.c_uint64, _vp]),
    "pai_gguf_close": (None, [_vp]),
    "pai_gguf_find_tensor": (C.c_void_p, [_vp, C.c_char_p]),
    "pai_gguf_dequant": (C.c_int32, [_vp, _vp, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
    "pai_gguf_type_bytes": (C.c_uint64, [C.c_uint32, C.c_uint64]),
    "pai_ref_gemm_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3),
    "pai_ref_silu_f32": (C.c_int32, [_vp, _vp, C.c_uint64]),
    "pai_ref_vecmul_f32": (C.c_int32, [_vp, _vp, _vp, C.c_uint64]),
    "pai_opt_gemv_f32": (C.c_int32, [C.c_uint64, C.c_uint64, _vp, _vp, _vp]),
    "pai_opt_gemm_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3),
    "pai_opt_gemm_w8_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_opt_backend_name": (C.c_char_p, []),
    "pai_op_registry_init": (C.c_int32, [_vp]),
    "pai_op_registry_builtin": (C.c_int32, [_vp]),
    "pai_op_registry_register": (C.c_int32, [_vp, _vp]),
    "pai_op_registry_lookup": (C.c_void_p, [_vp, C.c_char_p]),
    "pai_op_registry_count": (C.c_uint32, [_vp]),
    "pai_op_supports": (C.c_uint32, [_vp, C.c_uint32]),
}

_oracle = None
_ref = None
_libc = C.CDLL(None)
_libc.free.argtypes = [_vp]


def _bind(path: Path, sigs: dict) -> C.CDLL:
    h = C.CDLL(str(path))
    for name, (res, args) in sigs.items():
        fn = getattr(h, name)
        fn.restype, fn.argtypes = res, args
    return h


def oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_PATH.exists():
            raise RuntimeError(f"{ORACLE_PATH} missing; run make -C oracle")
        _oracle = _bind(ORACLE_PATH, _ORACLE_SIGS)
    return _oracle


def ref():
    """The reference-built checker, or None when it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        _ref = _bind(REF_PATH, _REF_SIGS)
    return _ref


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------- oracle wrappers
def f16_bits(h: np.ndarray) -> np.ndarray:
    """orc_f16_to_f32 on every element, as raw f32 bit patterns."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.uint32)
    oracle().orc_f16_to_f32_bits(_p(h), _p(out), h.size)
    return out


def dequant(qtype: int, blocks: np.ndarray, numel: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(numel, dtype=np.float32)
    st = oracle().orc_dequant(qtype, _p(b), _p(out), numel)
    if st != 0:
        raise RuntimeError(f"orc_dequant status {st}")
    return out


def qgemm_seq(qtype: int, n: int, k: int, blocks: np.ndarray, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    st = oracle().orc_qgemm_seq_f32(qtype, n, k, _p(b), x.shape[0], _p(x), _p(y))
    if st != 0:
        raise RuntimeError(f"orc_qgemm_seq_f32 status {st}")
    return y


def qgemm_f64(qtype: int, n: int, k: int, blocks: np.ndarray, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty((x.shape[0], n), dtype=np.float64)
    st = oracle().orc_qgemm_f64(qtype, n, k, _p(b), x.shape[0], _p(x), _p(y))
    if st != 0:
        raise RuntimeError(f"orc_qgemm_f64 status {st}")
    return y


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    st = oracle().orc_silu_mul_f32(_p(g), _p(u), _p(h), g.size)
    if st != 0:
        raise RuntimeError(f"orc_silu_mul_f32 status {st}")
    return h


# ---------------------------------------------------------------- reference wrappers
def gguf_image(qtype: int, dims: tuple, raw: bytes) -> bytes:
    """A one-tensor GGUF v3 file image (name "t", dims innermost first,
    default 32-byte alignment, no metadata), the layout
    adapters/llama/gguf.c:127-245 parses."""
    name = b"t"
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0)
    info = (struct.pack("<Q", len(name)) + name + struct.pack("<I", len(dims))
            + b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", qtype, 0))
    head = hdr + info
    pad = (-len(head)) % 32
    return head + b"\0" * pad + bytes(raw)


def ref_dequant(qtype: int, raw: bytes, numel: int, row: int | None = None) -> np.ndarray:
    """pai_gguf_dequant from the reference build on one tensor of raw blocks
    (2-D [numel/row][row] when `row` is given)."""
    r = ref()
    dims = (numel,) if row is None else (row, numel // row)
    img = gguf_image(qtype, dims, raw)
    buf = C.create_string_buffer(img, len(img))
    f = C.create_string_buffer(256)  # pai_gguf_t is 72 bytes
    st = r.pai_gguf_open(buf, len(img), f)
    if st != 0:
        raise RuntimeError(f"pai_gguf_open status {st}")
    try:
        t = r.pai_gguf_find_tensor(f, b"t")
        out = C.c_void_p()
        n = C.c_uint64()
        st = r.pai_gguf_dequant(f, t, C.byref(out), C.byref(n))
        if st != 0:
            raise RuntimeError(f"pai_gguf_dequant status {st}")
        arr = np.ctypeslib.as_array(C.cast(out, C.POINTER(C.c_float)), shape=(n.value,)).copy()
        _libc.free(out)
        return arr
    finally:
        r.pai_gguf_close(f)


class RefGGUFTensor(C.Structure):
    """pai_gguf_tensor_t (adapters/llama/gguf.h:54-60)."""
    _fields_ = [("name", C.c_char * 128), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("type", C.c_uint32), ("offset", C.c_uint64)]


class RefGGUF(C.Structure):
    """pai_gguf_t (adapters/llama/gguf.h:62-73)."""
    _fields_ = [("data", C.c_void_p), ("size", C.c_uint64), ("version", C.c_uint32),
                ("tensor_count", C.c_uint64), ("kv_count", C.c_uint64),
                ("alignment", C.c_uint64), ("kv_start", C.c_void_p),
                ("data_start", C.c_void_p), ("tensors", C.POINTER(RefGGUFTensor))]


def ref_gguf_directory(img: bytes):
    """pai_gguf_open from the reference build on a file image. Returns
    (status, layout, tensors): layout = (version, alignment, data_start
    offset); tensors = [(name, type, n_dims, dims, offset)]."""
    r = ref()
    buf = C.create_string_buffer(bytes(img), max(len(img), 1))
    f = RefGGUF()
    st = r.pai_gguf_open(buf, len(img), C.byref(f))
    if st != 0:
        return st, None, None
    try:
        base = C.addressof(buf)
        layout = (f.version, f.alignment, f.data_start - base)
        ts = []
        for i in range(f.tensor_count):
            t = f.tensors[i]
            ts.append((t.name.decode(errors="surrogateescape"), t.type, t.n_dims, tuple(t.dims), t.offset))
        return st, layout, ts
    finally:
        r.pai_gguf_close(C.byref(f))


def ref_gguf_dequant_status(img: bytes, name: str) -> int:
    """Status of pai_gguf_dequant for tensor `name` of a file image the
    reference opens."""
    r = ref()
    buf = C.create_string_buffer(bytes(img), max(len(img), 1))
    f = RefGGUF()
    st = r.pai_gguf_open(buf, len(img), C.byref(f))
    if st != 0:
        raise RuntimeError(f"pai_gguf_open status {st}")
    try:
        t = r.pai_gguf_find_tensor(C.byref(f), name.encode())
        if not t:
            raise RuntimeError(f"no tensor {name}")
        out, n = C.c_void_p(), C.c_uint64()
        st = r.pai_gguf_dequant(C.byref(f), t, C.byref(out), C.byref(n))
        if out.value:
            _libc.free(out)
        return st
    finally:
        r.pai_gguf_close(C.byref(f))
