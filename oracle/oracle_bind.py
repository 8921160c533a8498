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
    "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
    "orc_rmsnorm_gamma_f32": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, C.c_float]),
    "orc_rope_f32": (C.c_int32, [_vp] + [C.c_uint64] * 4 + [_vp, _vp, C.c_uint64, _vp]),
    "orc_rope_tables_llama": (None, [C.c_uint32] * 3 + [C.c_float, _vp, _vp]),
    "orc_attention_f32": (C.c_int32, [C.c_uint64] * 4 + [_vp] * 4),
    "orc_attention_last_f32": (C.c_int32, [C.c_uint64] * 5 + [_vp] * 4),
    "orc_argmax_first": (C.c_uint32, [_vp, C.c_uint64]),
    "orc_llama_step": (C.c_int32, [_vp, C.c_uint32, C.c_uint32, _vp, _vp]),
    "orc_quant_group_size": (C.c_int32, [_vp, C.c_uint64, _vp]),
    "orc_quant_num_groups": (C.c_uint64, [C.c_uint64, _vp]),
    "orc_quant_value_bytes": (C.c_uint64, [C.c_uint64, _vp]),
    "orc_quantize_v0_f32": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, _vp, _vp]),
    "orc_dequantize_v0_f32": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, _vp]),
    "orc_gemm_wq_seq_f32": (C.c_int32, [C.c_uint32] + [C.c_uint64] * 3 + [_vp] * 3 +
                            [C.c_uint64, _vp]),
    "orc_gemm_wq_f64": (C.c_int32, [C.c_uint32] + [C.c_uint64] * 3 + [_vp] * 3 +
                        [C.c_uint64, _vp]),
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
    "pai_ref_vecadd_f32": (C.c_int32, [_vp, _vp, _vp, C.c_uint64]),
    "pai_ref_rmsnorm_gamma_f32": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, C.c_float]),
    "pai_ref_rope_f32": (C.c_int32, [_vp] + [C.c_uint64] * 4 + [_vp, _vp, C.c_uint64, _vp]),
    "pai_ref_attention_f32": (C.c_int32, [C.c_uint64] * 4 + [_vp] * 4),
    "pai_opt_gemv_f32": (C.c_int32, [C.c_uint64, C.c_uint64, _vp, _vp, _vp]),
    "pai_opt_gemm_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3),
    "pai_opt_gemm_w8_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_opt_backend_name": (C.c_char_p, []),
    "pai_ref_gemm_w8_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_ref_gemm_w4_f32": (C.c_int32, [C.c_uint64] * 3 + [_vp] * 3 + [C.c_uint64, _vp]),
    "pai_quant_scheme_check": (C.c_int32, [_vp]),
    "pai_quant_num_groups": (C.c_uint64, [C.c_uint64, _vp]),
    "pai_quant_value_bytes": (C.c_uint64, [C.c_uint64, _vp]),
    "pai_quant_scale_bytes": (C.c_uint64, [C.c_uint64, _vp]),
    "pai_quant_weights_bytes": (C.c_uint64, [C.c_uint64, _vp]),
    "pai_quantize_f32": (C.c_int32, [_vp, C.c_uint64, _vp, _vp, _vp, _vp]),
    "pai_dequantize_f32": (C.c_int32, [_vp, _vp, C.c_uint64, _vp, _vp]),
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


class QuantScheme(C.Structure):
    """The v0 scheme record (models/quantize.h:36-40)."""
    _fields_ = [("bit_width", C.c_uint8), ("is_signed", C.c_uint8), ("group_size", C.c_uint16)]


def v0_value_bytes(n: int, bits: int) -> int:
    return (n + 1) // 2 if bits == 4 else n


def v0_num_groups(n: int, group_size: int) -> int:
    gs = n if group_size == 0 else group_size
    return -(-n // gs)


def v0_quantize(x: np.ndarray, bits: int, group_size: int, lib=None):
    """orc_quantize_v0_f32 (or the reference build's pai_quantize_f32 when
    `lib` is ref()): packed codes (int8) and one f32 scale per group."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    sch = QuantScheme(bits, 1, group_size)
    q = np.empty(v0_value_bytes(x.size, bits), np.int8)
    sc = np.empty(v0_num_groups(x.size, group_size), np.float32)
    ng = C.c_uint64(0)
    fn = lib.pai_quantize_f32 if lib is not None else oracle().orc_quantize_v0_f32
    _check(fn(_p(x), x.size, C.byref(sch), _p(q), _p(sc), C.byref(ng)), "v0 quantize")
    assert ng.value == sc.size
    return q, sc


def v0_dequantize(q: np.ndarray, scales: np.ndarray, n: int, bits: int, group_size: int,
                  lib=None) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    sch = QuantScheme(bits, 1, group_size)
    out = np.empty(n, np.float32)
    fn = lib.pai_dequantize_f32 if lib is not None else oracle().orc_dequantize_v0_f32
    _check(fn(_p(q), _p(scales), n, C.byref(sch), _p(out)), "v0 dequantize")
    return out


def gemm_wq_seq(bits: int, a: np.ndarray, w_q: np.ndarray, scales: np.ndarray, n: int,
                group_size: int, lib=None) -> np.ndarray:
    """c = a . dequant(W) with W [K][N] codes (int8, or nibbles over the flat
    index t*n+j) and scales [G][N]: the reference's sequential f32 sum
    (orc_gemm_wq_seq_f32, or pai_ref_gemm_w8_f32 / _w4_f32 of the reference
    build when `lib` is ref())."""
    a = _f32(a)
    m, k = a.shape
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    scales = _f32(scales)
    c = np.empty((m, n), np.float32)
    if lib is not None:
        fn = lib.pai_ref_gemm_w8_f32 if bits == 8 else lib.pai_ref_gemm_w4_f32
        st = fn(m, n, k, _p(a), _p(w_q), _p(scales), group_size, _p(c))
    else:
        st = oracle().orc_gemm_wq_seq_f32(bits, m, n, k, _p(a), _p(w_q), _p(scales), group_size,
                                          _p(c))
    _check(st, "gemm_wq_seq")
    return c


def gemm_wq_f64(bits: int, a: np.ndarray, w_q: np.ndarray, scales: np.ndarray, n: int,
                group_size: int) -> np.ndarray:
    a = _f32(a)
    m, k = a.shape
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    scales = _f32(scales)
    c = np.empty((m, n), np.float64)
    _check(oracle().orc_gemm_wq_f64(bits, m, n, k, _p(a), _p(w_q), _p(scales), group_size, _p(c)),
           "gemm_wq_f64")
    return c


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(st: int, name: str) -> None:
    if st != 0:
        raise RuntimeError(f"{name} status {st}")


def f32_to_f16(v: np.ndarray) -> np.ndarray:
    """orc_f32_to_f16 on every element (binary16 bit patterns)."""
    o = oracle()
    return np.array([o.orc_f32_to_f16(float(x)) for x in _f32(v).ravel()], np.uint16)


def rmsnorm(a: np.ndarray, gamma: np.ndarray, eps: float = 0.0) -> np.ndarray:
    a, gamma = _f32(a), _f32(gamma)
    c = np.empty_like(a)
    _check(oracle().orc_rmsnorm_gamma_f32(_p(a), _p(c), a.size, _p(gamma), eps), "rmsnorm")
    return c


def rope(x: np.ndarray, heads: int, cos_t: np.ndarray, sin_t: np.ndarray, r2: int) -> np.ndarray:
    """x: [seq * heads][hd] position-major; tables [seq][r2]."""
    x, cos_t, sin_t = _f32(x), _f32(cos_t), _f32(sin_t)
    rows, hd = x.shape
    out = np.empty_like(x)
    _check(oracle().orc_rope_f32(_p(x), rows, hd, rows // heads, heads, _p(cos_t), _p(sin_t), r2,
                                 _p(out)), "rope")
    return out


def rope_tables(ctx: int, r2: int, n_rot: int, theta: float):
    c = np.empty((ctx, r2), np.float32)
    s = np.empty((ctx, r2), np.float32)
    oracle().orc_rope_tables_llama(ctx, r2, n_rot, theta, _p(c), _p(s))
    return c, s


def attention(h: int, hk: int, q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """q: [seq][h][hd], k, v: [seq][hk][hd] -> [seq][h][hd] (causal)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    seq, hd = q.shape[0], q.shape[-1]
    out = np.empty_like(q)
    _check(oracle().orc_attention_f32(h, hk, seq, hd, _p(q), _p(k), _p(v), _p(out)), "attention")
    return out


def attention_last(h: int, hk: int, length: int, q: np.ndarray, kc: np.ndarray,
                   vc: np.ndarray) -> np.ndarray:
    """q: [h][hd]; caches [hk][ctx][hd] -> [h][hd] over positions < length."""
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    ctx, hd = kc.shape[1], kc.shape[2]
    out = np.empty((h, hd), np.float32)
    _check(oracle().orc_attention_last_f32(h, hk, ctx, length, hd, _p(q), _p(kc), _p(vc),
                                           _p(out)), "attention_last")
    return out


def argmax_first(x: np.ndarray) -> int:
    x = _f32(x)
    return int(oracle().orc_argmax_first(_p(x), x.size))


class _OrcLlama(C.Structure):
    """orc_llama_t (oracle/oracle.h)."""
    _fields_ = [(n, C.c_uint32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "n_ff",
                                          "vocab", "ctx", "n_rot")] + [
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("w", C.POINTER(C.c_void_p)),
        ("attn_norm", _vp), ("ffn_norm", _vp), ("token_embd", _vp), ("output", _vp),
        ("output_norm", _vp), ("k_cache", _vp), ("v_cache", _vp), ("kv_f16", C.c_int32)]


class LlamaOracle:
    """orc_llama_step over dequantized weights.

    cfg: dict with n_layer, n_embd, n_head, n_head_kv, n_ff, vocab, ctx,
    n_rot, rope_theta, norm_eps. layers: list of dicts with f32 matrices
    q, k, v, o, gate, up, down ([N][K]) and attn_norm, ffn_norm; head: dict
    with token_embd, output ([vocab][n_embd]) and output_norm."""

    def __init__(self, cfg: dict, layers: list, head: dict, kv_f16: bool = True):
        self.cfg = cfg
        hd = cfg["n_embd"] // cfg["n_head"]
        self._keep = []
        ws = []
        for L in layers:
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                a = _f32(L[name])
                self._keep.append(a)
                ws.append(_p(a))
        self._w = (C.c_void_p * len(ws))(*ws)
        self.attn_norm = _f32(np.stack([L["attn_norm"] for L in layers]))
        self.ffn_norm = _f32(np.stack([L["ffn_norm"] for L in layers]))
        self.token_embd = _f32(head["token_embd"])
        self.output = _f32(head["output"])
        self.output_norm = _f32(head["output_norm"])
        shape = (cfg["n_layer"], cfg["n_head_kv"], cfg["ctx"], hd)
        self.k_cache = np.zeros(shape, np.float32)
        self.v_cache = np.zeros(shape, np.float32)
        self._m = _OrcLlama(
            *[cfg[n] for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "n_ff", "vocab", "ctx",
                               "n_rot")],
            cfg["rope_theta"], cfg["norm_eps"], self._w, _p(self.attn_norm), _p(self.ffn_norm),
            _p(self.token_embd), _p(self.output), _p(self.output_norm), _p(self.k_cache),
            _p(self.v_cache), 1 if kv_f16 else 0)

    def step(self, token: int, pos: int):
        logits = np.empty(self.cfg["vocab"], np.float32)
        nxt = C.c_uint32()
        _check(oracle().orc_llama_step(C.byref(self._m), token, pos, _p(logits), C.byref(nxt)),
               "orc_llama_step")
        return logits, nxt.value


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
