"""A small GGUF writer for tests (little endian; u64 counts, lengths and
extents, as the reference reader expects in every version).

Metadata values are given as (value_type, value) pairs; arrays as
(9, (element_type, [values])). Tensor data is placed at offsets that are
multiples of the alignment, as llama.cpp writes it.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vt: int, v) -> bytes:
    if vt == STR:
        return _str(v)
    if vt == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def build(kv=(), tensors=(), *, version: int = 3, alignment: int = 32,
          data_pad: bytes = b"") -> bytes:
    """kv: [(key, value_type, value)]; tensors: [(name, dims, ggml_type, data_bytes)].
    `alignment` only places the data (write the general.alignment key in kv
    to announce it)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, vt, v in kv:
        out += _str(key) + struct.pack("<I", vt) + _value(vt, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, dims, gt, _), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gt, o)
    out += b"\0" * ((-len(out)) % alignment)
    for (_, _, _, data), o in zip(tensors, offsets):
        out += bytes(data) + b"\0" * ((-len(data)) % alignment)
    return bytes(out) + data_pad


def weight(name: str, qtype: int, blocks: np.ndarray) -> tuple:
    """A 2-D weight entry from native blocks uint8 [N][row_bytes] of W[N][K]."""
    from prosperoai_amd import BLOCK_BYTES, BLOCK_ELEMS
    n, rb = blocks.shape
    k = rb // BLOCK_BYTES[qtype] * BLOCK_ELEMS[qtype]
    return (name, [k, n], qtype, np.ascontiguousarray(blocks).tobytes())
