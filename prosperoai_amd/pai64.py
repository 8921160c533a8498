"""ctypes view of the 64-bit `.pai` container entry points (include/pai_pai64.h),
for tests and tooling."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib

META, MANIFEST, WEIGHTS, IR, TOKENIZER, TARGET, PROFILE = range(1, 8)
FLAG_COMPRESSED, FLAG_CRC = 1, 1 << 31
ALIGN = 256


class Section(C.Structure):
    _fields_ = [("type", C.c_uint32), ("flags", C.c_uint32), ("offset", C.c_uint64),
                ("size", C.c_uint64), ("crc", C.c_uint32)]


class Container(C.Structure):
    _fields_ = [("version", C.c_uint32), ("num_sections", C.c_uint32),
                ("sections", Section * 8), ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class SectionIn(C.Structure):
    _fields_ = [("type", C.c_uint32), ("flags", C.c_uint32), ("data", C.c_void_p),
                ("size", C.c_uint64)]


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("value_id", C.c_uint32), ("dtype", C.c_uint32),
                ("rank", C.c_uint32), ("shape", C.c_uint64 * 6), ("offset", C.c_uint64),
                ("size_bytes", C.c_uint64), ("gguf_type", C.c_uint32)]


def crc32(data: bytes, crc: int = 0) -> int:
    b = np.frombuffer(data, np.uint8) if len(data) else np.zeros(1, np.uint8)
    return lib().pai64_crc32(crc, b.ctypes.data, len(data))


def write(path: str, sections: list) -> int:
    """sections: (type, payload bytes or None with a size for a hole[, flags])."""
    keep, arr = [], (SectionIn * len(sections))()
    for i, sec in enumerate(sections):
        t, payload = sec[0], sec[1]
        flags = sec[2] if len(sec) > 2 else 0
        if isinstance(payload, int):  # a hole of that many zero bytes
            arr[i] = SectionIn(t, flags, None, payload)
        else:
            buf = np.frombuffer(payload, np.uint8) if len(payload) else np.zeros(1, np.uint8)
            keep.append(buf)
            arr[i] = SectionIn(t, flags, buf.ctypes.data if len(payload) else None, len(payload))
    n = C.c_uint64(0)
    check(lib().pai64_write_file(path.encode(), C.byref(arr), len(sections), C.byref(n)),
          "pai64_write_file")
    return n.value


class Mapped:
    """A mapped container file and its parsed view."""

    def __init__(self, path: str):
        self.ptr, self.n = C.c_void_p(), C.c_uint64()
        check(lib().pai64_map_file(path.encode(), C.byref(self.ptr), C.byref(self.n)),
              "pai64_map_file")
        self.view = Container()
        st = lib().pai64_open(self.ptr, self.n.value, C.byref(self.view))
        if st != 0:
            self.close()
            check(st, "pai64_open")

    def section(self, t: int) -> bytes | None:
        size = C.c_uint64(0)
        p = lib().pai64_section(C.byref(self.view), t, C.byref(size))
        return None if p is None else C.string_at(p, size.value)

    def close(self) -> None:
        if self.ptr:
            lib().pai64_unmap_file(self.ptr, self.n.value)
            self.ptr = C.c_void_p()


def open_status(blob: bytes) -> int:
    b = np.frombuffer(blob, np.uint8)
    view = Container()
    return lib().pai64_open(b.ctypes.data, len(blob), C.byref(view))


def manifest_encode(tensors: list) -> bytes:
    arr = (Tensor * len(tensors))(*tensors)
    total = lib().pai64_manifest_bytes(C.byref(arr), len(tensors))
    out = np.zeros(max(total, 1), np.uint8)
    n = C.c_uint64(0)
    check(lib().pai64_manifest_encode(C.byref(arr), len(tensors), out.ctypes.data, total,
                                      C.byref(n)), "pai64_manifest_encode")
    return out[:n.value].tobytes()


def manifest_decode(blob: bytes, max_tensors: int = 4096) -> list:
    b = np.frombuffer(blob, np.uint8)
    arr = (Tensor * max_tensors)()
    n = C.c_uint32(0)
    check(lib().pai64_manifest_decode(b.ctypes.data, len(blob), C.byref(arr), max_tensors,
                                      C.byref(n)), "pai64_manifest_decode")
    return [arr[i] for i in range(n.value)]


def tok_encode(ids: list, texts: list, merges: list) -> bytes:
    tb = [t.encode() if isinstance(t, str) else t for t in texts]
    carr = (C.c_char_p * max(len(tb), 1))(*tb)
    iarr = np.asarray(ids, np.uint32)
    marr = np.asarray(merges, np.uint32).reshape(-1)
    total = lib().pai64_tok_bytes(carr, len(tb), len(merges))
    out = np.zeros(max(total, 1), np.uint8)
    n = C.c_uint64(0)
    check(lib().pai64_tok_encode(iarr.ctypes.data, carr, len(tb),
                                 marr.ctypes.data if len(merges) else None, len(merges),
                                 out.ctypes.data, total, C.byref(n)), "pai64_tok_encode")
    return out[:n.value].tobytes()


def tok_decode(blob: bytes):
    """(ids, texts, merges) of a version-1 or version-2 tokenizer blob."""
    b = np.frombuffer(blob, np.uint8)
    nt, nm, mo = C.c_uint32(0), C.c_uint32(0), C.c_uint64(0)
    check(lib().pai64_tok_index(b.ctypes.data, len(blob), C.byref(nt), C.byref(nm), None, 0,
                                C.byref(mo)), "pai64_tok_index")
    offs = np.zeros(max(nt.value, 1), np.uint64)
    check(lib().pai64_tok_index(b.ctypes.data, len(blob), C.byref(nt), C.byref(nm),
                                offs.ctypes.data, nt.value, C.byref(mo)), "pai64_tok_index")
    ids, texts = [], []
    for o in offs[:nt.value].astype(np.int64):
        ids.append(int.from_bytes(blob[o:o + 4], "little"))
        ln = blob[o + 4]
        texts.append(blob[o + 5:o + 5 + ln])
    m = np.frombuffer(blob[mo.value:mo.value + 12 * nm.value], "<u4").reshape(-1, 3)
    return ids, texts, m


def tok_status(blob: bytes) -> int:
    b = np.frombuffer(blob, np.uint8)
    nt, nm = C.c_uint32(0), C.c_uint32(0)
    return lib().pai64_tok_index(b.ctypes.data, len(blob), C.byref(nt), C.byref(nm), None, 0,
                                 None)
