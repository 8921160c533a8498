"""GGUF tensor directory over a file in memory (pai_gguf_dir_* in
include/pai_hip.h) and upload of a tensor's native blocks as a QMat.

The file is memory-mapped; the directory points into the mapping, which
stays open while the GGUFDir lives.
"""
from __future__ import annotations

import ctypes as C
import mmap
import os
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib
from .qmat import QMat


@dataclass(frozen=True)
class TensorInfo:
    """The fields of pai_gguf_tensor_t (adapters/llama/gguf.h:54-60)."""
    name: str
    type: int
    n_dims: int
    dims: tuple
    offset: int  # from the start of the data section


class GGUFDir:
    def __init__(self, source):
        """`source`: a path, or a bytes-like object holding the whole file."""
        self._mm = None
        if isinstance(source, (str, os.PathLike)):
            with open(source, "rb") as f:
                size = os.fstat(f.fileno()).st_size
                self._mm = mmap.mmap(f.fileno(), size, access=mmap.ACCESS_READ) if size else b""
            self._buf = np.frombuffer(self._mm, dtype=np.uint8) if size else np.zeros(0, np.uint8)
        else:
            self._buf = np.frombuffer(bytes(source), dtype=np.uint8)
        self._h = C.c_void_p()
        # a zero-length file still needs a non-NULL pointer for the length check
        ptr = self._buf.ctypes.data if self._buf.size else C.addressof(C.c_char())
        check(lib().pai_gguf_dir_open(ptr, self._buf.size, C.byref(self._h)), "pai_gguf_dir_open")

    def close(self) -> None:
        if self._h.value:
            lib().pai_gguf_dir_close(self._h)
            self._h = C.c_void_p()
        self._buf = None
        if self._mm is not None and not isinstance(self._mm, bytes):
            self._mm.close()
        self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return int(lib().pai_gguf_dir_count(self._h))

    @property
    def layout(self) -> tuple[int, int, int]:
        """(version, alignment, data_start)."""
        v, a, s = C.c_uint32(), C.c_uint32(), C.c_uint64()
        check(lib().pai_gguf_dir_layout(self._h, C.byref(v), C.byref(a), C.byref(s)),
              "pai_gguf_dir_layout")
        return v.value, a.value, s.value

    def tensor(self, index: int) -> TensorInfo:
        name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        dims, off = (C.c_uint64 * 4)(), C.c_uint64()
        check(lib().pai_gguf_dir_tensor(self._h, index, C.byref(name), C.byref(t), C.byref(nd),
                                        dims, C.byref(off)), "pai_gguf_dir_tensor")
        return TensorInfo(name.value.decode(errors="surrogateescape"), t.value, nd.value, tuple(dims), off.value)

    def tensors(self) -> list[TensorInfo]:
        return [self.tensor(i) for i in range(len(self))]

    def find(self, name: str) -> int:
        i = C.c_uint64()
        check(lib().pai_gguf_dir_find(self._h, name.encode(), C.byref(i)), "pai_gguf_dir_find")
        return i.value

    def blocks(self, index: int) -> np.ndarray:
        """The tensor's native block bytes (a view into the file)."""
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().pai_gguf_dir_blocks(self._h, index, C.byref(p), C.byref(n)),
              "pai_gguf_dir_blocks")
        start = p.value - self._buf.ctypes.data
        return self._buf[start:start + n.value]

    def upload(self, name: str) -> QMat:
        """pai_qmat_upload_gguf: the 2-D tensor `name` as a resident W[N][K]."""
        h = C.c_void_p()
        check(lib().pai_qmat_upload_gguf(C.byref(h), self._h, name.encode()),
              "pai_qmat_upload_gguf")
        return QMat.adopt(h)
