"""The 64-bit `.pai` container and the uncapped tokenizer blob (no GPU):
version-2 round trips at Llama-3-8B sizes (a 128 256-token vocabulary,
280 000 merges, a section beyond 4 GiB), compatibility with version-1
files and blobs written by the reference's own pai/pai.c and
models/tokenizer.c (built into oracle/_ref), and the format's error
rules. The checksum is pinned against zlib's CRC-32 and the reference's."""
import ctypes as C
import os
import zlib

import numpy as np
import pytest

from prosperoai_amd import pai64
from prosperoai_amd._lib import lib


# ---------------------------------------------------------------- checksum
@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 255, 4096, 1 << 20])
def test_crc32_is_zlib_crc32(n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert pai64.crc32(data) == zlib.crc32(data)
    # continuing a running checksum
    assert pai64.crc32(data[n // 3:], pai64.crc32(data[:n // 3])) == zlib.crc32(data)


def test_crc32_equals_reference(ref_lib):
    fn = ref_lib.pai_proto_crc32
    fn.restype, fn.argtypes = C.c_uint32, [C.c_void_p, C.c_uint32]
    data = np.random.default_rng(5).integers(0, 256, 10007, dtype=np.uint8)
    assert fn(data.ctypes.data, data.size) == pai64.crc32(data.tobytes())


# ---------------------------------------------------------------- version 1
class RefBuilder(C.Structure):
    """pai_pai_builder_t (pai/pai.h:85-93)."""
    class Sec(C.Structure):
        _fields_ = [("type", C.c_uint32), ("flags", C.c_uint32), ("data", C.c_void_p),
                    ("size", C.c_uint32)]
    _fields_ = [("num_sections", C.c_uint32), ("sections", Sec * 8)]


def ref_v1_blob(ref_lib, sections):
    for name, res, args in (("pai_pai_builder_init", None, [C.c_void_p]),
                            ("pai_pai_builder_add_flags", C.c_int32,
                             [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32]),
                            ("pai_pai_encoded_size", C.c_uint32, [C.c_void_p]),
                            ("pai_pai_build", C.c_int32,
                             [C.c_void_p, C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)])):
        getattr(ref_lib, name).restype, getattr(ref_lib, name).argtypes = res, args
    b = RefBuilder()
    ref_lib.pai_pai_builder_init(C.byref(b))
    keep = []
    for t, payload, flags in sections:
        buf = np.frombuffer(payload, np.uint8).copy()
        keep.append(buf)
        assert ref_lib.pai_pai_builder_add_flags(C.byref(b), t, flags, buf.ctypes.data,
                                                 len(payload)) == 0
    total = ref_lib.pai_pai_encoded_size(C.byref(b))
    out = np.zeros(total, np.uint8)
    n = C.c_uint32(0)
    assert ref_lib.pai_pai_build(C.byref(b), out.ctypes.data, total, C.byref(n)) == 0
    return out.tobytes()


def test_reads_reference_version_1_containers(ref_lib, tmp_path):
    secs = [(pai64.META, b"m" * 64, 0), (pai64.WEIGHTS, os.urandom(1000), 1),
            (pai64.TOKENIZER, os.urandom(77), 0)]
    blob = ref_v1_blob(ref_lib, secs)
    path = tmp_path / "v1.pai"
    path.write_bytes(blob)
    m = pai64.Mapped(str(path))
    try:
        assert m.view.version == 1 and m.view.num_sections == 3
        for t, payload, flags in secs:
            assert m.section(t) == payload
        assert m.view.sections[1].flags == 1
        assert m.section(pai64.IR) is None
        # version 1 has no per-section checksum: open checked the whole file
        assert lib().pai64_verify_section(C.byref(m.view), pai64.WEIGHTS) == -3
    finally:
        m.close()
    # any flipped byte fails the whole-file checksum, as in pai_pai_open
    for pos in (1, 12, 20, len(blob) - 1):
        bad = bytearray(blob)
        bad[pos] ^= 0x40
        assert pai64.open_status(bytes(bad)) == -10
    assert pai64.open_status(blob[:-1]) == -10


# ---------------------------------------------------------------- version 2
def llama3_vocab(n=128256):
    rng = np.random.default_rng(3)
    texts = [bytes([(i % 255) + 1]) * (1 + i % 11) + str(i).encode() for i in range(n)]
    merges = rng.integers(0, n, (280000, 3), dtype=np.uint32)
    return list(range(n)), texts, merges


def test_version_2_round_trip_at_llama3_sizes(tmp_path, ref_lib):
    ids, texts, merges = llama3_vocab()
    tok = pai64.tok_encode(ids, texts, merges)
    tensors = [pai64.Tensor(b"blk.0.ffn_gate.weight", 7, 0, 2, (4096, 14336, 0, 0, 0, 0), 0,
                            14336 * 16 * 144, 12),
               pai64.Tensor(b"output_norm.weight", 9, 0, 1, (4096, 0, 0, 0, 0, 0), 33030144,
                            16384, 0)]
    man = pai64.manifest_encode(tensors)
    weights = os.urandom(33030144 + 16384)
    meta = bytes(64)
    path = tmp_path / "m.pai"
    n = pai64.write(str(path), [(pai64.META, meta), (pai64.MANIFEST, man),
                                (pai64.WEIGHTS, weights), (pai64.TOKENIZER, tok)])
    assert n == path.stat().st_size
    m = pai64.Mapped(str(path))
    try:
        assert m.view.version == 2 and m.view.num_sections == 4
        for i in range(4):
            assert m.view.sections[i].offset % 256 == 0
            assert m.view.sections[i].flags & pai64.FLAG_CRC
            assert lib().pai64_verify_section(C.byref(m.view), m.view.sections[i].type) == 0
        assert m.section(pai64.WEIGHTS) == weights
        got = pai64.manifest_decode(m.section(pai64.MANIFEST))
        assert [(t.name, t.gguf_type, tuple(t.shape), t.offset, t.size_bytes) for t in got] == \
            [(t.name, t.gguf_type, tuple(t.shape), t.offset, t.size_bytes) for t in tensors]
        gids, gtexts, gm = pai64.tok_decode(m.section(pai64.TOKENIZER))
        assert gids == ids and gtexts == texts and np.array_equal(gm, merges)
    finally:
        m.close()
    # the reference's tokenizer refuses the version-2 blob (version and caps)
    tok_t = C.create_string_buffer(64)
    ref_lib.pai_tok_init.argtypes = [C.c_void_p]
    ref_lib.pai_tok_deserialize.restype = C.c_int32
    ref_lib.pai_tok_deserialize.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
    ref_lib.pai_tok_init(tok_t)
    b = np.frombuffer(tok, np.uint8)
    assert ref_lib.pai_tok_deserialize(tok_t, b.ctypes.data, len(tok)) == -10


def test_manifest_layout_is_the_reference_layout(ref_lib):
    """The reference's pai_pai_manifest_decode reads the entries (the GGUF
    type sits in the field it ignores)."""
    class RefTensor(C.Structure):
        _fields_ = [("name", C.c_char * 64), ("value_id", C.c_uint32), ("dtype", C.c_int32),
                    ("rank", C.c_uint32), ("shape", C.c_uint64 * 6), ("offset", C.c_uint64),
                    ("size_bytes", C.c_uint64)]
    tensors = [pai64.Tensor(f"t{i}".encode(), i + 1, 0, 2, (256 * (i + 1), 64, 0, 0, 0, 0),
                            1000 * i, 144 * (i + 1) * 64, (2, 8, 12, 14)[i % 4])
               for i in range(9)]
    man = pai64.manifest_encode(tensors)
    out = (RefTensor * 16)()
    n = C.c_uint32(0)
    fn = ref_lib.pai_pai_manifest_decode
    fn.restype = C.c_int32
    fn.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]
    b = np.frombuffer(man, np.uint8)
    assert fn(b.ctypes.data, len(man), C.byref(out), 16, C.byref(n)) == 0 and n.value == 9
    for t, r in zip(tensors, out):
        assert (r.name, r.value_id, r.rank, tuple(r.shape), r.offset, r.size_bytes) == \
            (t.name, t.value_id, t.rank, tuple(t.shape), t.offset, t.size_bytes)


def test_reference_tokenizer_blob_reads_as_version_1(ref_lib):
    for name, res, args in (("pai_tok_init", None, [C.c_void_p]),
                            ("pai_tok_add_token", C.c_int32, [C.c_void_p, C.c_uint32, C.c_char_p]),
                            ("pai_tok_add_merge", C.c_int32,
                             [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32]),
                            ("pai_tok_blob_size", C.c_uint32, [C.c_void_p]),
                            ("pai_tok_serialize", C.c_int32,
                             [C.c_void_p, C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32)]),
                            ("pai_tok_destroy", None, [C.c_void_p])):
        getattr(ref_lib, name).restype, getattr(ref_lib, name).argtypes = res, args
    tok = C.create_string_buffer(64)
    ref_lib.pai_tok_init(tok)
    words = [b"hello", b"wor", b"ld", b"!"]
    for i, w in enumerate(words):
        assert ref_lib.pai_tok_add_token(tok, 300 + i, w) == 0
    assert ref_lib.pai_tok_add_merge(tok, 301, 302, 303) == 0
    n = ref_lib.pai_tok_blob_size(tok)
    out = np.zeros(n, np.uint8)
    got = C.c_uint32(0)
    assert ref_lib.pai_tok_serialize(tok, out.ctypes.data, n, C.byref(got)) == 0
    ref_lib.pai_tok_destroy(tok)
    ids, texts, merges = pai64.tok_decode(out.tobytes())
    assert ids == [300, 301, 302, 303] and texts == words
    assert merges.tolist() == [[301, 302, 303]]
    # a version-1 blob above version 1's caps is refused
    blob = bytearray(out.tobytes())
    blob[8:12] = (65537).to_bytes(4, "little")
    assert pai64.tok_status(bytes(blob)) == -10


def test_section_past_4_gib(tmp_path):
    """WEIGHTS behind a 4.25 GiB hole (a sparse file): 64-bit offsets in the
    table, a mapped read of the payload, and its checksum."""
    path = tmp_path / "big.pai"
    hole = (4 << 30) + (1 << 28)
    payload = os.urandom(1 << 20)
    try:
        n = pai64.write(str(path), [(pai64.TARGET, hole), (pai64.WEIGHTS, payload)])
    except Exception as e:  # a filesystem without sparse files
        pytest.skip(f"cannot create a sparse {hole >> 30} GiB file: {e}")
    assert n > (1 << 32)
    m = pai64.Mapped(str(path))
    try:
        w = [m.view.sections[i] for i in range(2) if m.view.sections[i].type == pai64.WEIGHTS][0]
        assert w.offset > (1 << 32) and w.offset % 256 == 0
        assert m.section(pai64.WEIGHTS) == payload
        assert lib().pai64_verify_section(C.byref(m.view), pai64.WEIGHTS) == 0
        assert lib().pai64_verify_section(C.byref(m.view), pai64.TARGET) == -3  # no checksum
    finally:
        m.close()
        path.unlink()


# ---------------------------------------------------------------- errors
def v2_blob(tmp_path, secs):
    p = tmp_path / "e.pai"
    pai64.write(str(p), secs)
    return p.read_bytes()


def test_open_rejects_malformed_version_2(tmp_path):
    blob = v2_blob(tmp_path, [(pai64.META, b"x" * 64), (pai64.WEIGHTS, b"w" * 300)])
    assert pai64.open_status(blob) == 0

    def patched(off, value, width=4, fix_crc=True):
        b = bytearray(blob)
        b[off:off + width] = value.to_bytes(width, "little")
        if fix_crc:  # keep the header checksum right so the rule itself is tested
            table_end = 32 + 32 * int.from_bytes(b[8:12], "little")
            crc = zlib.crc32(bytes(b[16:table_end]), zlib.crc32(bytes(b[:12])))
            b[12:16] = crc.to_bytes(4, "little")
        return bytes(b)

    assert pai64.open_status(patched(0, 0x12345678)) == -10          # magic
    assert pai64.open_status(patched(4, 3, 2)) == -10                 # version
    assert pai64.open_status(patched(6, 1, 2)) == -10                 # header flags
    assert pai64.open_status(patched(8, 0)) == -10                    # no sections
    assert pai64.open_status(patched(8, 9)) == -10                    # too many
    assert pai64.open_status(patched(12, 0, fix_crc=False)) == -10    # header checksum
    assert pai64.open_status(patched(24, 1, 8)) == -10                # reserved
    assert pai64.open_status(blob[:-1]) == -10                        # total size field
    e0, e1 = 32, 64
    assert pai64.open_status(patched(e0, 8)) == -10                   # section type
    assert pai64.open_status(patched(e1, 1)) == -10                   # repeated type
    assert pai64.open_status(patched(e0 + 4, 1 | (1 << 31))) == -10   # flags on META
    assert pai64.open_status(patched(e0 + 8, 64, 8)) == -10           # overlaps the table
    assert pai64.open_status(patched(e0 + 8, 264, 8)) == -10          # not aligned
    w_off = int.from_bytes(blob[e1 + 8:e1 + 16], "little")
    assert pai64.open_status(patched(e0 + 8, w_off, 8)) == -10        # overlaps WEIGHTS
    assert pai64.open_status(patched(e1 + 16, 10 ** 6, 8)) == -10     # leaves the file
    assert pai64.open_status(patched(e0 + 28, 1)) == -10              # reserved entry field
    # a flipped payload byte opens (checksums are checked on request) ...
    b = bytearray(blob)
    b[w_off + 5] ^= 1
    view = pai64.Container()
    arr = np.frombuffer(bytes(b), np.uint8)
    assert lib().pai64_open(arr.ctypes.data, len(b), C.byref(view)) == 0
    # ... and fails its section's check
    assert lib().pai64_verify_section(C.byref(view), pai64.WEIGHTS) == -10
    assert lib().pai64_verify_section(C.byref(view), pai64.META) == 0
    assert lib().pai64_verify_section(C.byref(view), pai64.IR) == -6


def test_writer_and_codecs_reject_bad_input(tmp_path):
    p = str(tmp_path / "x.pai")
    L = lib()
    for secs in ([], [(0, b"a")], [(8, b"a")], [(1, b"a"), (1, b"b")], [(1, b"a", 1)],
                 [(3, b"a", 2)]):
        arr = (pai64.SectionIn * max(len(secs), 1))()
        keep = []
        for i, s in enumerate(secs):
            buf = np.frombuffer(s[1], np.uint8)
            keep.append(buf)
            arr[i] = pai64.SectionIn(s[0], s[2] if len(s) > 2 else 0, buf.ctypes.data, len(s[1]))
        assert L.pai64_write_file(p.encode(), C.byref(arr), len(secs), None) == -1
    assert pai64.tok_status(b"PTK1" + bytes(8)) == -1                 # shorter than a header
    assert pai64.tok_status((0x314B5450).to_bytes(4, "little") + (3).to_bytes(4, "little")
                            + bytes(8)) == -10                         # version
    good = pai64.tok_encode([1, 2], ["a", "bc"], [])
    assert pai64.tok_status(good[:-1]) == -10                          # truncated text
    bad = bytearray(good)
    bad[16 + 4] = 0
    assert pai64.tok_status(bytes(bad)) == -10                         # empty text
    with pytest.raises(Exception):
        pai64.tok_encode([1], [""], [])
    with pytest.raises(Exception):
        pai64.manifest_encode([pai64.Tensor(b"", 1, 0, 1, (1, 0, 0, 0, 0, 0), 0, 4, 0)])
    man = pai64.manifest_encode([pai64.Tensor(b"w", 1, 0, 2, (64, 64, 0, 0, 0, 0), 0, 4, 8)])
    for off, val in ((4 + 2 + 1 + 4 + 1, 7),     # rank 7
                     (4 + 2 + 1 + 4, 9)):         # dtype 9
        b = bytearray(man)
        b[off] = val
        with pytest.raises(Exception):
            pai64.manifest_decode(bytes(b))
    with pytest.raises(Exception):
        pai64.manifest_decode(man[:-1])
