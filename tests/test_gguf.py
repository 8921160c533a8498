"""GGUF tensor directory (pai_gguf_dir_*), checked against the reference's
own reader (pai_gguf_open / pai_gguf_dequant, adapters/llama/gguf.c, built
from its sources into oracle/_ref) on the same file images: every decision
(status, version, alignment, data start, each tensor info) must agree.
No GPU: pai_qmat_upload_gguf is exercised only on its argument and
directory errors here; tests/test_gpu_gguf.py uploads."""
import ctypes as C
import struct

import numpy as np
import pytest

import gguf_file as gf
import oracle_bind as ob
import prosperoai_amd as pa

PROTOCOL, UNSUPPORTED, MISMATCH, INVALID = -10, -3, -6, -1


def mine(img: bytes):
    try:
        d = pa.GGUFDir(img)
    except pa.PaiError as e:
        return e.status, None, None
    with d:
        ts = [(t.name, t.type, t.n_dims, t.dims, t.offset) for t in d.tensors()]
        return 0, d.layout, ts


def agree(img: bytes):
    got = mine(img)
    want = ob.ref_gguf_directory(img)
    assert got == want
    return got


def sample_file(alignment_kv=None, align=32, version=3):
    rng = np.random.default_rng(7)
    kv = [("general.architecture", gf.STR, "llama"),
          ("general.name", gf.STR, "tiny"),
          ("llama.block_count", gf.U32, 2),
          ("llama.rope.freq_base", gf.F32, 10000.0),
          ("x.u8", gf.U8, 3), ("x.i8", gf.I8, -3), ("x.u16", gf.U16, 700), ("x.i16", gf.I16, -7),
          ("x.i32", gf.I32, -9), ("x.bool", gf.BOOL, True), ("x.u64", gf.U64, 1 << 40),
          ("x.i64", gf.I64, -(1 << 40)), ("x.f64", gf.F64, 0.25),
          ("tokenizer.ggml.tokens", gf.ARR, (gf.STR, ["<s>", "</s>", "a", "bb"])),
          ("tokenizer.ggml.scores", gf.ARR, (gf.F32, [0.0, -1.0, -2.5, 3.0])),
          ("x.nested", gf.ARR, (gf.ARR, [(gf.U16, [1, 2, 3]), (gf.STR, ["q"])])),
          ("x.empty", gf.ARR, (gf.I64, []))]
    if alignment_kv is not None:
        kv.insert(2, alignment_kv)
    tensors = []
    for i, (qt, n, k) in enumerate([(2, 3, 64), (8, 2, 96), (12, 4, 256), (14, 2, 512)]):
        w = pa.normal_f32(100 + i, n * k, 0.0, 0.05).reshape(n, k)
        tensors.append(gf.weight(f"blk.0.w{i}.weight", qt, pa.quantize(qt, w)))
    tensors.append(("blk.0.attn_norm.weight", [16], 0, rng.random(16, np.float32).tobytes()))
    tensors.append(("x.cube", [4, 2, 3], 1, rng.integers(0, 255, 48, np.uint8).tobytes()))
    return gf.build(kv, tensors, version=version, alignment=align), tensors


@pytest.mark.parametrize("version", [1, 2, 3])
def test_directory_matches_reference_reader(ref_lib, version):
    img, tensors = sample_file(version=version)
    st, layout, ts = agree(img)
    assert st == 0 and layout[0] == version and layout[1] == 32
    assert [t[0] for t in ts] == [t[0] for t in tensors]
    with pa.GGUFDir(img) as d:
        for i, (name, dims, qt, data) in enumerate(tensors):
            assert d.find(name) == i
            assert d.tensor(i).dims == tuple(dims) + (0,) * (4 - len(dims))
            if qt in pa.BLOCK_BYTES:
                assert d.blocks(i).tobytes() == data
        with pytest.raises(pa.PaiError) as e:
            d.find("missing.weight")
        assert e.value.status == MISMATCH


def test_directory_from_mapped_file(ref_lib, tmp_path):
    img, tensors = sample_file()
    p = tmp_path / "m.gguf"
    p.write_bytes(img)
    with pa.GGUFDir(p) as d:
        assert len(d) == len(tensors)
        assert d.blocks(2).tobytes() == tensors[2][3]
    with pa.GGUFDir(p) as d:
        assert [(t.name, t.type, t.n_dims, t.dims, t.offset) for t in d.tensors()] == \
            ob.ref_gguf_directory(img)[2]


@pytest.mark.parametrize("akv,align", [
    (("general.alignment", gf.U32, 64), 64),
    (("general.alignment", gf.U8, 16), 16),
    (("general.alignment", gf.I16, 256), 256),
    (("general.alignment", gf.F32, 1.0), 32),      # f32 bits 0x3f800000: not a power of two
    (("general.alignment", gf.BOOL, True), 1),
    (("general.alignment", gf.U32, 4096), 4096),
    (("general.alignment", gf.U32, 8192), 32),     # above 4096
    (("general.alignment", gf.U32, 0), 32),
    (("general.alignment", gf.U32, 48), 32),
    (("general.alignment", gf.STR, "64"), 32),     # not an integer type: default
    (("general.alignment", gf.ARR, (gf.U32, [64])), 32),
    (("general.alignmentX", gf.U32, 64), 32),
])
def test_alignment_key_matches_reference(ref_lib, akv, align):
    img, _ = sample_file(alignment_kv=akv, align=align)
    agree(img)


@pytest.mark.parametrize("vt,value,align", [(gf.U64, 128, 128), (gf.I64, 64, 64),
                                             (gf.U64, (1 << 32) | 64, 64)])
def test_alignment_key_of_8_byte_type(vt, value, align):
    """The reference reads an 8-byte alignment value into a variable its
    helper never writes (le_bytes_to_u64, adapters/llama/gguf.c:291-301,
    leaves *out unset), so its outcome is undefined and not compared here.
    This reader takes the value truncated to 32 bits, as it does for the
    other integer types."""
    img, _ = sample_file(alignment_kv=("general.alignment", vt, value), align=align)
    st, layout, _ = mine(img)
    assert st == 0 and layout[1] == align and layout[2] % align == 0


def test_first_alignment_key_decides(ref_lib):
    kv = [("general.alignment", gf.STR, "x"), ("general.alignment", gf.U32, 64)]
    t = [("w", [32, 2], 8, bytes(68))]
    st, layout, _ = agree(gf.build(kv, t, alignment=32))
    assert st == 0 and layout[1] == 32
    kv = [("general.alignment", gf.U32, 64), ("general.alignment", gf.U32, 3)]
    st, layout, _ = agree(gf.build(kv, t, alignment=64))
    assert st == 0 and layout[1] == 64


def test_reader_errors_match_reference_cases(ref_lib):
    # the cases of tests/test_gguf.c:563-629 in the reference
    buf = bytearray(b"\xaa" * 64)
    assert mine(bytes(buf[:4]))[0] == PROTOCOL
    assert mine(bytes(buf))[0] == PROTOCOL
    buf[:8] = b"GGUF" + struct.pack("<I", 99)
    assert mine(bytes(buf))[0] == UNSUPPORTED
    img = gf.build([], [("t", [32], 0, bytes(4))])
    assert agree(img)[0] == 0
    with pa.GGUFDir(img) as d:   # F32 is not a block format of this path
        with pytest.raises(pa.PaiError) as e:
            d.blocks(0)
        assert e.value.status == UNSUPPORTED
    assert agree(gf.build([], [("t", [(1 << 26) + 1], 0, bytes(8))]))[0] == PROTOCOL
    assert agree(gf.build([], [("t", [1 << 26], 0, bytes(8))]))[0] == 0


@pytest.mark.parametrize("case,status", [
    ("version0", UNSUPPORTED), ("version4", UNSUPPORTED), ("tensors1025", UNSUPPORTED),
    ("tensors1024", 0), ("name0", PROTOCOL), ("name127", 0), ("name128", PROTOCOL),
    ("dims0", PROTOCOL), ("dims5", PROTOCOL), ("kvtype13", PROTOCOL), ("zero_extent", 0),
    ("string_past_end", PROTOCOL), ("array_past_end", PROTOCOL), ("empty", PROTOCOL),
    ("bare_header", 0),
])
def test_malformed_headers(ref_lib, case, status):
    t1 = [("w", [32, 1], 8, bytes(34))]
    if case.startswith("version"):
        img = gf.build([], t1, version=int(case[7:]))
    elif case.startswith("tensors"):
        nt = int(case[7:])
        img = gf.build([], [(f"t{i}", [32], 8, bytes(34)) for i in range(nt)], alignment=32)
    elif case.startswith("name"):
        img = gf.build([], [("n" * int(case[4:]), [32], 8, bytes(34))])
    elif case.startswith("dims"):
        nd = int(case[4:])
        img = gf.build([], [("w", [32] + [1] * (nd - 1) if nd else [], 8, bytes(34))])
    elif case == "kvtype13":
        img = gf.build([("k", gf.U32, 1)], t1)
        i = img.index(b"k") + 1
        img = img[:i] + struct.pack("<I", 13) + img[i + 4:]
    elif case == "zero_extent":
        img = gf.build([], [("w", [0, 4], 8, b"")])
    elif case == "string_past_end":
        img = gf.build([("k", gf.STR, "abc")], [])
        i = img.index(b"abc") - 8
        img = img[:i] + struct.pack("<Q", 1 << 40) + img[i + 8:]
    elif case == "array_past_end":
        img = gf.build([("k", gf.ARR, (gf.U32, [1, 2]))], [])
        i = img.index(struct.pack("<IQ", gf.U32, 2)) + 4
        img = img[:i] + struct.pack("<Q", 1 << 61) + img[i + 8:]
    elif case == "empty":
        img = b""
    else:
        img = gf.build([], [])
    st = agree(img)[0]
    assert st == status


def test_every_truncation_matches_reference(ref_lib):
    img, _ = sample_file()
    with pa.GGUFDir(img) as d:
        start = d.layout[2]
    for cut in range(0, start + 8):
        agree(img[:cut])


def test_byte_mutations_match_reference(ref_lib):
    img, _ = sample_file(alignment_kv=("general.alignment", gf.U32, 64), align=64)
    with pa.GGUFDir(img) as d:
        start = d.layout[2]
    # the alignment value's type field: an 8-byte type there is undefined in
    # the reference (see test_alignment_key_of_8_byte_type), so skip those
    at = img.index(b"general.alignment") + 17
    rng = np.random.default_rng(2024)
    special = [0x00, 0x01, 0x02, 0x04, 0x08, 0x0c, 0x0d, 0x10, 0x7f, 0x80, 0xff]
    seen = set()
    for _ in range(3000):
        b = bytearray(img)
        for _ in range(int(rng.integers(1, 3))):
            pos = int(rng.integers(0, start))
            b[pos] = int(rng.choice(special)) if rng.random() < 0.7 else int(rng.integers(0, 256))
        if struct.unpack_from("<I", b, at)[0] in (10, 11, 12):
            continue
        seen.add(agree(bytes(b))[0])
    # the mutations reach accepting and both rejecting outcomes
    assert {0, PROTOCOL} <= seen


def test_block_checks_match_reference_dequant(ref_lib):
    q = pa.quantize(12, pa.normal_f32(3, 2 * 256).reshape(2, 256))
    good = gf.weight("w", 12, q)
    cases = {
        "ok": gf.build([], [good]),
        "past_eof": gf.build([], [good])[:-100],
        "offset_past_end": None,
        "ragged": gf.build([], [("w", [32, 2], 12, bytes(144))]),  # 64 elements of Q4_K
        "zero_numel": gf.build([], [("w", [0, 2], 12, b"")]),
    }
    img = bytearray(gf.build([], [good]))
    i = img.index(b"w") + 1 + 4 + 16 + 4
    img[i:i + 8] = struct.pack("<Q", 1 << 50)
    cases["offset_past_end"] = bytes(img)
    for name, img in cases.items():
        with pa.GGUFDir(img) as d:
            try:
                blk = d.blocks(0)
                st = 0
            except pa.PaiError as e:
                st, blk = e.status, None
        assert st == ob.ref_gguf_dequant_status(img, "w"), name
        if name == "ok":
            assert blk.tobytes() == q.tobytes()


def test_upload_gguf_errors_before_device():
    img = gf.build([], [("v", [32], 8, bytes(34)), ("w", [32, 1], 8, bytes(34))])
    lib = pa.lib()
    h = C.c_void_p()
    with pa.GGUFDir(img) as d:
        with pytest.raises(pa.PaiError) as e:
            d.upload("absent")
        assert e.value.status == MISMATCH
        with pytest.raises(pa.PaiError) as e:
            d.upload("v")            # 1-D: not a weight matrix
        assert e.value.status == MISMATCH
        assert lib.pai_qmat_upload_gguf(None, d._h, b"w") == INVALID
        assert lib.pai_qmat_upload_gguf(C.byref(h), None, b"w") == INVALID
        assert lib.pai_qmat_upload_gguf(C.byref(h), d._h, None) == INVALID
        assert lib.pai_gguf_dir_tensor(d._h, 2, None, None, None, None, None) == INVALID
    assert lib.pai_gguf_dir_open(None, 10, C.byref(h)) == INVALID
    assert lib.pai_gguf_dir_count(None) == 0
    lib.pai_gguf_dir_close(None)
