"""The drop-in boundary on the CPU: the CPU twin the qgemm descriptors carry
as their reference function, the GGUF IR tag, and a C program compiled
against the reference's own op.h / ir.h that registers the descriptors into
the registry built from the reference's sources.

Bars: the CPU twin equals the oracle's sequential composition and the
reference build's own composition (pai_gguf_dequant, transpose,
pai_ref_gemm_f32) bit for bit; the tag maps the four formats one to one.
"""
import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import prosperoai_amd as pa
from prosperoai_amd._lib import lib

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
QK = pa.BLOCK_ELEMS


def blocks_for(qtype: int, n: int, k: int, seed: int) -> np.ndarray:
    import make_golden
    rng = np.random.default_rng(seed)
    return make_golden.random_blocks(rng, qtype, n * k // QK[qtype]).reshape(n, -1)


def twin(qtype: int, blocks: np.ndarray, x: np.ndarray, n: int) -> np.ndarray:
    m, k = x.shape
    y = np.empty((m, n), np.float32)
    b = np.ascontiguousarray(blocks)
    st = lib().pai_qgemm_ref_f32(qtype, m, n, k, x.ctypes.data, b.ctypes.data, y.ctypes.data)
    assert st == 0, st
    return y


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m,n,kb", [(1, 7, 2), (3, 5, 1), (5, 33, 3)])
def test_cpu_twin_equals_oracle_sequential_sum(orc, qtype, m, n, kb):
    k = kb * QK[qtype]
    blocks = blocks_for(qtype, n, k, 31 * qtype + m + n)
    x = np.random.default_rng(m + n).standard_normal((m, k)).astype(np.float32)
    want = orc.qgemm_seq(qtype, n, k, blocks, x)
    assert np.array_equal(twin(qtype, blocks, x, n).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
def test_cpu_twin_equals_reference_composition(ref_lib, orc, qtype):
    """pai_gguf_dequant of the reference build, the [N][K] -> [K][N]
    transpose, and its pai_ref_gemm_f32: the CPU operator the reference runs
    for the same weight today."""
    m, n, k = 3, 9, 2 * QK[qtype] * (8 if QK[qtype] == 32 else 1)
    blocks = blocks_for(qtype, n, k, 7 + qtype)
    x = np.random.default_rng(qtype).standard_normal((m, k)).astype(np.float32)
    w = orc.ref_dequant(qtype, blocks.tobytes(), n * k, row=k).reshape(n, k)
    wt = np.ascontiguousarray(w.T)
    want = np.empty((m, n), np.float32)
    assert ref_lib.pai_ref_gemm_f32(m, n, k, x.ctypes.data, wt.ctypes.data, want.ctypes.data) == 0
    assert np.array_equal(twin(qtype, blocks, x, n).view(np.uint32), want.view(np.uint32))


def test_cpu_twin_keeps_nan_scale_payload(orc):
    """A block whose f16 scale is a NaN dequantizes to NaN products, as in
    the reference (the payload reaches every product)."""
    blocks = np.zeros((1, 18), np.uint8)
    blocks[0, 0:2] = np.frombuffer(np.uint16(0x7E01).tobytes(), np.uint8)
    blocks[0, 2:] = 0x99
    x = np.ones((1, 32), np.float32)
    assert np.isnan(twin(2, blocks, x, 1)[0, 0])


def test_cpu_twin_argument_errors():
    L = lib()
    x = np.zeros((1, 32), np.float32)
    y = np.zeros((1, 1), np.float32)
    b = np.zeros(18, np.uint8)
    assert L.pai_qgemm_ref_f32(2, 1, 1, 32, None, b.ctypes.data, y.ctypes.data) == -1
    assert L.pai_qgemm_ref_f32(2, 0, 1, 32, x.ctypes.data, b.ctypes.data, y.ctypes.data) == -1
    assert L.pai_qgemm_ref_f32(3, 1, 1, 32, x.ctypes.data, b.ctypes.data, y.ctypes.data) == -3
    assert L.pai_qgemm_ref_f32(12, 1, 1, 32, x.ctypes.data, b.ctypes.data, y.ctypes.data) == -3


class Quant(C.Structure):
    """pai_hip_ir_quant_t (the layout of the reference's pai_ir_quant_t)."""
    _fields_ = [("present", C.c_uint8), ("bit_width", C.c_uint8), ("scale_repr", C.c_uint8),
                ("zero_point_repr", C.c_uint8), ("is_signed", C.c_uint8),
                ("block_structure", C.c_uint8), ("group_size", C.c_uint16)]


def test_gguf_tag_round_trip_and_injective():
    L = lib()
    seen = set()
    for t, bits, signed, group in ((8, 8, 1, 32), (2, 4, 0, 32), (12, 4, 0, 256), (14, 6, 1, 256)):
        q = Quant()
        assert L.pai_hip_quant_tag(t, C.byref(q)) == 0
        assert (q.present, q.bit_width, q.is_signed, q.group_size) == (1, bits, signed, group)
        assert q.block_structure == 3 and q.scale_repr == 1
        assert L.pai_hip_quant_type(C.byref(q)) == t
        key = (q.bit_width, q.group_size, q.is_signed)
        assert key not in seen
        seen.add(key)
    assert L.pai_hip_quant_tag(3, C.byref(Quant())) == -3
    assert L.pai_hip_quant_tag(2, None) == -1
    # not a GGUF tag, absent, or a combination of no format
    q = Quant()
    assert L.pai_hip_quant_tag(12, C.byref(q)) == 0
    for field, value in (("block_structure", 2), ("present", 0), ("group_size", 64),
                         ("is_signed", 1)):
        r = Quant.from_buffer_copy(q)
        setattr(r, field, value)
        assert L.pai_hip_quant_type(C.byref(r)) == 0, field
    assert L.pai_hip_quant_type(None) == 0


def test_c_program_against_reference_headers(ref_lib, tmp_path):
    """The descriptor and tag layouts checked by the compiler against the
    reference's headers; registration into the registry built from the
    reference's sources; a GGUF-tagged GEMM resolves to its descriptor."""
    if not (REF / "sdk" / "include" / "pai" / "op.h").exists() or shutil.which("gcc") is None:
        pytest.skip("reference headers or gcc absent")
    exe = tmp_path / "boundary"
    libdir = ROOT / "prosperoai_amd" / "lib"
    refdir = ROOT / "oracle" / "_ref"
    cmd = ["gcc", "-std=c11", "-Wall", "-Werror", f"-I{REF / 'sdk' / 'include'}", f"-I{REF}",
           f"-I{ROOT / 'include'}", str(ROOT / "tests" / "c" / "boundary.c"), "-o", str(exe),
           f"-L{libdir}", "-lpai_hip", str(refdir / "libpairef.so"),
           f"-Wl,-rpath,{libdir}:{refdir}", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert "boundary ok: 6 descriptors" in r.stdout


def test_gemm_branch_against_reference_executor(ref_lib, tmp_path):
    """pai_qgemm_shape_check against run_gemm itself (scheduler.c:280-343),
    driven through one-op graphs in the reference executor: equal statuses
    on 5488 shape combinations of GEMM and GEMV, and the three accepted
    forms' results on the dequantized weight equal to the CPU twin."""
    if not (REF / "scheduler" / "scheduler.h").exists() or shutil.which("gcc") is None:
        pytest.skip("reference headers or gcc absent")
    exe = tmp_path / "sched_gemm"
    libdir = ROOT / "prosperoai_amd" / "lib"
    refdir = ROOT / "oracle" / "_ref"
    cmd = ["gcc", "-std=c11", "-Wall", "-Werror", f"-I{REF / 'sdk' / 'include'}", f"-I{REF}",
           f"-I{REF / 'memory'}", f"-I{ROOT / 'include'}", str(ROOT / "tests" / "c" / "sched_gemm.c"),
           "-o", str(exe), f"-L{libdir}", "-lpai_hip", str(refdir / "libpairef.so"),
           f"-Wl,-rpath,{libdir}:{refdir}", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert "statuses: 5488 cases, 54 accepted, 0 differ" in r.stdout
    assert "run_gemm parity ok" in r.stdout


@pytest.mark.parametrize("is_gemv,a,b,c,w,tokens", [
    (True, [1024, 4096], [4096], [1024], (1024, 4096), 1),
    (False, [4096], [4096, 1024], [1024], (1024, 4096), 1),
    (False, [4096], [4096, 1024], [1, 1024], (1024, 4096), 1),
    (False, [512, 4096], [4096, 14336], [512, 14336], (14336, 4096), 512),
])
def test_gemm_branch_accepts_the_llama_forms(is_gemv, a, b, c, w, tokens):
    assert pa.gemm_shape_check(is_gemv, a, b, c, *w) == tokens


@pytest.mark.parametrize("is_gemv,a,b,c,w", [
    (True, [4096, 1024], [4096], [1024], (1024, 4096)),     # A is [k, n]: not the weight rows
    (True, [1024, 4096], [4096], [1, 1024], (1024, 4096)),  # GEMV output of rank 2
    (False, [4096], [4096, 1024], [2, 1024], (1024, 4096)),  # row vector, two output rows
    (False, [4096], [1024, 4096], [1024], (1024, 4096)),   # B untransposed
    (False, [8, 4096], [4096, 1024], [1024], (1024, 4096)),  # GEMM output of rank 1
    (False, [8, 4096], [4096, 1024], [8, 1024], (1000, 4096)),  # another weight
    (False, [2, 8, 4096], [4096, 1024], [16, 1024], (1024, 4096)),  # rank-3 activations
])
def test_gemm_branch_rejects_as_run_gemm(is_gemv, a, b, c, w):
    with pytest.raises(pa.PaiError, match="MISMATCH"):
        pa.gemm_shape_check(is_gemv, a, b, c, *w)


def test_gemm_branch_argument_errors_without_a_gpu():
    L = lib()
    dims = (C.c_uint64 * 2)(4, 4)
    m = C.c_uint64(0)
    assert L.pai_qgemm_shape_check(0, 2, None, 2, dims, 2, dims, 4, 4, C.byref(m)) == -1
    assert L.pai_qgemm_shape_check(0, 2, dims, 2, dims, 2, dims, 4, 4, None) == -1
    assert L.pai_qgemm_run(None, 0, 2, dims, 2, dims, 2, dims, None, None, 0) == -1


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("m,n,k,gs", [(3, 5, 8, 4), (2, 33, 70, 32), (1, 64, 128, 0), (4, 7, 9, 100)])
def test_v0_cpu_twins_equal_reference_build(ref_lib, bits, m, n, k, gs):
    """pai_gemm_w8_ref_f32 / _w4_ref_f32 against the reference build's
    pai_ref_gemm_w8_f32 / _w4_f32, bit for bit."""
    import oracle_bind as ob
    rng = np.random.default_rng(m + n + k + bits)
    nbytes = k * n if bits == 8 else (k * n + 1) // 2
    w = rng.integers(-128, 128, nbytes).astype(np.int8)
    sc = rng.uniform(0.001, 0.05, (-(-k // (gs if 0 < gs <= k else k)), n)).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    want = ob.gemm_wq_seq(bits, a, w, sc, n, gs, lib=ref_lib)
    got = np.empty((m, n), np.float32)
    fn = lib().pai_gemm_w8_ref_f32 if bits == 8 else lib().pai_gemm_w4_ref_f32
    assert fn(m, n, k, a.ctypes.data, w.ctypes.data, sc.ctypes.data, gs, got.ctypes.data) == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert fn(0, n, k, a.ctypes.data, w.ctypes.data, sc.ctypes.data, gs, got.ctypes.data) == -1
    assert fn(m, n, k, None, w.ctypes.data, sc.ctypes.data, gs, got.ctypes.data) == -1


def test_v0_entry_points_check_arguments_without_a_gpu():
    """Argument errors come back before any device work (no GPU here)."""
    L = lib()
    a = np.zeros(4, np.float32)
    w = np.zeros(4, np.int8)
    for fn in (L.pai_hip_gemm_w8_f32, L.pai_hip_gemm_w4_f32):
        assert fn(0, 1, 1, a.ctypes.data, w.ctypes.data, a.ctypes.data, 0, a.ctypes.data) == -1
        assert fn(1, 1, 1, None, w.ctypes.data, a.ctypes.data, 0, a.ctypes.data) == -1
    assert L.pai_hip_gemm_wq_f32_async(6, 1, 1, 1, a.ctypes.data, w.ctypes.data, a.ctypes.data,
                                       0, a.ctypes.data, None, 0, None) == -3
    bad = Scheme(16, 1, 0)
    unsigned = Scheme(8, 0, 0)
    assert L.pai_hip_quantize_f32(a.ctypes.data, 4, C.byref(bad), w.ctypes.data, a.ctypes.data,
                                  None) == -3
    assert L.pai_hip_quantize_f32(a.ctypes.data, 4, C.byref(unsigned), w.ctypes.data,
                                  a.ctypes.data, None) == -3
    assert L.pai_hip_quantize_f32(a.ctypes.data, 4, None, w.ctypes.data, a.ctypes.data,
                                  None) == -1
    assert L.pai_hip_quantize_f32(None, 4, C.byref(Scheme(8, 1, 0)), w.ctypes.data,
                                  a.ctypes.data, None) == -1
    # n == 0 with one group over the array: a zero group size (quantize.c:20-23)
    assert L.pai_hip_quantize_f32(a.ctypes.data, 0, C.byref(Scheme(8, 1, 0)), w.ctypes.data,
                                  a.ctypes.data, None) == -1
    assert L.pai_hip_dequantize_f32(w.ctypes.data, None, 4, C.byref(Scheme(8, 1, 0)),
                                    a.ctypes.data) == -1


class Scheme(C.Structure):
    """pai_hip_quant_scheme_t (the layout of the reference's pai_quant_scheme_t)."""
    _fields_ = [("bit_width", C.c_uint8), ("is_signed", C.c_uint8), ("group_size", C.c_uint16)]
