"""The oracle's v0 per-group schemes (models/quantize.c) and the GEMMs over
the [K][N] int8 / nibble layouts (cpu/reference/ref_ops.c:446-499), pinned
against the reference's own test cases (tests/test_quantize.c), closed
forms, brute force, and the reference's sources built into oracle/_ref."""
import ctypes as C

import numpy as np
import pytest

import oracle_bind as ob


def sch(bits, signed=1, gs=0):
    return ob.QuantScheme(bits, signed, gs)


# ---------------------------------------------------------------- scheme sizing
def test_scheme_and_sizes_reference_cases():
    """tests/test_quantize.c:37-60."""
    o = ob.oracle()
    gs = C.c_uint64(0)
    assert o.orc_quant_group_size(None, 1, C.byref(gs)) == -1
    assert o.orc_quant_group_size(C.byref(sch(8)), 1, C.byref(gs)) == 0
    assert o.orc_quant_group_size(C.byref(sch(16)), 1, C.byref(gs)) == -3
    assert o.orc_quant_group_size(C.byref(sch(4, 0)), 1, C.byref(gs)) == -3
    assert o.orc_quant_value_bytes(256, C.byref(sch(8))) == 256
    assert o.orc_quant_value_bytes(256, C.byref(sch(4))) == 128
    assert o.orc_quant_value_bytes(3, C.byref(sch(4))) == 2
    assert o.orc_quant_num_groups(256, C.byref(sch(4))) == 1
    assert o.orc_quant_num_groups(256, C.byref(sch(4, gs=64))) == 4
    assert o.orc_quant_num_groups(257, C.byref(sch(4, gs=64))) == 5


def test_sizes_equal_reference_build(ref_lib):
    o = ob.oracle()
    for bits in (4, 8, 16):
        for signed in (0, 1):
            for gs in (0, 1, 3, 64, 65535):
                s = sch(bits, signed, gs)
                for n in (0, 1, 2, 3, 255, 256, 257, 100000):
                    assert o.orc_quant_num_groups(n, C.byref(s)) == \
                        ref_lib.pai_quant_num_groups(n, C.byref(s))
                    assert o.orc_quant_value_bytes(n, C.byref(s)) == \
                        ref_lib.pai_quant_value_bytes(n, C.byref(s))


# ---------------------------------------------------------------- quantize / dequantize
def test_quantize_reference_exact_cases():
    """tests/test_quantize.c:79-117, with the codes the definition fixes."""
    q, s = ob.v0_quantize(np.array([0.0, 100.0, -100.0, 100.0]), 8, 0)
    assert s[0] == np.float32(100.0) / np.float32(127.0)
    assert q.tolist() == [0, 127, -127, 127]
    d = ob.v0_dequantize(q, s, 4, 8, 0)
    assert np.all(np.abs(d - [0, 100, -100, 100]) < 1e-4)

    # q4: scale fl(2/7) lies above 2/7, so 1 / scale = 3.4999998 in f32 and
    # the code of 1.0 is 3
    q, s = ob.v0_quantize(np.array([0.0, 2.0, -2.0, 1.0]), 4, 0)
    assert s[0] == np.float32(2.0) / np.float32(7.0)
    assert np.float32(1.0) / s[0] < np.float32(3.5)
    assert (q.view(np.uint8).tolist()) == [0x70, 0x39]  # codes 0, 7 | -7 (0x9), 3
    d = ob.v0_dequantize(q, s, 4, 4, 0)
    assert d[0] == 0 and abs(d[1] - 2) < 1e-4 and abs(d[2] + 2) < 1e-4 and abs(d[3] - 1) < 0.2

    # odd length: the last byte's high nibble stays zero
    q, s = ob.v0_quantize(np.array([4.0, -4.0, 4.0]), 4, 0)
    assert q.view(np.uint8).tolist() == [0x97, 0x07]
    d = ob.v0_dequantize(q, s, 3, 4, 0)
    assert np.all(np.abs(d - [4, -4, 4]) < 1e-4)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [0, 1, 7, 32, 64, 1000])
def test_quantize_closed_forms(bits, gs):
    rng = np.random.default_rng(bits * 1000 + gs)
    n = 2049
    x = rng.standard_normal(n).astype(np.float32)
    x[100:140] = 0.0  # a zero run (a whole group for the small sizes)
    q, s = ob.v0_quantize(x, bits, gs)
    qmax = 127 if bits == 8 else 7
    g = n if gs == 0 else gs
    codes = q.astype(np.int32) if bits == 8 else np.stack(
        [((q.view(np.uint8) & 15) ^ 8).astype(np.int32) - 8,
         ((q.view(np.uint8) >> 4) ^ 8).astype(np.int32) - 8], 1).ravel()[:n]
    d = ob.v0_dequantize(q, s, n, bits, gs)
    for gi in range(s.size):
        sl = slice(gi * g, min(n, (gi + 1) * g))
        amax = np.abs(x[sl]).max()
        if amax == 0:
            assert s[gi] == 0 and np.all(codes[sl] == 0)
            continue
        assert s[gi] == np.float32(amax) / np.float32(qmax)
        assert np.abs(codes[sl]).max() == qmax          # the extreme element maps to +-qmax
        assert np.all(np.abs(codes[sl]) <= qmax)
        assert np.all(np.abs(d[sl] - x[sl]) <= s[gi] * 0.5000001 + 1e-7)  # half a step
        assert np.array_equal(d[sl], (s[gi] * codes[sl].astype(np.float32)).astype(np.float32))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [0, 1, 5, 32, 64, 4097])
@pytest.mark.parametrize("n", [1, 2, 31, 4096, 4097])
def test_quantize_equals_reference_build(ref_lib, bits, gs, n):
    x = np.random.default_rng(n + gs + bits).standard_normal(n).astype(np.float32) * 3
    q, s = ob.v0_quantize(x, bits, gs)
    rq, rs = ob.v0_quantize(x, bits, gs, lib=ref_lib)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    d = ob.v0_dequantize(q, s, n, bits, gs)
    rd = ob.v0_dequantize(q, s, n, bits, gs, lib=ref_lib)
    assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))


def test_quantize_argument_errors(ref_lib):
    x = np.ones(4, np.float32)
    q, sc = np.zeros(4, np.int8), np.zeros(1, np.float32)
    o = ob.oracle()
    for fn in (o.orc_quantize_v0_f32, ref_lib.pai_quantize_f32):
        assert fn(None, 4, C.byref(sch(8)), q.ctypes.data, sc.ctypes.data, None) == -1
        assert fn(x.ctypes.data, 4, C.byref(sch(16)), q.ctypes.data, sc.ctypes.data, None) == -3
        assert fn(x.ctypes.data, 0, C.byref(sch(8)), q.ctypes.data, sc.ctypes.data, None) == -1
    for fn in (o.orc_dequantize_v0_f32, ref_lib.pai_dequantize_f32):
        assert fn(q.ctypes.data, None, 4, C.byref(sch(8)), x.ctypes.data) == -1


# ---------------------------------------------------------------- [K][N] GEMMs
def kn_operands(w: np.ndarray, bits: int, gs: int):
    """[K][N] codes and [G][N] scales, each column quantized in K groups of
    gs as in tests/test_quantize.c:155-176; 4-bit codes repacked over the
    flat index t*n+j."""
    k, n = w.shape
    g = k if gs == 0 else gs
    ng = -(-k // g)
    codes = np.zeros((k, n), np.int32)
    scales = np.zeros((ng, n), np.float32)
    for j in range(n):
        q, s = ob.v0_quantize(w[:, j], bits, gs)
        if bits == 4:
            u = q.view(np.uint8)
            c = np.stack([(u & 15), (u >> 4)], 1).ravel()[:k].astype(np.int32)
            codes[:, j] = np.where(c & 8, c - 16, c)
        else:
            codes[:, j] = q
        scales[:, j] = s
    if bits == 8:
        return codes.astype(np.int8), scales
    flat = (codes.ravel() & 15).astype(np.uint8)
    if flat.size % 2:
        flat = np.r_[flat, np.uint8(0)]
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8).view(np.int8)
    return packed, scales


def dequant_kn(bits, w_q, scales, k, n, gs, dtype=np.float32):
    g = k if (gs == 0 or gs > k) else gs
    if bits == 8:
        codes = w_q.astype(np.int32).reshape(k, n)
    else:
        u = w_q.view(np.uint8)
        c = np.stack([(u & 15), (u >> 4)], 1).ravel()[:k * n].astype(np.int32)
        codes = np.where(c & 8, c - 16, c).reshape(k, n)
    return (codes.astype(dtype) * scales[np.arange(k) // g].astype(dtype)).astype(dtype)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("m,n,k,gs", [(3, 5, 8, 4), (2, 33, 70, 32), (1, 64, 128, 0),
                                      (4, 7, 9, 100), (1, 16, 64, 16)])
def test_gemm_equals_reference_build(ref_lib, bits, m, n, k, gs):
    rng = np.random.default_rng(m * 100 + n + k + bits)
    w_q, sc = kn_operands(rng.standard_normal((k, n)).astype(np.float32), bits, gs)
    a = rng.standard_normal((m, k)).astype(np.float32)
    got = ob.gemm_wq_seq(bits, a, w_q, sc, n, gs)
    want = ob.gemm_wq_seq(bits, a, w_q, sc, n, gs, lib=ref_lib)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4])
def test_gemm_one_hot_returns_dequantized_rows(bits):
    """a = e_t picks row t of the dequantized [K][N] matrix, exactly: a
    transposed operand, a wrong nibble or a wrong group index fails."""
    k, n, gs = 12, 7, 4  # odd n: 4-bit rows start mid-byte
    rng = np.random.default_rng(bits)
    w_q, sc = kn_operands(rng.standard_normal((k, n)).astype(np.float32), bits, gs)
    deq = dequant_kn(bits, w_q, sc, k, n, gs)
    got = ob.gemm_wq_seq(bits, np.eye(k, dtype=np.float32), w_q, sc, n, gs)
    assert np.array_equal(got, deq)


@pytest.mark.parametrize("bits", [8, 4])
def test_gemm_reference_tolerance_case_and_f64(bits):
    """tests/test_quantize.c:135-236: against the f32 GEMM of the dequantized
    weights (1e-3 for w8, 1e-2 for w4), and the f64 brute force."""
    m, n, k, gs = 3, 5, 8, 4
    rng = np.random.default_rng(7)
    w_q, sc = kn_operands(rng.uniform(-1, 1, (k, n)).astype(np.float32), bits, gs)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    got = ob.gemm_wq_seq(bits, a, w_q, sc, n, gs)
    dense = a.astype(np.float64) @ dequant_kn(bits, w_q, sc, k, n, gs).astype(np.float64)
    tol = 1e-3 if bits == 8 else 1e-2
    assert np.all(np.abs(got - dense) <= np.maximum(tol, np.abs(dense) * tol))
    f64 = ob.gemm_wq_f64(bits, a, w_q, sc, n, gs)
    exact = a.astype(np.float64) @ dequant_kn(bits, w_q, sc, k, n, gs, np.float64)
    assert np.allclose(f64, exact, rtol=1e-14, atol=1e-14)
    assert np.abs(got - f64).max() <= 1e-5 * np.abs(f64).max()


def test_gemm_group_size_zero_and_past_k_are_per_tensor():
    k, n = 20, 6
    rng = np.random.default_rng(3)
    w_q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    sc = rng.uniform(0.01, 0.02, (1, n)).astype(np.float32)
    a = rng.standard_normal((2, k)).astype(np.float32)
    y0 = ob.gemm_wq_seq(8, a, w_q, sc, n, 0)
    y1 = ob.gemm_wq_seq(8, a, w_q, sc, n, 21)
    assert np.array_equal(y0, y1)
