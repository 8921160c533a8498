"""The CPU oracle pinned against the reference's golden vectors, the
reference-built checker, closed forms and brute force (no GPU)."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle_bind as ob

GOLD = Path(__file__).resolve().parent / "golden"
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
QK = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BB = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}


def f16_closed_form(h: int) -> int:
    """binary16 -> binary32 bit pattern from the IEEE 754 definition."""
    s, e, f = (h >> 15) & 1, (h >> 10) & 0x1F, h & 0x3FF
    if e == 0x1F:
        return (s << 31) | 0x7F800000 | (f << 13)
    val = (f / 1024.0) * 2.0 ** -14 if e == 0 else (1 + f / 1024.0) * 2.0 ** (e - 15)
    return int(np.array([-val if s else val], np.float32).view(np.uint32)[0])


# ---------------------------------------------------------------- f16
def test_f16_exhaustive_vs_numpy_and_closed_form():
    hs = np.arange(65536, dtype=np.uint32)
    got = ob.f16_bits(hs.astype(np.uint16))
    want_np = hs.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    finite = ((hs >> 10) & 0x1F) != 0x1F
    assert np.array_equal(got[finite], want_np[finite])
    # inf/NaN: the payload is shifted, never quieted (gguf.c:624-625)
    nonfin = np.nonzero(~finite)[0]
    assert all(got[h] == f16_closed_form(int(h)) for h in nonfin)
    for h in (0x0001, 0x03FF, 0x0400, 0x8001, 0x7BFF, 0xFBFF, 0x3555):
        assert got[h] == f16_closed_form(h)


def test_f16_reference_literals():
    d = json.loads((GOLD / "gguf_hand_vectors.json").read_text())
    for h, v in d["f16_literals"]:
        assert ob.oracle().orc_f16_to_f32(h) == v


# ---------------------------------------------------------------- K-scale unpack
def test_scale_min_k4_closed_form():
    """Brute force: the 8 (scale, min) pairs are fixed 6-bit fields of the
    12-byte little-endian word: sc_j = bits [6j] for j<4 from bytes 0-3,
    else low nibble of byte j+4 and the top 2 bits of byte j-4; likewise
    for the mins with the high nibble and bytes 4-7."""
    rng = np.random.default_rng(1)
    o = ob.oracle()
    import ctypes as C
    for _ in range(300):
        q = rng.integers(0, 256, 12, dtype=np.uint8)
        bits = int.from_bytes(q.tobytes(), "little")
        fld = lambda byte, lo, n: (bits >> (8 * byte + lo)) & ((1 << n) - 1)  # noqa: E731
        for j in range(8):
            sc, mn = C.c_uint8(), C.c_uint8()
            o.orc_scale_min_k4(j, q.ctypes.data, C.addressof(sc), C.addressof(mn))
            if j < 4:
                want = (fld(j, 0, 6), fld(j + 4, 0, 6))
            else:
                want = (fld(j + 4, 0, 4) | (fld(j - 4, 6, 2) << 4),
                        fld(j + 4, 4, 4) | (fld(j, 6, 2) << 4))
            assert (sc.value, mn.value) == want


# ---------------------------------------------------------------- dequant
def test_dequant_hand_vectors():
    d = json.loads((GOLD / "gguf_hand_vectors.json").read_text())
    for c in d["cases"]:
        raw = np.frombuffer(bytes.fromhex(c["raw"]), np.uint8)
        got = ob.dequant(c["type"], raw, c["numel"])
        assert np.array_equal(got, np.asarray(c["expect"], np.float32)), c["name"]


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_dequant_matches_reference_fixture(qtype):
    z = np.load(GOLD / "ref_vectors.npz")
    raw, want = z[f"dq_raw_{qtype}"], z[f"dq_out_{qtype}"]
    got = ob.dequant(qtype, raw, raw.shape[0] * QK[qtype])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_dequant_matches_reference_build(ref_lib, qtype):
    import make_golden
    rng = np.random.default_rng(100 + qtype)
    raw = make_golden.random_blocks(rng, qtype, 200)
    got = ob.dequant(qtype, raw, 200 * QK[qtype])
    want = ob.ref_dequant(qtype, raw.tobytes(), 200 * QK[qtype])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_invariants():
    rng = np.random.default_rng(7)
    for qtype in (Q4_0, Q8_0, Q4_K, Q6_K):
        z = np.zeros(BB[qtype], np.uint8)
        assert not ob.dequant(qtype, z, QK[qtype]).any()  # zero block -> 0
    # linearity in d: doubling the f16 scale (exponent + 1) doubles every value
    for qtype, off in ((Q4_0, 0), (Q8_0, 0), (Q6_K, 208)):
        raw = rng.integers(0, 256, BB[qtype], dtype=np.uint8)
        raw[off:off + 2] = np.frombuffer(np.float16(0.375).tobytes(), np.uint8)
        a = ob.dequant(qtype, raw, QK[qtype])
        raw[off:off + 2] = np.frombuffer(np.float16(0.75).tobytes(), np.uint8)
        assert np.array_equal(ob.dequant(qtype, raw, QK[qtype]), 2 * a)
    # Q4_K with dmin = 0 reduces to d*sc*q
    raw = rng.integers(0, 256, 144, dtype=np.uint8)
    raw[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    raw[2:4] = 0
    vals = ob.dequant(Q4_K, raw, 256)
    bits = int.from_bytes(raw[4:16].tobytes(), "little")
    for e in range(256):
        c, hi, l = e // 64, (e // 32) & 1, e % 32
        j = 2 * c + hi
        sc = ((bits >> (8 * j)) & 63) if j < 4 else \
            (((bits >> (8 * (j + 4))) & 15) | (((bits >> (8 * (j - 4) + 6)) & 3) << 4))
        code = raw[16 + 32 * c + l] >> 4 if hi else raw[16 + 32 * c + l] & 15
        assert vals[e] == np.float32(0.25) * np.float32(sc) * np.float32(code)
    # Q6_K with ql = qh = 0: every value is -32 * d * sc[e/16]
    raw = np.zeros(210, np.uint8)
    raw[192:208] = rng.integers(-128, 128, 16).astype(np.int8).view(np.uint8)
    raw[208:210] = np.frombuffer(np.float16(-1.5).tobytes(), np.uint8)
    sc = raw[192:208].view(np.int8).astype(np.float32)
    want = (np.float32(-1.5) * sc) * np.float32(-32.0)
    assert np.array_equal(ob.dequant(Q6_K, raw, 256), np.repeat(want, 16))


def test_type_bytes_semantics(ref_lib):
    o = ob.oracle()
    for t in (Q4_0, Q8_0, Q4_K, Q6_K, 0, 1, 3, 9, 13, 15, 99):
        for numel in (0, 1, 32, 64, 255, 256, 4096, 14336):
            assert o.orc_type_bytes(t, numel) == (
                ref_lib.pai_gguf_type_bytes(t, numel) if t in (Q4_0, Q8_0, Q4_K, Q6_K) else 0)


# ---------------------------------------------------------------- GEMM oracles
def test_gemm_seq_matches_reference_fixture():
    z = np.load(GOLD / "ref_vectors.npz")
    a, b, c = z["gemm_a"], z["gemm_b"], z["gemm_c"]
    m, k = a.shape
    n = b.shape[1]
    got = np.empty((m, n), np.float32)
    assert ob.oracle().orc_gemm_seq_f32(m, n, k, a.ctypes.data, b.ctypes.data,
                                        got.ctypes.data) == 0
    assert np.array_equal(got.view(np.uint32), c.view(np.uint32))


def test_gemm_seq_brute_force_and_args():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((2, 5)).astype(np.float32)
    b = rng.standard_normal((5, 3)).astype(np.float32)
    c = np.empty((2, 3), np.float32)
    o = ob.oracle()
    assert o.orc_gemm_seq_f32(2, 3, 5, a.ctypes.data, b.ctypes.data, c.ctypes.data) == 0
    want = np.zeros((2, 3), np.float32)
    for i in range(2):
        for j in range(3):
            s = np.float32(0)
            for l in range(5):
                s = np.float32(s + np.float32(a[i, l] * b[l, j]))
            want[i, j] = s
    assert np.array_equal(c, want)
    assert o.orc_gemm_seq_f32(0, 3, 5, a.ctypes.data, b.ctypes.data, c.ctypes.data) == -1
    assert o.orc_gemm_seq_f32(2, 3, 5, None, b.ctypes.data, c.ctypes.data) == -1


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_qgemm_oracles_one_hot_and_f64(qtype):
    import make_golden
    rng = np.random.default_rng(11 + qtype)
    n, k = 5, 2 * QK[qtype]
    raw = make_golden.random_blocks(rng, qtype, n * k // QK[qtype])
    w = ob.dequant(qtype, raw, n * k).reshape(n, k)
    # one-hot x returns column j exactly
    for j in (0, 1, k // 2 + 3, k - 1):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        assert np.array_equal(ob.qgemm_seq(qtype, n, k, raw, x)[0], w[:, j])
    # f64 oracle equals the exact sum of the f32 products on integers-valued x
    x = rng.integers(-3, 4, size=(3, k)).astype(np.float32)
    y64 = ob.qgemm_f64(qtype, n, k, raw, x)
    assert np.allclose(y64, x.astype(np.float64) @ w.astype(np.float64).T, rtol=1e-12,
                       atol=1e-6 * np.abs(w).max())


def test_avx2_restatements_match_reference_fixture():
    z = np.load(GOLD / "ref_vectors.npz")
    o = ob.oracle()
    a, x, y = z["gemv_a"], z["gemv_x"], z["gemv_y"]
    got = np.empty_like(y)
    assert o.orc_opt_gemv_avx2(a.shape[0], a.shape[1], a.ctypes.data, x.ctypes.data,
                               got.ctypes.data) == 0
    assert np.array_equal(got.view(np.uint32), y.view(np.uint32))
    got_mt = np.empty_like(y)
    assert o.orc_opt_gemv_avx2_mt(a.shape[0], a.shape[1], a.ctypes.data, x.ctypes.data,
                                  got_mt.ctypes.data, 4) == 0
    assert np.array_equal(got_mt, got)
    wa, wq, ws, wc = z["w8_a"], z["w8_q"], z["w8_s"], z["w8_c"]
    gs = int(z["w8_gs"][0])
    got = np.empty_like(wc)
    assert o.orc_opt_gemm_w8_avx2(wa.shape[0], wq.shape[1], wa.shape[1], wa.ctypes.data,
                                  wq.ctypes.data, ws.ctypes.data, gs, got.ctypes.data) == 0
    assert np.array_equal(got.view(np.uint32), wc.view(np.uint32))


def test_avx2_restatements_match_reference_build(ref_lib):
    rng = np.random.default_rng(5)
    o = ob.oracle()
    for m, k in ((1, 4096), (17, 333)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        y1, y2 = np.empty(m, np.float32), np.empty(m, np.float32)
        o.orc_opt_gemv_avx2(m, k, a.ctypes.data, x.ctypes.data, y1.ctypes.data)
        ref_lib.pai_opt_gemv_f32(m, k, a.ctypes.data, x.ctypes.data, y2.ctypes.data)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    m, n, k = 3, 21, 64
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c1, c2 = np.empty((m, n), np.float32), np.empty((m, n), np.float32)
    o.orc_opt_gemm_avx2(m, n, k, a.ctypes.data, b.ctypes.data, c1.ctypes.data)
    ref_lib.pai_opt_gemm_f32(m, n, k, a.ctypes.data, b.ctypes.data, c2.ctypes.data)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
    c3 = np.empty((m, n), np.float32)
    ref_lib.pai_ref_gemm_f32(m, n, k, a.ctypes.data, b.ctypes.data, c3.ctypes.data)
    o.orc_gemm_seq_f32(m, n, k, a.ctypes.data, b.ctypes.data, c1.ctypes.data)
    assert np.array_equal(c1.view(np.uint32), c3.view(np.uint32))


def test_compare_semantics():
    a = np.array([1.0, 2.0, 3.0], np.float32)
    b = np.array([1.0, 2.1, 3.0], np.float32)
    import ctypes as C
    bad = C.c_uint64()
    assert ob.oracle().orc_compare_f32(a.ctypes.data, b.ctypes.data, 3, 1e-5, 1e-5,
                                       C.addressof(bad)) == -6
    assert bad.value == 1
    assert ob.oracle().orc_compare_f32(a.ctypes.data, b.ctypes.data, 3, 0.2, 0.0,
                                       C.addressof(bad)) == 0


def _silu_mul_inputs():
    rng = np.random.default_rng(31)
    g = np.concatenate([rng.normal(0, 3, 4000), rng.normal(0, 40, 1000),
                        [0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 89.0, -104.0, -110.0, 1e30,
                         -1e30, np.inf, -np.inf]]).astype(np.float32)
    u = rng.normal(0, 1, g.size).astype(np.float32)
    return g, u


def test_silu_mul_matches_reference_build(ref_lib):
    """orc_silu_mul_f32 is the reference's SILU then MUL, bit for bit
    (cpu/reference/ref_ops.c:219-228 and :124-133)."""
    g, u = _silu_mul_inputs()
    s, want = np.empty_like(g), np.empty_like(g)
    assert ref_lib.pai_ref_silu_f32(g.ctypes.data, s.ctypes.data, g.size) == 0
    assert ref_lib.pai_ref_vecmul_f32(s.ctypes.data, u.ctypes.data, want.ctypes.data, g.size) == 0
    got = ob.silu_mul(g, u)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_silu_mul_closed_form():
    g, u = _silu_mul_inputs()
    h = ob.silu_mul(g, np.ones_like(u))
    fin = np.isfinite(g) & (np.abs(g) < 1e29)
    # against the f64 closed form g / (1 + e^-g): a few ulp, where e^-g
    # stays finite in f32 (below g = -88.7 the f32 composition gives -0)
    fin &= g > -87.0
    ref = g[fin].astype(np.float64) / (1.0 + np.exp(-g[fin].astype(np.float64)))
    assert np.all(np.abs(h[fin] - ref) <= 4 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-38)
    # fixed points: silu(0) = 0, silu(x) = x for large x, -> -0 for very negative x
    assert h[g == 0].tolist() == [0.0, 0.0]
    assert h[g == 89.0][0] == 89.0 and h[g == 1e30][0] == 1e30
    assert h[g == -110.0][0] == 0.0 and np.signbit(h[g == -110.0][0])
    assert np.isnan(h[g == -np.inf][0]) and h[g == np.inf][0] == np.inf
    # the product is the elementwise one
    fin = np.isfinite(g) & (np.abs(g) < 1e29)
    assert np.array_equal(ob.silu_mul(g, u)[fin], (h * u)[fin])
