"""Host encoders, f16 conversions and the seeded generator of libpai_hip.so
(no GPU). The reference has no GGUF encoder, so encoder parity is
unpinned by it: Q8_0/Q4_0 are checked bit-for-bit against the oracle's
textbook llama.cpp encoders, and all four against round-trip bounds that
follow from how each format spends its bits."""
import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa


def test_f16_roundtrip_exhaustive():
    lib = pa.lib()
    hs = np.arange(65536, dtype=np.uint32)
    got = np.array([lib.paiq_f16_to_f32(int(h)) for h in hs], np.float32)
    want = hs.astype(np.uint16).view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    # f32 -> f16 of every finite half value is the identity
    back = np.array([lib.paiq_f32_to_f16(float(v)) for v in want[fin]], np.uint32)
    assert np.array_equal(back, hs[fin])


def test_f32_to_f16_round_to_nearest_even():
    lib = pa.lib()
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(
            -9, 5, 20000).astype(np.float32),
        np.array([65504, 65519.99, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001,
                  3 * 2 ** -26, 6.1e-5, -0.0, 0.0, np.inf, -np.inf], np.float32)])
    got = np.array([lib.paiq_f32_to_f16(float(x)) for x in v], np.uint16)
    want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert lib.paiq_f32_to_f16(float("nan")) & 0x7C00 == 0x7C00


@pytest.mark.parametrize("qtype,encode", [(8, "orc_q8_0_encode_ref"), (2, "orc_q4_0_encode_ref")])
def test_q8_0_q4_0_match_textbook_encoders(qtype, encode):
    rng = np.random.default_rng(qtype)
    w = (rng.standard_normal((7, 512)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0  # all-zero block
    w[1, 5] = 3.0    # outlier
    got = pa.quantize(qtype, w)
    want = np.empty_like(got)
    getattr(ob.oracle(), encode)(w.ctypes.data, want.ctypes.data, w.size)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_textbook_encoders_hand_cases(sign):
    """Codes fixed by the definitions: Q8_0 scales a block by d = amax/127
    (f16), so its largest |x| takes code +-127; Q4_0 uses d = max/-8 with
    max the signed value of largest magnitude, which takes code 0 and
    dequantizes back to itself exactly when it is a power of two."""
    o = ob.oracle()
    x = np.full(32, 0.25 * sign, np.float32)
    x[3] = 1.0 * sign
    x[7] = 0.0
    q8 = np.empty(34, np.uint8)
    o.orc_q8_0_encode_ref(x.ctypes.data, q8.ctypes.data, 32)
    d = np.frombuffer(q8[:2].tobytes(), np.float16)[0]
    assert d == np.float16(np.float32(1.0) / np.float32(127.0))
    codes = q8[2:].view(np.int8)
    assert codes[3] == 127 * sign and codes[7] == 0
    q4 = np.empty(18, np.uint8)
    o.orc_q4_0_encode_ref(x.ctypes.data, q4.ctypes.data, 32)
    d4 = np.frombuffer(q4[:2].tobytes(), np.float16)[0]
    assert d4 == np.float16(-sign / 8.0)
    assert q4[2 + 3] & 0x0F == 0              # element 3 (low nibble of byte 3): code 0
    assert (q4[2 + 7] & 0x0F) == 8            # zero -> code 8
    assert ob.dequant(2, q4, 32)[3] == np.float32(sign)


def _bounds_check(qtype, w, blocks):
    qk = pa.BLOCK_ELEMS[qtype]
    deq = ob.dequant(qtype, blocks, w.size).reshape(w.shape)
    err = np.abs(deq - w)
    nblk = w.size // qk
    wb, eb = w.reshape(nblk, qk), err.reshape(nblk, qk)
    amax = np.abs(wb).max(axis=1)
    if qtype == 8:    # half a quantum of max/127, plus f16 rounding of d
        bound = amax / 127 * (0.5 + 2 ** -10 * 127)
    elif qtype == 2:  # half a quantum of max/8 (clipping at +7 adds one quantum)
        bound = amax / 8 * (1.0 + 2 ** -9 * 8)
    elif qtype == 12:  # per sub-block step (range/15), 6-bit scales, min rounding
        sub = w.reshape(-1, 32)
        step = (sub.max(1) - np.minimum(sub.min(1), 0)) / 15
        bound = np.repeat(step.reshape(nblk, 8).max(1) * 1.6 + amax / 63, 1)
    else:              # Q6_K: per 16-element group step max/32, int8 scales
        bound = amax / 32 * 1.2
    assert (eb <= bound[:, None] + 1e-12).all()
    return deq


@pytest.mark.parametrize("qtype", [8, 2, 12, 14])
def test_roundtrip_bounds_and_code_ranges(qtype):
    rng = np.random.default_rng(40 + qtype)
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    w[3] = np.abs(w[3])          # one-signed rows
    w[4] = -np.abs(w[4])
    w[5, :256] = 0.0             # zero super-block
    blocks = pa.quantize(qtype, w)
    deq = _bounds_check(qtype, w, blocks)
    assert not deq.reshape(16, 1024)[5, :256].any()
    rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
    assert rel < {8: 0.01, 2: 0.12, 12: 0.12, 14: 0.05}[qtype]


@pytest.mark.parametrize("qtype", [8, 2])
def test_reencode_is_idempotent(qtype):
    rng = np.random.default_rng(qtype)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    b1 = pa.quantize(qtype, w)
    d1 = ob.dequant(qtype, b1, w.size).reshape(w.shape)
    d2 = ob.dequant(qtype, pa.quantize(qtype, d1), w.size).reshape(w.shape)
    assert np.array_equal(d1, d2)


def test_quantize_errors_and_threads():
    w = np.zeros((3, 100), np.float32)
    with pytest.raises(pa.PaiError):
        pa.quantize(12, w)  # K not a multiple of 256
    rng = np.random.default_rng(9)
    w = rng.standard_normal((33, 512)).astype(np.float32)
    assert np.array_equal(pa.quantize(12, w, threads=1), pa.quantize(12, w, threads=5))


def test_normal_generator():
    a = pa.normal_f32(123, 1001)
    b = pa.normal_f32(123, 1001)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, pa.normal_f32(124, 1001))
    big = pa.normal_f32(123, 1 << 20, 0.0, 0.02)  # threaded path
    small = pa.normal_f32(123, 1 << 10, 0.0, 0.02)  # serial path, same stream
    assert np.array_equal(big[:1 << 10], small)
    assert abs(big.mean()) < 2e-4 and abs(big.std() - 0.02) < 2e-4
    assert np.array_equal(pa.normal_f32(123, 1001, 0.0, 1.0)[:1000], a[:1000])
