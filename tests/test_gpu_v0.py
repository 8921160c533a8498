"""The v0 per-group formats on the GPU, through the C-ABI, against the oracle
(restating models/quantize.c and cpu/reference/ref_ops.c:446-499, itself
bit-equal to the reference build).

Bars:
  quantize / dequantize   bit-exact (codes, scale bits, values); NaN
                          results compare as NaN (their sign and payload
                          come from the host FPU in the reference);
  GEMM, strip kernel      rel-L2 <= 1e-5 against the f64 sums and against
                          the reference's sequential f32 result, and
                          repeatable bit for bit;
  GEMM, sequential kernel bit-exact against the reference's sum.

Weights of the 4096 x 4096 case are f32 N(0, 0.02^2) from a fixed seed,
quantized per column in groups of 32 rows by the oracle's quantizer (as
tests/test_quantize.c:155-176 builds them); activations are N(0, 1).
"""
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from prosperoai_amd import hipmem as hm
from prosperoai_amd import v0

pytestmark = pytest.mark.gpu

TOL = 1e-5


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def device():
    say("[gpu] pai_hip_init")
    pa.init()
    yield


def kn_operands(w: np.ndarray, bits: int, gs: int):
    """[K][N] codes and [G][N] scales: each column of w quantized in groups
    of gs rows (K a multiple of gs, or gs = 0), through the flat quantizer
    on W^T (whose groups are then exactly (column, row group))."""
    k, n = w.shape
    assert gs == 0 or k % gs == 0
    g = k if gs == 0 else gs  # one group per column when gs = 0 (per-tensor over k)
    q, s = ob.v0_quantize(np.ascontiguousarray(w.T), bits, g)
    ng = k // g
    scales = np.ascontiguousarray(s.reshape(n, ng).T)
    if bits == 8:
        return np.ascontiguousarray(q.reshape(n, k).T), scales
    u = q.view(np.uint8)
    codes_t = np.stack([u & 15, u >> 4], 1).reshape(n, k)           # nibbles of W^T
    flat = np.ascontiguousarray(codes_t.T).ravel()                   # [K][N] flat order
    if flat.size % 2:
        flat = np.r_[flat, np.uint8(0)]
    return (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8).view(np.int8), scales


def rel_l2(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


@pytest.mark.parametrize("bits", [8, 4])
def test_gemm_4096_group32_one_token(bits):
    n = k = 4096
    say(f"[gpu] v0 gemm w{bits} 4096x4096 gs32 m=1")
    w = pa.normal_f32(0xC0DE0010 + bits, n * k, 0.0, 0.02).reshape(k, n)
    w_q, sc = kn_operands(w, bits, 32)
    x = pa.normal_f32(0xC0DE0019, k).reshape(1, k)
    c = v0.gemm(bits, x, w_q, sc, n, 32)
    assert rel_l2(c, ob.gemm_wq_f64(bits, x, w_q, sc, n, 32)) <= TOL
    assert rel_l2(c, ob.gemm_wq_seq(bits, x, w_q, sc, n, 32)) <= TOL
    again = v0.gemm(bits, x, w_q, sc, n, 32)
    assert np.array_equal(again.view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("m", [2, 3, 5, 8, 33])
@pytest.mark.parametrize("gs", [16, 64, 0])
def test_gemm_tokens_and_groups(bits, m, gs):
    """n = 1296 (a last strip of 16 columns), k = 1024 + 64 + 16 (a last
    block of 16 rows; gs 64 leaves a partial last group)."""
    n, k = 1296, 1104
    say(f"[gpu] v0 gemm w{bits} m={m} gs={gs}")
    rng = np.random.default_rng(bits * 100 + m + gs)
    w_bytes = k * n if bits == 8 else k * n // 2
    w_q = rng.integers(-128, 128, w_bytes).astype(np.int8)
    g = k if gs == 0 else gs
    sc = rng.uniform(0.001, 0.03, (-(-k // g), n)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    c = v0.gemm(bits, x, w_q, sc, n, gs)
    assert rel_l2(c, ob.gemm_wq_f64(bits, x, w_q, sc, n, gs)) <= TOL
    assert np.array_equal(v0.gemm(bits, x, w_q, sc, n, gs).view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("m,n,k,gs,forced", [(3, 33, 70, 7, False), (2, 15, 64, 32, False),
                                             (1, 7, 9, 100, False), (2, 64, 128, 32, True),
                                             (4, 48, 200, 0, True)])
def test_gemm_sequential_kernel_bit_exact(bits, m, n, k, gs, forced):
    """Shapes the strip kernel does not take (n % 16, gs % 16), and the
    one-thread-per-output kernel forced on shapes it would take."""
    say(f"[gpu] v0 gemm seq w{bits} m={m} n={n} k={k} gs={gs}")
    rng = np.random.default_rng(m * 7 + n + k + bits)
    w_q = rng.integers(-128, 128, k * n if bits == 8 else (k * n + 1) // 2).astype(np.int8)
    g = k if (gs == 0 or gs > k) else gs
    sc = rng.uniform(0.001, 0.03, (-(-k // g), n)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    with pa.tuning(v0_sequential=1 if forced else 0):
        c = v0.gemm(bits, x, w_q, sc, n, gs)
    want = ob.gemm_wq_seq(bits, x, w_q, sc, n, gs)
    assert np.array_equal(c.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [8, 4])
def test_gemm_async_workspace_sizes(bits):
    """Device pointers on a stream: the full workspace (split K, parts summed
    in order), a workspace that fits fewer parts, and none (no split)."""
    m, n, k, gs = 1, 2048, 4096, 32
    say(f"[gpu] v0 gemm async w{bits}")
    rng = np.random.default_rng(11 + bits)
    w_q = rng.integers(-127, 128, k * n if bits == 8 else k * n // 2).astype(np.int8)
    sc = rng.uniform(0.001, 0.03, (k // gs, n)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = ob.gemm_wq_f64(bits, x, w_q, sc, n, gs)
    xd, wd, sd = (hm.DeviceBuffer.from_array(a) for a in (x, w_q, sc))
    cd = hm.DeviceBuffer(m * n * 4)
    ws = hm.DeviceBuffer(v0.WORKSPACE_BYTES)
    st = hm.Stream()
    outs = []
    for ws_ptr, ws_bytes in ((ws.ptr, v0.WORKSPACE_BYTES), (ws.ptr, 4 * m * n * 3), (None, 0)):
        for _ in range(2):
            v0.gemm_async(bits, m, n, k, xd.ptr, wd.ptr, sd.ptr, gs, cd.ptr, ws_ptr, ws_bytes,
                          st.handle)
            st.synchronize()
            outs.append(cd.download((m, n)))
        assert np.array_equal(outs[-1].view(np.uint32), outs[-2].view(np.uint32))
        assert rel_l2(outs[-1], ref) <= TOL
    st.destroy()
    for b in (xd, wd, sd, cd, ws):
        b.free()


def special_input(n: int, gs: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    g = n if gs == 0 else gs
    if n >= 4 * g and g >= 4:
        x[:g] = 0.0                                       # a zero group
        x[g:2 * g] = rng.standard_normal(g).astype(np.float32) * np.float32(1e-41)  # subnormal
        x[2 * g + 1] = np.nan                             # NaN is skipped by the maximum
        x[3 * g + 2] = np.inf                             # an infinite maximum
        x[3 * g + 3] = -0.0
    return x


def same_values(a: np.ndarray, b: np.ndarray) -> bool:
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                          b[~nb].view(np.uint32)))


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("n,gs", [(1, 0), (17, 5), (4097, 32), (40000, 0), (40000, 20000),
                                  (100003, 1), (65536, 64), (4099, 4100)])
def test_quantize_dequantize_bit_exact(bits, n, gs):
    say(f"[gpu] v0 quantize w{bits} n={n} gs={gs}")
    x = special_input(n, gs, n + gs + bits)
    q, s = v0.quantize(x, bits, gs)
    rq, rs = ob.v0_quantize(x, bits, gs)
    assert np.array_equal(q, rq)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    d = v0.dequantize(q, s, n, bits, gs)
    assert same_values(d, ob.v0_dequantize(rq, rs, n, bits, gs))


def test_quantize_reference_cases_on_gpu():
    """tests/test_quantize.c:79-117 through the GPU entry points."""
    q, s = v0.quantize(np.array([0.0, 100.0, -100.0, 100.0], np.float32), 8, 0)
    assert q.tolist() == [0, 127, -127, 127] and s[0] == np.float32(100) / np.float32(127)
    q, s = v0.quantize(np.array([0.0, 2.0, -2.0, 1.0], np.float32), 4, 0)
    assert q.view(np.uint8).tolist() == [0x70, 0x39]
    q, s = v0.quantize(np.array([4.0, -4.0, 4.0], np.float32), 4, 0)
    assert q.view(np.uint8).tolist() == [0x97, 0x07]
    d = v0.dequantize(q, s, 3, 4, 0)
    assert np.all(np.abs(d - [4, -4, 4]) < 1e-4)


def test_session_load_of_a_v0_tensor():
    """models/model.c:264-290 on the device: a q4 blob of a 1024 x 4096
    weight (values then scales, group 64) dequantized into f32, equal to the
    reference's pai_dequantize_f32 restated by the oracle."""
    n, gs = 1024 * 4096, 64
    say("[gpu] v0 session load")
    w = pa.normal_f32(0xC0DE0031, n, 0.0, 0.02)
    q, s = ob.v0_quantize(w, 4, gs)
    d = v0.dequantize(q, s, n, 4, gs)
    assert np.array_equal(d.view(np.uint32), ob.v0_dequantize(q, s, n, 4, gs).view(np.uint32))
