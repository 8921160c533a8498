"""Fused feed-forward gate/up (pai_qgemm_f32_gate_up_async) against the
reference's four-op composition GEMM(gate), GEMM(up), SILU, MUL.

Bars:
  M < 8   h within 4 ulp (elementwise) of the oracle's silu*mul applied to
          the GPU's separate gate and up products of the same tokens, which
          the fused launch reproduces bit for bit; and rel-L2 <= 1e-5
          against the oracle's sequential f32 composition.
  M >= 8  with the launches unsplit on both sides, the same 4-ulp bar; by
          default rel-L2 <= 2e-3 (fp16 operands) against the f64 oracle
          products passed through the oracle's silu*mul.
"""
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa

pytestmark = pytest.mark.gpu

TOL_F32, TOL_F16 = 1e-5, 2e-3


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def device():
    say("[gpu] pai_hip_init")
    pa.init()
    yield


def weights(qtype: int, n: int, k: int, seed: int) -> np.ndarray:
    w = pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    return pa.quantize(qtype, w)


def rel_l2(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def max_ulps(a: np.ndarray, b: np.ndarray) -> int:
    """Largest distance in units of the last place between finite f32 arrays."""
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)  # sign-magnitude -> monotone
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.abs(ia - ib).max())


def run(qtype, n, k, m, seed, flags=0):
    from prosperoai_amd.hipmem import DeviceBuffer, Stream
    bg, bu = weights(qtype, n, k, seed), weights(qtype, n, k, seed + 1)
    wg, wu = pa.QMat(qtype, n, k, bg), pa.QMat(qtype, n, k, bu)
    x = pa.normal_f32(seed + 2, m * k).reshape(m, k)
    xd, hd = DeviceBuffer.from_array(x), DeviceBuffer(m * n * 4)
    st = Stream()
    pa.gate_up_async(wg, wu, xd.ptr, hd.ptr, m, flags, st.handle)
    st.synchronize()
    h = hd.download((m, n))
    # separate calls with the same tokens: they take the same kernel and
    # token grouping as the fused launch (one token: the integer-dot GEMV;
    # 2..7 tokens: the matrix-core GEMV where it takes K, both summing each
    # row in one pass; from 8 tokens: the MFMA GEMM)
    g_sep, u_sep = wg.gemm(x, flags), wu.gemm(x, flags)
    st.destroy()
    return h, g_sep, u_sep, bg, bu, x


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 7])
def test_gemv_gate_up_matches_composition(qtype, m):
    n, k = 200, 1024  # 200 rows: ragged against every row-group size
    say(f"[gpu] gate_up gemv type={qtype} m={m}")
    h, g, u, bg, bu, x = run(qtype, n, k, m, 4000 + 10 * qtype + m)
    assert max_ulps(h, ob.silu_mul(g, u)) <= 4
    ref = ob.silu_mul(ob.qgemm_seq(qtype, n, k, bg, x), ob.qgemm_seq(qtype, n, k, bu, x))
    assert rel_l2(h, ref) <= TOL_F32


def test_gemv_gate_up_llama8b_shape():
    """gate/up of Llama-3-8B (14336 x 4096, Q4_K) at M = 1."""
    say("[gpu] gate_up gemv llama shape")
    h, g, u, *_ = run(12, 14336, 4096, 1, 4242)
    assert max_ulps(h, ob.silu_mul(g, u)) <= 4


def test_gemv_gate_up_longest_rows():
    """K = 18720, the longest row one launch holds at M = 1 (585 chunks),
    and 9344 at M = 2 and 4672 at M = 4 through token groups."""
    say("[gpu] gate_up gemv long rows")
    for m, k in ((1, 18720), (3, 9344), (6, 4672)):
        h, g, u, *_ = run(8, 96, k, m, 4300 + m)
        assert max_ulps(h, ob.silu_mul(g, u)) <= 4, (m, k)


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [8, 33, 300])
def test_mfma_gate_up_unsplit_matches_composition(qtype, m):
    n, k = 320, 1024
    say(f"[gpu] gate_up mfma unsplit type={qtype} m={m}")
    with pa.tuning(gemm_splits=1):
        h, g, u, *_ = run(qtype, n, k, m, 5000 + 10 * qtype + m)
    assert max_ulps(h, ob.silu_mul(g, u)) <= 4


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("m,k", [(8, 2048), (64, 2048), (32, 4096)])
def test_mfma_gate_up_against_f64_oracle(qtype, m, k):
    # With 32 and 64 tokens both products split over K (few row tiles): the
    # up product goes to the handle's workspace and a third launch forms
    # silu(gate) * up.
    n = 1024
    say(f"[gpu] gate_up mfma type={qtype} m={m}")
    h, g, u, bg, bu, x = run(qtype, n, k, m, 6000 + qtype + m)
    ref = ob.silu_mul(ob.qgemm_f64(qtype, n, k, bg, x).astype(np.float32),
                      ob.qgemm_f64(qtype, n, k, bu, x).astype(np.float32))
    assert rel_l2(h, ref) <= TOL_F16


def test_mfma_gate_up_split_workspace_regrows():
    """The split-K gate/up path keeps the split parts in a workspace owned by
    the gate matrix's handle and forms silu(gate) * up while summing them in
    a fixed order; calls with more tokens on the same handles grow the
    workspace, every call stays within the 16-bit bar of the f64 oracle, and
    a repeated call gives the same bits."""
    from prosperoai_amd.hipmem import DeviceBuffer, Stream
    qtype, n, k = 12, 1024, 4096
    say("[gpu] gate_up split workspace regrow")
    bg, bu = weights(qtype, n, k, 7100), weights(qtype, n, k, 7101)
    wg, wu = pa.QMat(qtype, n, k, bg), pa.QMat(qtype, n, k, bu)
    st = Stream()
    for m in (16, 48, 32):
        x = pa.normal_f32(7102 + m, m * k).reshape(m, k)
        xd, hd = DeviceBuffer.from_array(x), DeviceBuffer(m * n * 4)
        pa.gate_up_async(wg, wu, xd.ptr, hd.ptr, m, 0, st.handle)
        st.synchronize()
        h1 = hd.download((m, n))
        ref = ob.silu_mul(ob.qgemm_f64(qtype, n, k, bg, x).astype(np.float32),
                          ob.qgemm_f64(qtype, n, k, bu, x).astype(np.float32))
        assert rel_l2(h1, ref) <= TOL_F16, m
        pa.gate_up_async(wg, wu, xd.ptr, hd.ptr, m, 0, st.handle)
        st.synchronize()
        assert np.array_equal(hd.download((m, n)).view(np.uint32), h1.view(np.uint32)), m
    st.destroy()


def test_gate_up_argument_errors():
    from prosperoai_amd.hipmem import DeviceBuffer
    say("[gpu] gate_up errors")
    a = pa.QMat(12, 64, 512, weights(12, 64, 512, 1))
    b = pa.QMat(12, 32, 512, weights(12, 32, 512, 2))
    c = pa.QMat(14, 64, 512, weights(14, 64, 512, 3))
    xd, hd = DeviceBuffer(4 * 512 * 4), DeviceBuffer(4 * 64 * 4)
    for other in (b, c):
        with pytest.raises(pa.PaiError) as e:
            pa.gate_up_async(a, other, xd.ptr, hd.ptr, 1)
        assert e.value.status == -6
    with pytest.raises(pa.PaiError) as e:
        pa.gate_up_async(a, a, xd.ptr, hd.ptr, 0)
    assert e.value.status == -1
    big = pa.QMat(8, 8, 18752, weights(8, 8, 18752, 4))
    xb, hb = DeviceBuffer(18752 * 4), DeviceBuffer(8 * 4)
    with pytest.raises(pa.PaiError) as e:
        pa.gate_up_async(big, big, xb.ptr, hb.ptr, 1)
    assert e.value.status == -3
