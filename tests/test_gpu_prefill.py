"""The prefill GEMMs (256 tokens and more per call) against the f64 oracle,
through the C-ABI: the kernel the dispatch picks per format (Q6_K: weights
dequantized once per workgroup into LDS, both MFMA operands from LDS;
the other formats: weights dequantized in registers, 128-token tiles), and
the LDS-shared kernel forced for every format (gemm_tile = 4).

Bars: rel-L2 <= 2e-3 with fp16 operands and <= 1.6e-2 with bf16, against
the f64 oracle; launches that are not split over K, or that sum their parts
in a fixed order, repeat bit for bit; the SiLU*mul epilogue is within 4 ulp
of the oracle's silu*mul applied to the same kernel's separate gate and up
products.
"""
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from prosperoai_amd import hipmem as hm

pytestmark = pytest.mark.gpu

TOL_F16, TOL_BF16 = 2e-3, 1.6e-2
QK = pa.BLOCK_ELEMS


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def device():
    say("[gpu] pai_hip_init")
    pa.init()
    yield


def weights(qtype: int, n: int, k: int, seed: int) -> np.ndarray:
    return pa.quantize(qtype, pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k))


def rel_l2(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def max_ulps(a: np.ndarray, b: np.ndarray) -> int:
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.abs(ia - ib).max())


def ragged_k(qtype: int) -> int:
    # 37 blocks of 32 (a partial 64-column stage) or 5 super-blocks
    return 32 * 37 if QK[qtype] == 32 else 256 * 5


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m,n", [(256, 200), (300, 1000), (520, 130)])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("kind", [0, 4])
def test_prefill_parity(qtype, m, n, bf16, kind):
    k = ragged_k(qtype)
    say(f"[gpu] prefill type={qtype} m={m} n={n} k={k} bf16={bf16} kind={kind}")
    blocks = weights(qtype, n, k, 0x9100 + 7 * m + qtype)
    x = pa.normal_f32(0x9200 + m, m * k).reshape(m, k)
    qm = pa.QMat(qtype, n, k, blocks)
    flags = pa.FLAG_MFMA_BF16 if bf16 else 0
    with pa.tuning(gemm_tile=kind):
        y = qm.gemm(x, flags)
        again = qm.gemm(x, flags)
    err = rel_l2(y, ob.qgemm_f64(qtype, n, k, blocks, x))
    assert 0.0 < err <= (TOL_BF16 if bf16 else TOL_F16), err
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("splits", [2, 3, 5])
def test_prefill_forced_splits(qtype, splits):
    """K split into uneven parts (36 stages of the LDS-shared kernel over 2,
    3 or 5 parts of a multiple of 4 stages), partial sums added into the
    zeroed output."""
    m, n, k = 300, 300, 256 * 9
    say(f"[gpu] prefill split={splits} type={qtype}")
    blocks = weights(qtype, n, k, 0x9300 + splits + qtype)
    x = pa.normal_f32(0x9301 + splits, m * k).reshape(m, k)
    with pa.tuning(gemm_splits=splits, gemm_tile=4):
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
    assert rel_l2(y, ob.qgemm_f64(qtype, n, k, blocks, x)) <= TOL_F16


@pytest.mark.parametrize("qtype", [2, 12])
def test_prefill_small_m_forced(qtype):
    """The prefill kernel forced at 100 tokens (a partly empty token tile)."""
    m, n, k = 100, 260, 256 * 4
    say(f"[gpu] prefill forced at m=100 type={qtype}")
    blocks = weights(qtype, n, k, 0x9400 + qtype)
    x = pa.normal_f32(0x9401, m * k).reshape(m, k)
    with pa.tuning(gemm_tile=4):
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
    assert rel_l2(y, ob.qgemm_f64(qtype, n, k, blocks, x)) <= TOL_F16


@pytest.mark.parametrize("qtype", [12, 14])
def test_prefill_multi_matrix(qtype):
    """q/k/v-shaped matrices in one launch at 300 tokens: K split in two
    with the parts summed in a fixed order; each output within the bar and a
    second call bit-identical."""
    m, k, shapes = 300, 2048, [512, 128, 128]
    say(f"[gpu] prefill multi type={qtype}")
    blocks = [weights(qtype, n, k, 0x9500 + 10 * i + qtype) for i, n in enumerate(shapes)]
    mats = [pa.QMat(qtype, n, k, b) for n, b in zip(shapes, blocks)]
    x = pa.normal_f32(0x9510, m * k).reshape(m, k)
    xd = hm.DeviceBuffer.from_array(x)
    yd = [hm.DeviceBuffer(m * n * 4) for n in shapes]
    st = hm.Stream()
    first = []
    for rep in range(2):
        pa.gemm_multi_async(mats, xd.ptr, [y.ptr for y in yd], m, 0, st.handle)
        st.synchronize()
        for i, (b, y, n) in enumerate(zip(blocks, yd, shapes)):
            got = y.download((m, n))
            if rep == 0:
                first.append(got)
                assert rel_l2(got, ob.qgemm_f64(qtype, n, k, b, x)) <= TOL_F16, n
            else:
                assert np.array_equal(got.view(np.uint32), first[i].view(np.uint32)), n
    st.destroy()
    for b in [xd, *yd]:
        b.free()


@pytest.mark.parametrize("qtype", [12, 2, 14])
def test_prefill_gate_up_epilogue(qtype):
    """h = silu(x Wg^T) * (x Wu^T) at 300 tokens: the up launch forms the
    product from the gate output it reads back."""
    m, n, k = 300, 700, 1024
    say(f"[gpu] prefill gate/up type={qtype}")
    bg, bu = weights(qtype, n, k, 0x9600 + qtype), weights(qtype, n, k, 0x9601 + qtype)
    wg, wu = pa.QMat(qtype, n, k, bg), pa.QMat(qtype, n, k, bu)
    x = pa.normal_f32(0x9602, m * k).reshape(m, k)
    xd = hm.DeviceBuffer.from_array(x)
    hd = hm.DeviceBuffer(m * n * 4)
    st = hm.Stream()
    pa.gate_up_async(wg, wu, xd.ptr, hd.ptr, m, 0, st.handle)
    st.synchronize()
    h = hd.download((m, n))
    g, u = wg.gemm(x), wu.gemm(x)
    assert max_ulps(h, ob.silu_mul(g, u)) <= 4
    ref = ob.silu_mul(ob.qgemm_f64(qtype, n, k, bg, x).astype(np.float32),
                      ob.qgemm_f64(qtype, n, k, bu, x).astype(np.float32))
    assert rel_l2(h, ref) <= TOL_F16
    st.destroy()
    xd.free()
    hd.free()


def test_prefill_token_blocks_past_workspace():
    """1100 tokens: the 16-bit workspace holds 1024, so the call runs as a
    1024-token block on the prefill kernel and a 76-token block on the
    batched kernel; sampled tokens against the oracle."""
    qtype, m, n, k = 12, 1100, 384, 1024
    say("[gpu] prefill m=1100")
    blocks = weights(qtype, n, k, 0x9700)
    x = pa.normal_f32(0x9701, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x)
    toks = np.r_[np.arange(0, 1024, 61), np.arange(1024, m, 7)]
    ref = ob.qgemm_f64(qtype, n, k, blocks, x[toks])
    assert rel_l2(y[toks], ref) <= TOL_F16
