"""GPU parity: every kernel of libpai_hip.so against the CPU oracle, called
through the C-ABI.

Bars:
  dequant                      bit-exact (NaN outputs compared as NaN)
  M < 8 and PAI_QGEMM_FP32     rel-L2 <= 1e-5 vs the reference's sequential
                               f32 operator (and vs the f64 oracle)
  M >= 8 MFMA                  rel-L2 <= 2e-3 (fp16 operands), 1.6e-2 (bf16)
                               vs the f64 oracle
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa

pytestmark = pytest.mark.gpu

TOL_F32, TOL_F16, TOL_BF16 = 1e-5, 2e-3, 1.6e-2
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
    w = pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    return pa.quantize(qtype, w)


def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("n,nblk", [(1, 1), (5, 3), (64, 16), (33, 7)])
def test_dequant_bit_exact(qtype, n, nblk):
    import make_golden
    say(f"[gpu] dequant type={qtype} n={n} blocks/row={nblk}")
    rng = np.random.default_rng(1000 * qtype + n + nblk)
    k = nblk * QK[qtype]
    raw = make_golden.random_blocks(rng, qtype, n * nblk).reshape(n, -1)
    w = pa.QMat(qtype, n, k, raw)
    got = w.dequant()
    want = ob.dequant(qtype, raw, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_every_f16_scale():
    """Q8_0 rows whose scale runs over all 65536 f16 patterns."""
    say("[gpu] dequant all f16 scales")
    n = 65536
    blk = np.zeros((n, 34), np.uint8)
    h = np.arange(n, dtype=np.uint32)
    blk[:, 0] = (h & 0xFF).astype(np.uint8)
    blk[:, 1] = (h >> 8).astype(np.uint8)
    codes = np.array([1, -1, 127, -128, 0, 2, 3, -7] * 4, np.int8)
    blk[:, 2:] = codes.view(np.uint8)
    got = pa.QMat(8, n, 32, blk).dequant()
    want = ob.dequant(8, blk, n * 32).reshape(n, 32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_dequant_hand_vectors():
    import json
    from pathlib import Path
    say("[gpu] dequant reference hand vectors")
    d = json.loads((Path(__file__).parent / "golden" / "gguf_hand_vectors.json").read_text())
    for c in d["cases"]:
        raw = np.frombuffer(bytes.fromhex(c["raw"]), np.uint8)
        got = pa.QMat(c["type"], 1, c["numel"], raw).dequant()[0]
        assert np.array_equal(got, np.asarray(c["expect"], np.float32)), c["name"]


# ------------------------------------------------------------------ M = 1 GEMV
SHAPES_M1 = [
    (1, None), (7, None), (33, 3), (129, 9), (1000, 65), (64, 448),  # K in blocks
]


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("n,kb", SHAPES_M1)
def test_gemv_m1_parity(qtype, n, kb):
    qk = QK[qtype]
    k = qk * (kb if kb is not None else (1 if qk == 256 else 3))
    say(f"[gpu] gemv M=1 type={qtype} n={n} k={k}")
    blocks = weights(qtype, n, k, 7 * n + k + qtype)
    x = pa.normal_f32(99 + k, k).reshape(1, k)
    w = pa.QMat(qtype, n, k, blocks)
    y = w.gemm(x)
    ref = ob.qgemm_seq(qtype, n, k, blocks, x)
    ref64 = ob.qgemm_f64(qtype, n, k, blocks, x)
    assert rel_l2(y, ref) <= TOL_F32
    assert rel_l2(y, ref64) <= TOL_F32


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
def test_gemv_one_hot_returns_exact_column(qtype):
    n, k = 70, 4 * QK[qtype] if QK[qtype] == 256 else 2048 + 64
    say(f"[gpu] gemv one-hot type={qtype}")
    blocks = weights(qtype, n, k, 5 + qtype)
    w = pa.QMat(qtype, n, k, blocks)
    deq = ob.dequant(qtype, blocks, n * k).reshape(n, k)
    for j in (0, 17, k // 2 + 5, k - 1):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        assert np.array_equal(w.gemm(x)[0], deq[:, j])


LLAMA8B = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
           "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}


@pytest.mark.parametrize("qtype", [2, 12])
@pytest.mark.parametrize("proj", ["k", "o", "gate", "down"])
def test_gemv_llama8b_shapes(qtype, proj):
    n, k = LLAMA8B[proj]
    say(f"[gpu] gemv 8B shape type={qtype} proj={proj} n={n} k={k}")
    blocks = weights(qtype, n, k, 0xC0DE0000 + 16 * 2 + list(LLAMA8B).index(proj))
    x = pa.normal_f32(0x5A5A, k).reshape(1, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x)
    assert rel_l2(y, ob.qgemm_seq(qtype, n, k, blocks, x)) <= TOL_F32


def test_gemv_q8_0_config1_and_q6_k_down():
    for qtype, (n, k) in ((8, (4096, 4096)), (14, (4096, 14336))):
        say(f"[gpu] gemv type={qtype} n={n} k={k}")
        blocks = weights(qtype, n, k, 0xC0DE0010 + qtype)
        x = pa.normal_f32(0xC0DE0010 ^ 0x5A5A, k).reshape(1, k)
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
        assert rel_l2(y, ob.qgemm_seq(qtype, n, k, blocks, x)) <= TOL_F32


# ------------------------------------------------------------------ small batch
@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 7, 8])
def test_small_batch_parity(qtype, m):
    n, k = 300, 2 * QK[qtype] * (8 if QK[qtype] == 32 else 1)
    say(f"[gpu] gemm M={m} type={qtype} n={n} k={k}")
    blocks = weights(qtype, n, k, 31 * m + qtype)
    x = pa.normal_f32(3 * m, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x)
    ref = ob.qgemm_seq(qtype, n, k, blocks, x)
    for i in range(m):
        assert rel_l2(y[i], ref[i]) <= TOL_F32, i


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("n,k", [(1000, 4096), (777, 7168)])
def test_gemv_launch_shapes_same_bits(qtype, n, k):
    """The one-token GEMV's launch shape (rows per group 1, 2 or 4, which
    sets the ring to 4, 2 or 1 blocks; 8- or 16-wave workgroups; grid
    size) changes which wave owns a row, never a row's summation order:
    every shape gives the same bits, within 1e-5 of the reference."""
    say(f"[gpu] gemv launch shapes type={qtype} n={n} k={k}")
    blocks = weights(qtype, n, k, 5 * n + qtype)
    x = pa.normal_f32(41 + k, k).reshape(1, k)
    w = pa.QMat(qtype, n, k, blocks)
    y0 = w.gemm(x)
    assert rel_l2(y0, ob.qgemm_seq(qtype, n, k, blocks, x)) <= TOL_F32
    shapes = [{"gemv_rows": 1}, {"gemv_rows": 2}, {"gemv_rows": 4}, {"gemv_nw": 8},
              {"gemv_nw": 16}, {"gemv_wgs": 37}, {"gemv_wgs": 256, "gemv_rows": 1}]
    for kw in shapes:
        with pa.tuning(**kw):
            y = w.gemm(x)
        assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), kw
    w.free()


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [2, 3, 4, 7])
def test_integer_dot_token_groups(qtype, m):
    """Calls of 2..8 tokens on the integer-dot kernel's token groups (2 or 4
    tokens per launch) instead of the matrix cores: the reference's bar."""
    n, k = 257, 4096
    say(f"[gpu] gemv token groups type={qtype} m={m}")
    blocks = weights(qtype, n, k, 11 * m + qtype)
    x = pa.normal_f32(7 * m + k, m * k).reshape(m, k)
    w = pa.QMat(qtype, n, k, blocks)
    with pa.tuning(gemv_no_mx=1):
        y = w.gemm(x)
    ref = ob.qgemm_seq(qtype, n, k, blocks, x)
    for i in range(m):
        assert rel_l2(y[i], ref[i]) <= TOL_F32, i
    w.free()


@pytest.mark.parametrize("qtype", [2, 12])
def test_batched_decode_llama8b_m8(qtype):
    """Eight tokens at the 8B shapes: q (K = 4096) takes the matrix-core
    GEMV (one launch covers the tokens), down (K = 14336) the 16-bit GEMM."""
    m = 8
    for proj, tol in (("q", TOL_F32), ("gate", TOL_F32), ("down", TOL_F16)):
        n, k = LLAMA8B[proj]
        say(f"[gpu] batched decode M=8 type={qtype} proj={proj}")
        blocks = weights(qtype, n, k, 0xC0DE0100 + list(LLAMA8B).index(proj))
        x = pa.normal_f32(0xC0DE0100 ^ 0x5A5A, m * k).reshape(m, k)
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
        rows = np.arange(0, n, 7)
        ref = ob.qgemm_f64(qtype, len(rows), k, blocks[rows], x)
        assert rel_l2(y[:, rows], ref) <= tol, proj


def test_batched_gemv_longer_rows_fewer_tokens():
    """K = 14336 holds 2 tokens per matrix-core launch: 5 tokens run as
    launches of 2, 2 and 1; K = 9344 (73 steps) splits unevenly over waves."""
    for qtype, n, k, m in ((14, 100, 14336, 5), (2, 64, 9344, 3)):
        say(f"[gpu] batched gemv type={qtype} k={k} m={m}")
        blocks = weights(qtype, n, k, 4400 + m)
        x = pa.normal_f32(4401 + m, m * k).reshape(m, k)
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
        assert rel_l2(y, ob.qgemm_seq(qtype, n, k, blocks, x)) <= TOL_F32


# ------------------------------------------------------------------ MFMA path
@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [12, 31, 32, 33, 64, 100, 300])
@pytest.mark.parametrize("bf16", [False, True])
def test_mfma_parity(qtype, m, bf16):
    n, k = 200, 3 * 256
    say(f"[gpu] gemm MFMA M={m} type={qtype} bf16={bf16} n={n} k={k}")
    blocks = weights(qtype, n, k, 17 * m + qtype)
    x = pa.normal_f32(5 * m + 1, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x, pa.FLAG_MFMA_BF16 if bf16 else 0)
    ref64 = ob.qgemm_f64(qtype, n, k, blocks, x)
    err = rel_l2(y, ref64)
    assert err <= (TOL_BF16 if bf16 else TOL_F16), err
    assert err > 0.0  # it really is the reduced-precision path


def test_mfma_ragged_k_for_32_blocks():
    """Q4_0/Q8_0 with K not a multiple of the 256-column tile."""
    for qtype in (2, 8):
        n, k, m = 77, 32 * 11, 40
        say(f"[gpu] gemm MFMA ragged K type={qtype}")
        blocks = weights(qtype, n, k, 3 + qtype)
        x = pa.normal_f32(11, m * k).reshape(m, k)
        y = pa.QMat(qtype, n, k, blocks).gemm(x)
        assert rel_l2(y, ob.qgemm_f64(qtype, n, k, blocks, x)) <= TOL_F16


def test_fp32_flag_gives_reference_precision_at_large_m():
    qtype, n, k, m = 12, 96, 512, 48
    say("[gpu] gemm FP32 flag M=48")
    blocks = weights(qtype, n, k, 77)
    x = pa.normal_f32(78, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x, pa.FLAG_FP32)
    ref = ob.qgemm_seq(qtype, n, k, blocks, x)
    assert rel_l2(y, ref) <= TOL_F32


def test_prefill_shape_gate_q4k_m512():
    qtype, (n, k), m = 12, LLAMA8B["gate"], 512
    say("[gpu] prefill gate M=512")
    blocks = weights(qtype, n, k, 0xC0DE0040)
    x = pa.normal_f32(0xC0DE0040 ^ 0x5A5A, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x)
    rows = np.arange(0, m, 37)
    ref = ob.qgemm_f64(qtype, n, k, blocks, x[rows])
    assert rel_l2(y[rows], ref) <= TOL_F16


def test_prefill_shape_down_q6k_m512():
    """Few output tiles: the K range is split across workgroups."""
    qtype, (n, k), m = 14, LLAMA8B["down"], 512
    say("[gpu] prefill down Q6_K M=512 (split K)")
    blocks = weights(qtype, n, k, 0xC0DE0046)
    x = pa.normal_f32(0xC0DE0046 ^ 0x5A5A, m * k).reshape(m, k)
    y = pa.QMat(qtype, n, k, blocks).gemm(x)
    rows = np.arange(3, m, 41)
    ref = ob.qgemm_f64(qtype, n, k, blocks, x[rows])
    assert rel_l2(y[rows], ref) <= TOL_F16


@pytest.mark.parametrize("splits", [2, 3, 7])
def test_mfma_forced_split_k_ragged(splits):
    """K split into uneven ranges, last step with a single chunk."""
    for qtype, m in ((2, 70), (8, 33)):
        n, k = 300, 32 * 37
        say(f"[gpu] gemm MFMA split={splits} type={qtype} m={m}")
        blocks = weights(qtype, n, k, 90 + splits + qtype)
        x = pa.normal_f32(91 + splits, m * k).reshape(m, k)
        with pa.tuning(gemm_splits=splits):
            y = pa.QMat(qtype, n, k, blocks).gemm(x)
        assert rel_l2(y, ob.qgemm_f64(qtype, n, k, blocks, x)) <= TOL_F16


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
@pytest.mark.parametrize("m", [40, 300])
def test_mfma_16bit_copy_matches_register_staging(qtype, m):
    """The activations reach LDS either from the matrix's 16-bit workspace
    (DMA) or through registers; both round x and the weights the same way.
    Below 256 tokens both kernels also accumulate in the same order, so the
    outputs are identical; from 256 tokens the workspace path runs the
    LDS-shared prefill kernel, whose MFMAs group the columns differently:
    the f32 sums agree to rel-L2 1e-5."""
    n, k = 300, 32 * 37 if QK[qtype] == 32 else 256 * 5
    say(f"[gpu] gemm MFMA x16 vs registers type={qtype} m={m}")
    blocks = weights(qtype, n, k, 120 + qtype)
    x = pa.normal_f32(121 + m, m * k).reshape(m, k)
    qm = pa.QMat(qtype, n, k, blocks)
    y16 = qm.gemm(x)
    with pa.tuning(gemm_no_x16=1):
        yreg = qm.gemm(x)
    if m < 256:
        assert np.array_equal(y16, yreg)
    else:
        assert rel_l2(y16, yreg) <= 1e-5
    assert rel_l2(y16, ob.qgemm_f64(qtype, n, k, blocks, x)) <= TOL_F16


# ------------------------------------------------------------------ device pointers
def test_device_pointer_path_matches_host_path():
    from prosperoai_amd.hipmem import DeviceBuffer, Stream
    qtype, n, k = 12, 512, 2048
    say("[gpu] device-pointer path")
    blocks = weights(qtype, n, k, 4)
    w = pa.QMat(qtype, n, k, blocks)
    stream = Stream()
    for m in (1, 3, 40):
        x = pa.normal_f32(m, m * k).reshape(m, k)
        xd = DeviceBuffer.from_array(x)
        yd = DeviceBuffer(m * n * 4)
        w.gemm_async(xd.ptr, yd.ptr, m, 0, stream.handle)
        stream.synchronize()
        assert np.array_equal(yd.download((m, n)), w.gemm(x))
    stream.destroy()


def test_upload_from_device_blocks():
    from prosperoai_amd.hipmem import DeviceBuffer
    qtype, n, k = 14, 40, 512
    say("[gpu] upload from device")
    blocks = weights(qtype, n, k, 8)
    dev = DeviceBuffer.from_array(blocks.reshape(-1))
    w2 = pa.QMat(qtype, n, k, None, device_ptr=dev.ptr)
    assert np.array_equal(w2.dequant(), pa.QMat(qtype, n, k, blocks).dequant())


def test_gpu_argument_errors():
    from prosperoai_amd.hipmem import DeviceBuffer
    say("[gpu] argument errors")
    lib = pa.lib()
    w = pa.QMat(2, 8, 64, weights(2, 8, 64, 1))
    x = DeviceBuffer(65 * 4)
    y = DeviceBuffer(16 * 4)
    assert lib.pai_qgemm_f32_async(w.handle, 0, x.ptr, y.ptr, 1, None) == -1
    assert lib.pai_qgemm_f32_async(w.handle, 1, x.ptr + 4, y.ptr, 1, None) == -1
    assert lib.pai_qgemm_f32_async(w.handle, 1, None, y.ptr, 1, None) == -1
    t, nn, kk = C.c_uint32(), C.c_uint64(), C.c_uint64()
    assert lib.pai_qmat_shape(w.handle, C.byref(t), C.byref(nn), C.byref(kk)) == 0
    assert (t.value, nn.value, kk.value) == (2, 8, 64)
    assert w.nbytes == 8 * 36


# ------------------------------------------------------------------ fused projections
@pytest.mark.parametrize("qtype", [2, 12, 14])
@pytest.mark.parametrize("m", [1, 3, 40])
def test_multi_matches_separate_calls(qtype, m):
    """q/k/v-shaped matrices in one fused call give the same bits as three
    separate calls (and the oracle's values within the f32 bar)."""
    from prosperoai_amd.hipmem import DeviceBuffer, Stream
    k = 1024
    shapes = [512, 128, 128]
    say(f"[gpu] multi type={qtype} m={m}")
    mats, blocks = [], []
    for i, n in enumerate(shapes):
        b = weights(qtype, n, k, 900 + 10 * i + qtype)
        blocks.append(b)
        mats.append(pa.QMat(qtype, n, k, b))
    x = pa.normal_f32(77 + m, m * k).reshape(m, k)
    xd = DeviceBuffer.from_array(x)
    yd = [DeviceBuffer(m * n * 4) for n in shapes]
    st = Stream()
    pa.gemm_multi_async(mats, xd.ptr, [y.ptr for y in yd], m, 0, st.handle)
    st.synchronize()
    for w, b, y, n in zip(mats, blocks, yd, shapes):
        got = y.download((m, n))
        single = w.gemm(x)
        assert np.array_equal(got, single)
        if m < pa.MFMA_MIN_M:
            assert rel_l2(got, ob.qgemm_seq(qtype, n, k, b, x)) <= TOL_F32
    st.destroy()


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("m,k", [(32, 4096), (64, 2048)])
@pytest.mark.parametrize("bf16", [False, True])
def test_multi_mfma_split_k_against_oracle(qtype, m, k, bf16):
    """q/k/v-shaped matrices on the MFMA path in one launch whose row tiles
    are few, so K is split over workgroups (parts summed in a fixed order):
    each output within the 16-bit bar (fp16 or bf16 operands) of the f64
    oracle, and a second call equal to the first bit for bit."""
    from prosperoai_amd.hipmem import DeviceBuffer, Stream
    shapes = [512, 128, 128]
    say(f"[gpu] multi mfma split-k type={qtype} m={m} k={k} bf16={bf16}")
    flags = pa.FLAG_MFMA_BF16 if bf16 else 0
    tol = TOL_BF16 if bf16 else TOL_F16
    mats, blocks = [], []
    for i, n in enumerate(shapes):
        b = weights(qtype, n, k, 1900 + 10 * i + qtype)
        blocks.append(b)
        mats.append(pa.QMat(qtype, n, k, b))
    x = pa.normal_f32(91 + m, m * k).reshape(m, k)
    xd = DeviceBuffer.from_array(x)
    yd = [DeviceBuffer(m * n * 4) for n in shapes]
    st = Stream()
    first = []
    for rep in range(2):
        pa.gemm_multi_async(mats, xd.ptr, [y.ptr for y in yd], m, flags, st.handle)
        st.synchronize()
        for i, (w, b, y, n) in enumerate(zip(mats, blocks, yd, shapes)):
            got = y.download((m, n))
            assert rel_l2(got, ob.qgemm_f64(qtype, n, k, b, x)) <= tol, (rep, n)
            # the parts are summed in a fixed order: calls repeat bit for bit
            if rep == 0:
                first.append(got)
            else:
                assert np.array_equal(got.view(np.uint32), first[i].view(np.uint32)), n
    st.destroy()


def test_multi_rejects_mixed_k():
    from prosperoai_amd.hipmem import DeviceBuffer
    say("[gpu] multi mismatch")
    a = pa.QMat(12, 64, 512, weights(12, 64, 512, 1))
    b = pa.QMat(12, 64, 256, weights(12, 64, 256, 2))
    xd, y0, y1 = DeviceBuffer(512 * 4), DeviceBuffer(64 * 4), DeviceBuffer(64 * 4)
    with pytest.raises(pa.PaiError) as e:
        pa.gemm_multi_async([a, b], xd.ptr, [y0.ptr, y1.ptr], 1)
    assert e.value.status == -6


def test_graph_replays_match_eager():
    """GEMV and fused GEMV launches captured into a HIP graph give the eager
    result on every replay, with eager work between replays."""
    from prosperoai_amd.hipmem import DeviceBuffer, Graph, Stream
    say("[gpu] graph replays")
    k = 2048
    a = pa.QMat(12, 300, k, weights(12, 300, k, 41))
    b = pa.QMat(12, 100, k, weights(12, 100, k, 42))
    x = pa.normal_f32(43, k)
    xd = DeviceBuffer.from_array(x)
    ya, yb, yc = DeviceBuffer(300 * 4), DeviceBuffer(100 * 4), DeviceBuffer(300 * 4)
    st = Stream()
    want_a, want_b = a.gemm(x.reshape(1, k))[0], b.gemm(x.reshape(1, k))[0]

    def enqueue(sh):
        pa.gemm_multi_async([a, b], xd.ptr, [ya.ptr, yb.ptr], 1, 0, sh)
        a.gemm_async(xd.ptr, yc.ptr, 1, 0, sh)

    g = Graph(st, enqueue)
    for rep in range(4):
        for buf, n in ((ya, 300), (yb, 100), (yc, 300)):
            buf.upload(np.full(n, np.nan, np.float32))
        g.launch(st)
        st.synchronize()
        assert np.array_equal(ya.download(300), want_a), rep
        assert np.array_equal(yb.download(100), want_b), rep
        assert np.array_equal(yc.download(300), want_a), rep
        a.gemm(x.reshape(1, k))  # eager work between replays
    g.destroy()
    st.destroy()


# ------------------------------------------------------------------ the executor's GEMM branch
@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("form,m", [("gemv", 1), ("row", 1), ("row2d", 1), ("gemm", 5),
                                    ("gemm", 40)])
def test_gemm_branch_forms(qtype, form, m):
    """pai_qgemm_run in run_gemm's three forms (scheduler/scheduler.c:280-338)
    on a 1024 x 4096 weight: bit-equal to pai_qgemm_f32 on the same tokens,
    and within its tolerance of the oracle's f64 product (16-bit MFMA at 40
    tokens, the integer-dot kernels below 8). K is kept in one part so that
    the MFMA results repeat bit for bit (more than two parts add with
    atomics in arrival order)."""
    n, k = 1024, 4096
    say(f"[gpu] gemm branch {form} type={qtype} m={m}")
    blocks = weights(qtype, n, k, 0xB0 + qtype)
    w = pa.QMat(qtype, n, k, blocks)
    x = pa.normal_f32(0xB1 + m, m * k).reshape(m, k)
    if form == "gemv":
        shapes = ([n, k], [k], [n])
    elif form == "row":
        shapes = ([k], [k, n], [n])
    elif form == "row2d":
        shapes = ([k], [k, n], [1, n])
    else:
        shapes = ([m, k], [k, n], [m, n])
    with pa.tuning(gemm_splits=1):
        y = pa.gemm_run(w, form == "gemv", *shapes, x)
        direct = w.gemm(x)
    assert list(y.shape) == shapes[2]
    assert np.array_equal(y.reshape(m, n).view(np.uint32), direct.view(np.uint32))
    tol = TOL_F32 if m < pa.MFMA_MIN_M else TOL_F16
    assert rel_l2(y.reshape(m, n), ob.qgemm_f64(qtype, n, k, blocks, x)) <= tol
    with pytest.raises(pa.PaiError, match="MISMATCH"):
        pa.gemm_run(w, form == "gemv", shapes[0], shapes[1], [n + 1], x)
