"""The no-allocation entry point (pai_qgemm_f32_noalloc_async) against
pai_qgemm_f32_async, through the C-ABI, on two calls in a row per shape, the
second with fewer tokens (the shared scratch array keeps the first call's
contents).

Bars: bit-identical where the launches repeat bit for bit (no K split, or
two parts; GEMV-path calls of up to 8 tokens); where a launch adds more
than two K parts with atomics (4096 rows at 300 or 256 tokens), rel-L2
<= 1e-6 against the async call. Every call within 2e-3 (fp16 operands) of
the f64 oracle on sampled rows (1e-5 on the GEMV path). A K above the
scratch's limit is rejected with PAI_ERR_UNSUPPORTED before any launch.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from prosperoai_amd import hipmem as hm
from prosperoai_amd._lib import lib

pytestmark = pytest.mark.gpu

TOL_F16 = 2e-3


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def rel_l2(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def run(entry, w, x, y, m, n, flags=0):
    st = getattr(lib(), entry)(w.handle, m, x.ptr, y.ptr, flags | pa.FLAG_DEVICE_PTRS, None)
    assert st == 0, (entry, st, lib().pai_hip_last_error())
    hm.synchronize()
    return y.download((m, n))


# (type, n, k, first m, second m, whether the launches repeat bit for bit):
# 14336 rows at 512 tokens fill the chip unsplit; 1000 rows at 64 tokens
# split K in two; 4096 rows at 300 tokens (K = 14336) and 2048 rows at 256
# tokens split K into more parts.
CASES = [(pa.Q4_K, 14336, 4096, 512, 8, True), (pa.Q6_K, 4096, 14336, 300, 16, False),
         (pa.Q8_0, 1000, 2048, 64, 3, True), (pa.Q4_0, 2048, 4096, 256, 5, False)]


@pytest.mark.parametrize("qtype,n,k,m1,m2,exact", CASES)
def test_noalloc_matches_async(qtype, n, k, m1, m2, exact):
    pa.init()
    say(f"[gpu] noalloc type={qtype} n={n} k={k} m={m1} then {m2}")
    blocks = pa.quantize(qtype, pa.normal_f32(0x7A00 + qtype, n * k, 0.0, 0.02).reshape(n, k))
    w = pa.QMat(qtype, n, k, blocks)
    xh = pa.normal_f32(0x7A10 + qtype, m1 * k)
    x = hm.DeviceBuffer.from_array(xh)
    y_ref, y_na = hm.DeviceBuffer(4 * m1 * n), hm.DeviceBuffer(4 * m1 * n)
    for m in (m1, m2):
        want = run("pai_qgemm_f32_async", w, x, y_ref, m, n)
        got = run("pai_qgemm_f32_noalloc_async", w, x, y_na, m, n)
        if exact or m <= 8:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), m
        else:
            assert rel_l2(got, want) <= 1e-6, m
        rows = np.arange(1, n, 29)
        ref = ob.qgemm_f64(qtype, len(rows), k, blocks[rows], xh[:m * k].reshape(m, k))
        assert rel_l2(got[:, rows], ref) <= (TOL_F16 if m > 8 else 1e-5), m
    for b in (x, y_ref, y_na):
        b.free()
    w.free()


def test_noalloc_rejects_k_above_scratch():
    pa.init()
    n, k = 8, 256 * 129  # 33024 > 32768
    say(f"[gpu] noalloc rejects k={k}")
    blocks = np.zeros((n, pa.qtype_bytes(pa.Q4_K, k)), np.uint8)
    w = pa.QMat(pa.Q4_K, n, k, blocks)
    x, y = hm.DeviceBuffer(4 * 16 * k), hm.DeviceBuffer(4 * 16 * n)
    st = lib().pai_qgemm_f32_noalloc_async(w.handle, 16, x.ptr, y.ptr, pa.FLAG_DEVICE_PTRS, None)
    assert st == -3 and b"32768" in lib().pai_hip_last_error()
    for b in (x, y):
        b.free()
    w.free()


@pytest.mark.parametrize("qtype", [pa.Q4_K, pa.Q6_K, pa.Q8_0, pa.Q4_0])
def test_noalloc_copy_matches_register_tiles(qtype):
    """Up to 32 tokens the allocating entry rounds x to 16 bits inside the
    register-staged GEMM (activations requested two steps ahead), while this
    entry first copies x to 16 bits in its scratch and stages it by DMA. Both
    round x and the weights the same way and accumulate in the same order,
    so with K in one part the outputs are identical."""
    pa.init()
    n, k = 1000, 4096
    say(f"[gpu] noalloc copy vs register tiles type={qtype}")
    blocks = pa.quantize(qtype, pa.normal_f32(0x7B00 + qtype, n * k, 0.0, 0.02).reshape(n, k))
    w = pa.QMat(qtype, n, k, blocks)
    xh = pa.normal_f32(0x7B10 + qtype, 32 * k)
    x = hm.DeviceBuffer.from_array(xh)
    y_ref, y_na = hm.DeviceBuffer(4 * 32 * n), hm.DeviceBuffer(4 * 32 * n)
    with pa.tuning(gemm_splits=1):
        for m in (32, 9, 17):
            want = run("pai_qgemm_f32_async", w, x, y_ref, m, n)
            got = run("pai_qgemm_f32_noalloc_async", w, x, y_na, m, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), m
    rows = np.arange(3, n, 31)
    ref = ob.qgemm_f64(qtype, len(rows), k, blocks[rows], xh[:17 * k].reshape(17, k))
    assert rel_l2(got[:, rows], ref) <= TOL_F16
    for b in (x, y_ref, y_na):
        b.free()
    w.free()
