"""Packed GGUF tensors carried in a 64-bit `.pai` container go straight
from the mapped file to the device (pai64_qmat_upload): the device copy
dequantizes bit-exactly to the oracle and the GEMV equals the one over the
same blocks uploaded directly, bit for bit. Weights are f32 N(0, 0.02^2)
from a fixed seed, quantized by libpai_hip's encoders."""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from prosperoai_amd import pai64
from prosperoai_amd._lib import lib

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def device():
    say("[gpu] pai_hip_init")
    pa.init()
    yield


def test_upload_from_container(tmp_path):
    say("[gpu] container upload")
    shapes = [(pa.Q4_K, 1024, 4096), (pa.Q6_K, 512, 2048), (pa.Q8_0, 256, 1024),
              (pa.Q4_0, 300, 512)]
    blobs, tensors, off = [], [], 0
    for i, (qt, n, k) in enumerate(shapes):
        b = pa.quantize(qt, pa.normal_f32(0xA000 + i, n * k, 0.0, 0.02).reshape(n, k))
        blobs.append(b)
        # logical [K][N]; 256-byte aligned inside WEIGHTS
        tensors.append(pai64.Tensor(f"w{i}".encode(), i + 1, 0, 2, (k, n, 0, 0, 0, 0), off,
                                    b.nbytes, qt))
        off += (b.nbytes + 255) // 256 * 256
    weights = np.zeros(off, np.uint8)
    for t, b in zip(tensors, blobs):
        weights[t.offset:t.offset + b.nbytes] = b.ravel()
    path = tmp_path / "model.pai"
    pai64.write(str(path), [(pai64.MANIFEST, pai64.manifest_encode(tensors)),
                            (pai64.WEIGHTS, weights.tobytes())])
    m = pai64.Mapped(str(path))
    try:
        for t, b, (qt, n, k) in zip(pai64.manifest_decode(m.section(pai64.MANIFEST)), blobs,
                                    shapes):
            h = C.c_void_p()
            assert lib().pai64_qmat_upload(C.byref(m.view), C.byref(t), C.byref(h)) == 0
            from_file = pa.QMat.adopt(h)
            direct = pa.QMat(qt, n, k, b)
            assert (from_file.qtype, from_file.n, from_file.k) == (qt, n, k)
            want = ob.dequant(qt, b, n * k).reshape(n, k)
            assert np.array_equal(from_file.dequant().view(np.uint32), want.view(np.uint32))
            x = pa.normal_f32(0xA100, 3 * k).reshape(3, k)
            y1 = from_file.gemm(x, pa.FLAG_FP32)
            y2 = direct.gemm(x, pa.FLAG_FP32)
            assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
            from_file.free()
            direct.free()
        # a tensor that is not GGUF blocks, or leaves WEIGHTS
        t = pai64.Tensor(b"f", 1, 0, 2, (64, 64, 0, 0, 0, 0), 0, 64 * 64 * 4, 0)
        h = C.c_void_p()
        assert lib().pai64_qmat_upload(C.byref(m.view), C.byref(t), C.byref(h)) == -3
        t = pai64.Tensor(b"g", 1, 0, 2, (256, 4, 0, 0, 0, 0), off - 100, 4 * 144, 12)
        assert lib().pai64_qmat_upload(C.byref(m.view), C.byref(t), C.byref(h)) == -6
    finally:
        m.close()
