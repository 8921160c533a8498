"""Upload straight from a GGUF file (pai_qmat_upload_gguf) on the GPU: the
resident matrix must be the one pai_qmat_upload makes from the same
blocks (dequant bit-exact against the oracle, products bit-identical)."""
import sys

import numpy as np
import pytest

import gguf_file as gf
import oracle_bind as ob
import prosperoai_amd as pa

pytestmark = pytest.mark.gpu

SHAPES = {2: (96, 512), 8: (64, 1024), 12: (80, 2048), 14: (48, 1536)}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    say("[gpu] pai_hip_init")
    pa.init()
    tensors, blocks = [], {}
    for qt, (n, k) in SHAPES.items():
        w = pa.normal_f32(500 + qt, n * k, 0.0, 0.03).reshape(n, k)
        b = pa.quantize(qt, w)
        blocks[qt] = b
        tensors.append(gf.weight(f"blk.0.t{qt}.weight", qt, b))
    tensors.append(("blk.0.attn_norm.weight", [16], 0, bytes(64)))
    kv = [("general.architecture", gf.STR, "llama"), ("general.alignment", gf.U32, 256)]
    p = tmp_path_factory.mktemp("gguf") / "w.gguf"
    p.write_bytes(gf.build(kv, tensors, alignment=256))
    return p, blocks


@pytest.mark.parametrize("qtype", [2, 8, 12, 14])
def test_upload_from_file_matches_upload_from_blocks(model_file, qtype):
    path, blocks = model_file
    n, k = SHAPES[qtype]
    say(f"[gpu] upload_gguf qtype={qtype} n={n} k={k}")
    with pa.GGUFDir(path) as d:
        w = d.upload(f"blk.0.t{qtype}.weight")
    assert (w.qtype, w.n, w.k) == (qtype, n, k)
    assert w.nbytes == blocks[qtype].nbytes
    want = ob.dequant(qtype, blocks[qtype], n * k).reshape(n, k)
    got = w.dequant()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = pa.QMat(qtype, n, k, blocks[qtype])
    for m in (1, 5, 16):
        x = pa.normal_f32(900 + m, m * k).reshape(m, k)
        assert np.array_equal(w.gemm(x).view(np.uint32), ref.gemm(x).view(np.uint32)), m
    w.free()
    ref.free()


def test_upload_from_file_rejects_non_block_tensor(model_file):
    path, _ = model_file
    with pa.GGUFDir(path) as d:
        with pytest.raises(pa.PaiError) as e:
            d.upload("blk.0.attn_norm.weight")
        assert e.value.status == -3  # F32 vector: UNSUPPORTED before the dims check
