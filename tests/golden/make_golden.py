"""Writes the committed golden fixtures under tests/golden/.

1. gguf_hand_vectors.json — the reference's hand-computed dequant vectors
   for the four formats on this path and its f16 literals, re-expressed as
   data (raw block bytes + expected f32 values):
     f16 literals      tests/test_gguf.c:270-276
     Q8_0 d=1, q=i-16  tests/test_gguf.c:284-298
     Q4_0 d=1          tests/test_gguf.c:317-332
     Q4_K dmin=0       tests/test_gguf.c:451-468
     Q4_K dmin=0.5     tests/test_gguf.c:470-491
     Q6_K ql=qh=0      tests/test_gguf.c:519-538

2. ref_vectors.npz — outputs of the reference's own C code, compiled from
   its sources by oracle/Makefile into oracle/_ref/libpairef.so and run in
   this container: pai_gguf_dequant on seeded random blocks of each format
   (with f16 scales spanning zero, subnormal and normal magnitudes), and
   pai_ref_gemm_f32 / pai_opt_gemv_f32 / pai_opt_gemm_w8_f32 on small seeded
   shapes. These pin the oracle where the reference tree is absent.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "oracle"))

import oracle_bind as ob  # noqa: E402

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def f16(v: float) -> bytes:
    return np.float16(v).tobytes()


def hand_vectors() -> dict:
    cases = []
    # Q8_0: d = 1, qs[i] = i - 16
    raw = f16(1.0) + bytes((i - 16) & 0xFF for i in range(32))
    cases.append({"name": "q8_0", "type": Q8_0, "numel": 32, "raw": raw.hex(),
                  "expect": [float(i - 16) for i in range(32)]})
    # Q4_0: d = 1, byte j = j | ((j ^ 8) << 4)
    raw = f16(1.0) + bytes(j | ((j ^ 8) << 4) for j in range(16))
    exp = [float(j - 8) for j in range(16)] + [float((j ^ 8) - 8) for j in range(16)]
    cases.append({"name": "q4_0", "type": Q4_0, "numel": 32, "raw": raw.hex(), "expect": exp})
    # Q4_K: d = 1, dmin = 0, scales 0x01, codes 0x12
    raw = f16(1.0) + f16(0.0) + b"\x01" * 12 + b"\x12" * 128
    exp = [1.0 if (e & 32) else 2.0 for e in range(256)]
    cases.append({"name": "q4_k", "type": Q4_K, "numel": 256, "raw": raw.hex(), "expect": exp})
    # Q4_K: d = 1, dmin = 0.5 (m = 1 for the first two 64-groups)
    raw = f16(1.0) + f16(0.5) + b"\x01" * 12 + b"\x12" * 128
    exp = [(1.0 if (e & 32) else 2.0) - (0.5 if e < 128 else 0.0) for e in range(256)]
    cases.append({"name": "q4_k_min", "type": Q4_K, "numel": 256, "raw": raw.hex(),
                  "expect": exp})
    # Q6_K: ql = qh = 0, scales 1, d = 1 -> every value -32
    raw = b"\x00" * 128 + b"\x00" * 64 + b"\x01" * 16 + f16(1.0)
    cases.append({"name": "q6_k", "type": Q6_K, "numel": 256, "raw": raw.hex(),
                  "expect": [-32.0] * 256})
    f16_literals = [[0x3C00, 1.0], [0xC000, -2.0], [0x3800, 0.5], [0x0000, 0.0]]
    return {"source": "reference tests/test_gguf.c hand vectors", "cases": cases,
            "f16_literals": f16_literals}


BLOCK = {Q4_0: (32, 18, 0), Q8_0: (32, 34, 0), Q4_K: (256, 144, 0), Q6_K: (256, 210, 208)}


def random_blocks(rng: np.random.Generator, qtype: int, nblk: int) -> np.ndarray:
    """Random block bytes whose f16 scale fields span zero, subnormal and
    normal magnitudes of both signs (never inf/NaN)."""
    qk, bb, doff = BLOCK[qtype]
    raw = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    fields = [doff] if qtype != Q4_K else [0, 2]
    for off in fields:
        h = rng.integers(0, 0x7C00, size=nblk, dtype=np.uint16)  # finite magnitudes
        h[::7] = rng.integers(0, 0x0400, size=h[::7].shape, dtype=np.uint16)  # subnormals
        h[::11] = 0
        h |= (rng.integers(0, 2, size=nblk, dtype=np.uint16) << 15)
        raw[:, off] = (h & 0xFF).astype(np.uint8)
        raw[:, off + 1] = (h >> 8).astype(np.uint8)
    return raw


def ref_vectors() -> dict:
    r = ob.ref()
    if r is None:
        raise SystemExit("oracle/_ref/libpairef.so is not built (make -C oracle)")
    rng = np.random.default_rng(20261201)
    out = {}
    for qtype in (Q4_0, Q8_0, Q4_K, Q6_K):
        qk = BLOCK[qtype][0]
        raw = random_blocks(rng, qtype, 64)
        vals = ob.ref_dequant(qtype, raw.tobytes(), 64 * qk)
        out[f"dq_raw_{qtype}"] = raw
        out[f"dq_out_{qtype}"] = vals
    # pai_ref_gemm_f32: a[m][k] * b[k][n]
    m, n, k = 3, 37, 96
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = np.empty((m, n), np.float32)
    assert r.pai_ref_gemm_f32(m, n, k, a.ctypes.data, b.ctypes.data, c.ctypes.data) == 0
    out.update(gemm_a=a, gemm_b=b, gemm_c=c)
    # pai_opt_gemv_f32: A[m][k] * x[k]  (k not a multiple of 8: scalar tail)
    gm, gk = 29, 203
    ga = rng.standard_normal((gm, gk)).astype(np.float32)
    gx = rng.standard_normal(gk).astype(np.float32)
    gy = np.empty(gm, np.float32)
    assert r.pai_opt_gemv_f32(gm, gk, ga.ctypes.data, gx.ctypes.data, gy.ctypes.data) == 0
    out.update(gemv_a=ga, gemv_x=gx, gemv_y=gy)
    # pai_opt_gemm_w8_f32 at group 32 (n not a multiple of 8: scalar tail)
    wm, wn, wk, gs = 2, 19, 96, 32
    wa = rng.standard_normal((wm, wk)).astype(np.float32)
    wq = rng.integers(-127, 128, size=(wk, wn), dtype=np.int8)
    ws = (rng.random((wk // gs, wn)) * 0.05).astype(np.float32)
    wc = np.empty((wm, wn), np.float32)
    assert r.pai_opt_gemm_w8_f32(wm, wn, wk, wa.ctypes.data, wq.ctypes.data, ws.ctypes.data,
                                 gs, wc.ctypes.data) == 0
    out.update(w8_a=wa, w8_q=wq, w8_s=ws, w8_c=wc, w8_gs=np.array([gs]))
    out["opt_backend"] = np.array([r.pai_opt_backend_name().decode()])
    return out


def main() -> None:
    (HERE / "gguf_hand_vectors.json").write_text(json.dumps(hand_vectors(), indent=1) + "\n")
    np.savez_compressed(HERE / "ref_vectors.npz", **ref_vectors())
    print("wrote", HERE / "gguf_hand_vectors.json", HERE / "ref_vectors.npz")


if __name__ == "__main__":
    main()
