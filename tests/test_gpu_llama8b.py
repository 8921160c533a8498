"""Parity at the Llama-3-8B workloads themselves, through the dispatch the
benchmark runs.

  * Batched decode at 32 tokens (Q4_K at the seven projection shapes): q/k/v
    in one multi-matrix call (6144 rows), o, gate/up as a two-matrix call
    and as the fused SiLU*mul call (14336 rows), down at K = 14336. Sampled
    rows against the f64 oracle at the fp16-operand bar; a second call is
    bit-identical wherever the launch sums its K parts in a fixed order
    (all but o and down, whose single-matrix launches add more than two
    parts with atomics: there the two calls agree to rel-L2 1e-6).
  * A captured HIP graph replayed after an eager call with more tokens has
    grown the handles' workspaces: the replay still equals the eager result.
  * The decode step of the Llama-3-8B shape (n_embd 4096, 32/8 heads, head
    size 128, n_ff 14336, vocab 128256, fp16 KV cache prefilled to 2048
    positions): one full-width layer against orc_llama_step (logits
    rel-L2 <= 1e-4, greedy tokens equal unless the oracle's top two logits
    are within 1e-4 of each other), and the full 32-layer model through
    size-independent properties (finite logits, the token is the first
    argmax of the downloaded logits, a repeated step is bit-identical).
"""
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from decode_util import dequantized_model
from prosperoai_amd import hipmem as hm
from prosperoai_amd.llama import LlamaConfig, synthetic_weights, upload

pytestmark = pytest.mark.gpu

TOL_F16, TOL_LOGITS = 2e-3, 1e-4
SHAPES = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
          "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def device():
    say("[gpu] pai_hip_init")
    pa.init()
    yield


def rel_l2(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(y, np.float64) - ref) / max(np.linalg.norm(ref), 1e-30))


def weights(qtype: int, n: int, k: int, seed: int) -> np.ndarray:
    return pa.quantize(qtype, pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k))


# ------------------------------------------------------------- batched decode
def test_batched_decode_llama8b_m32():
    m = 32
    say("[gpu] batched decode M=32 Q4_K at the 8B shapes: building weights")
    blocks = {p: weights(pa.Q4_K, n, k, 0xC0DE0030 + i) for i, (p, (n, k)) in
              enumerate(SHAPES.items())}
    mats = {p: pa.QMat(pa.Q4_K, *SHAPES[p], blocks[p]) for p in SHAPES}
    xh = pa.normal_f32(0xC0DE0030 ^ 0x5A5A, m * 14336)
    x = hm.DeviceBuffer.from_array(xh)
    out = {p: hm.DeviceBuffer(4 * m * n) for p, (n, _) in SHAPES.items()}
    h = hm.DeviceBuffer(4 * m * 14336)
    st = hm.Stream()

    def step():
        pa.gemm_multi_async([mats["q"], mats["k"], mats["v"]], x.ptr,
                            [out["q"].ptr, out["k"].ptr, out["v"].ptr], m, 0, st.handle)
        mats["o"].gemm_async(x.ptr, out["o"].ptr, m, 0, st.handle)
        pa.gemm_multi_async([mats["gate"], mats["up"]], x.ptr, [out["gate"].ptr, out["up"].ptr],
                            m, 0, st.handle)
        pa.gate_up_async(mats["gate"], mats["up"], x.ptr, h.ptr, m, 0, st.handle)
        mats["down"].gemm_async(x.ptr, out["down"].ptr, m, 0, st.handle)
        st.synchronize()
        res = {p: out[p].download((m, n)) for p, (n, _) in SHAPES.items()}
        res["h"] = h.download((m, 14336))
        return res

    say("[gpu]   first call")
    first = step()
    say("[gpu]   second call")
    second = step()
    for p in ("q", "k", "v", "gate", "up", "h"):
        assert np.array_equal(first[p].view(np.uint32), second[p].view(np.uint32)), p
    for p in ("o", "down"):  # K split into 8 and 7 parts, added with atomics
        assert rel_l2(second[p], first[p]) <= 1e-6, p
    f64 = {}
    for p, (n, k) in SHAPES.items():
        rows = np.arange(3, n, 11)
        xk = xh[:m * k].reshape(m, k)
        ref = ob.qgemm_f64(pa.Q4_K, len(rows), k, blocks[p][rows], xk)
        f64[p] = (rows, ref)
        err = rel_l2(first[p][:, rows], ref)
        say(f"[gpu]   {p}: rows={len(rows)} rel_l2={err:.2e}")
        assert err <= TOL_F16, (p, err)
    rows = f64["gate"][0]
    ref_h = ob.silu_mul(f64["gate"][1].astype(np.float32), f64["up"][1].astype(np.float32))
    err = rel_l2(first["h"][:, rows], ref_h)
    say(f"[gpu]   silu(gate)*up: rel_l2={err:.2e}")
    assert err <= TOL_F16
    st.destroy()
    for b in [x, h, *out.values()]:
        b.free()
    for w in mats.values():
        w.free()


def test_graph_replay_after_workspace_growth():
    """Graph captured at 32 tokens (16-bit copy of 256 tokens, split parts),
    then an eager call of 512 tokens on the same handles (both workspaces
    grow), then three replays with eager work between them: each replay
    equals the eager 32-token result bit for bit."""
    k = 4096
    ns = (1024, 256, 256)
    say("[gpu] graph replay after workspace growth")
    blocks = [weights(pa.Q4_K, n, k, 0x6A00 + i) for i, n in enumerate(ns)]
    mats = [pa.QMat(pa.Q4_K, n, k, b) for n, b in zip(ns, blocks)]
    gb, ub = weights(pa.Q4_K, 2048, k, 0x6A10), weights(pa.Q4_K, 2048, k, 0x6A11)
    g, u = pa.QMat(pa.Q4_K, 2048, k, gb), pa.QMat(pa.Q4_K, 2048, k, ub)
    xh = pa.normal_f32(0x6A20, 512 * k)
    x = hm.DeviceBuffer.from_array(xh)
    st = hm.Stream()

    def bufs(m):
        return [hm.DeviceBuffer(4 * m * n) for n in ns], hm.DeviceBuffer(4 * m * 2048)

    def enqueue(m, ys, h, sh):
        pa.gemm_multi_async(mats, x.ptr, [y.ptr for y in ys], m, 0, sh)
        pa.gate_up_async(g, u, x.ptr, h.ptr, m, 0, sh)

    def read(m, ys, h):
        return [y.download((m, n)) for y, n in zip(ys, ns)] + [h.download((m, 2048))]

    ys_e, h_e = bufs(32)
    enqueue(32, ys_e, h_e, st.handle)  # eager first: workspaces sized for 32 tokens
    st.synchronize()
    eager = read(32, ys_e, h_e)
    ys_g, h_g = bufs(32)
    graph = hm.Graph(st, lambda sh: enqueue(32, ys_g, h_g, sh))
    ys_b, h_b = bufs(512)
    for rep in range(3):
        enqueue(512, ys_b, h_b, st.handle)  # grows (first time) and uses the workspaces
        st.synchronize()
        graph.launch(st)
        st.synchronize()
        got = read(32, ys_g, h_g)
        for a, b in zip(got, eager):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), rep
    big = read(512, ys_b, h_b)
    rows = np.arange(0, 1024, 37)
    ref = ob.qgemm_f64(pa.Q4_K, len(rows), k, blocks[0][rows], xh.reshape(512, k))
    assert rel_l2(big[0][:, rows], ref) <= TOL_F16
    graph.destroy()
    st.destroy()
    for b in [x, h_e, h_g, h_b, *ys_e, *ys_g, *ys_b]:
        b.free()
    for w in [*mats, g, u]:
        w.free()


# ------------------------------------------------------------- decode step, 8B shape
FILL = 2048


def config(n_layer: int) -> LlamaConfig:
    return LlamaConfig(n_layer=n_layer, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336,
                       vocab=128256, ctx=FILL + 8, n_rot=0, rope_theta=500000.0,
                       norm_eps=1e-5)


@pytest.fixture(scope="module")
def one_layer_weights():
    say("[gpu] Llama-3-8B shape: quantizing one layer and the 128256-row head")
    return synthetic_weights(config(1), seed=0xC0DE0050, norms_one=True)


def kv_prefill(rng, n_layer):
    for _ in range(n_layer):
        k = rng.standard_normal((FILL, 8, 128), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((FILL, 8, 128), dtype=np.float32).astype(np.float16)
        yield k, v


def test_decode_llama8b_one_layer_matches_oracle(one_layer_weights):
    cfg = config(1)
    w = one_layer_weights
    say("[gpu] 8B-shape layer: oracle weights")
    layers, head = dequantized_model(cfg.as_dict(), w)
    orc = ob.LlamaOracle(cfg.as_dict(), layers, head, kv_f16=True)
    m = upload(cfg, w)
    for L, (k, v) in enumerate(kv_prefill(np.random.default_rng(0xC0DE005F), 1)):
        m.kv_write(L, 0, k, v)
        orc.k_cache[L, :, :FILL] = k.astype(np.float32).transpose(1, 0, 2)
        orc.v_cache[L, :, :FILL] = v.astype(np.float32).transpose(1, 0, 2)
    token = 128000
    for pos in range(FILL, FILL + 3):
        nxt, logits = m.decode(token, pos)
        want, want_next = orc.step(token, pos)
        err = rel_l2(logits, want)
        say(f"[gpu]   pos={pos} token={token} rel_l2={err:.2e} next={nxt}/{want_next}")
        assert np.isfinite(logits).all()
        assert err <= TOL_LOGITS, (pos, err)
        if nxt != want_next:
            top = np.sort(want)[-2:]
            assert top[1] - top[0] <= 1e-4 * abs(top[1]), (pos, nxt, want_next)
        token = nxt
    m.free()


def test_decode_llama8b_32_layers_properties(one_layer_weights):
    """The full-depth model (the one layer's weights uploaded as each of the
    32 layers, distinct device copies; every layer's cache prefilled with its
    own random keys and values)."""
    cfg = config(32)
    w1 = one_layer_weights
    say("[gpu] 8B-shape model, 32 layers: upload")
    w = type(w1)([w1.layers[0]] * 32, w1.head)
    m = upload(cfg, w)
    for L, (k, v) in enumerate(kv_prefill(np.random.default_rng(0xC0DE006F), 32)):
        m.kv_write(L, 0, k, v)
    say("[gpu]   decode at position 2048, twice")
    nxt1, logits1 = m.decode(128000, FILL)
    nxt2, logits2 = m.decode(128000, FILL)
    assert np.isfinite(logits1).all()
    assert nxt1 == ob.argmax_first(logits1)
    assert nxt1 == nxt2 and np.array_equal(logits1.view(np.uint32), logits2.view(np.uint32))
    say(f"[gpu]   token={nxt1}; next step")
    nxt3, logits3 = m.decode(nxt1, FILL + 1)
    assert np.isfinite(logits3).all() and nxt3 == ob.argmax_first(logits3)
    m.free()
