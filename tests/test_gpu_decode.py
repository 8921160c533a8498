"""The decode step on the GPU (include/pai_llama.h) against the oracle's
restatement of the reference's operators and of the adapter's graph.

Bars:
  RMSNorm (+ residual add)  bit-exact (same products; the double sum of
                            squares differs in order, which moves a float
                            result only at a rounding tie)
  RoPE + KV append          bit-exact: rotated q, fp16 k and v in the cache
  attention                 rel-L2 <= 1e-5 per head against the oracle's
                            last-row attention over the same fp16 cache; or,
                            for large scores, where the oracle's own f32
                            error is of that size, an error against a
                            float64 evaluation at most twice the oracle's
  argmax                    exact index, with the reference's tie and NaN
                            rules
  model step                logits rel-L2 <= 1e-4 against orc_llama_step
                            (fp16 cache) after a random fp16 prefill and
                            through several greedy steps; the greedy token
                            equal unless the oracle's top two logits are
                            within 1e-4 of each other (relative to the
                            largest logit)
"""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle_bind as ob
import prosperoai_amd as pa
from decode_util import dequantized_model
from prosperoai_amd import hipmem as hm
from prosperoai_amd._lib import check, lib
from prosperoai_amd.llama import LlamaConfig, synthetic_weights, upload

pytestmark = pytest.mark.gpu

TOL_ATTN, TOL_LOGITS = 1e-5, 1e-4


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


def dev(a: np.ndarray) -> hm.DeviceBuffer:
    return hm.DeviceBuffer.from_array(np.ascontiguousarray(a))


def f16(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.float32).astype(np.float16)


# ---------------------------------------------------------------- operators
@pytest.mark.parametrize("n", [1, 100, 4096, 14336, 16384])
@pytest.mark.parametrize("with_delta", [False, True])
def test_rmsnorm(n, with_delta):
    say(f"[gpu] rmsnorm n={n} delta={with_delta}")
    rng = np.random.default_rng(n + with_delta)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    d = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    bx, bd, bg, bo = dev(x), dev(d), dev(g), hm.DeviceBuffer(4 * n)
    check(lib().pai_rmsnorm_f32_async(bx.ptr, bd.ptr if with_delta else None, bg.ptr, bo.ptr, n,
                                      0.0, None), "pai_rmsnorm_f32_async")
    hm.synchronize()
    xs = x + d if with_delta else x
    assert np.array_equal(bx.download(n).view(np.uint32), xs.view(np.uint32))
    want = ob.rmsnorm(xs, g)
    assert np.array_equal(bo.download(n).view(np.uint32), want.view(np.uint32))


FUSED_CASES = [(pa.Q4_K, 4096, 1024), (pa.Q6_K, 14336, 512), (pa.Q4_0, 256, 300),
               (pa.Q8_0, 2048, 96)]


def packed(qtype, n, k, seed):
    w = pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
    blocks = pa.quantize(qtype, w)
    return blocks, pa.QMat(qtype, n, k, blocks)


def ptr_array(ptrs):
    return (C.c_void_p * len(ptrs))(*ptrs)


@pytest.mark.parametrize("qtype,k,n", FUSED_CASES)
def test_fused_rmsnorm_projections(qtype, k, n):
    """rmsnorm(x) W_i^T in one launch (one, then three matrices) against the
    oracle's RMSNorm followed by its sequential qgemm (f32 bar), and within
    1e-6 of pai_rmsnorm_f32_async followed by pai_qgemm_f32_multi_async (the
    fused kernel scales the finished dot products by rms instead of each
    element: one rounding moved)."""
    say(f"[gpu] fused rmsnorm+gemv type={qtype} k={k} n={n}")
    rng = np.random.default_rng(k + n)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    mats = [packed(qtype, n + 32 * i, k, 0xF00 + 16 * qtype + i) for i in range(3)]
    bx, bg, bxn = dev(x), dev(g), hm.DeviceBuffer(4 * k)
    xn = ob.rmsnorm(x, g)
    for count in (1, 3):
        ys = [hm.DeviceBuffer(4 * (n + 32 * i)) for i in range(count)]
        ys2 = [hm.DeviceBuffer(4 * (n + 32 * i)) for i in range(count)]
        hs = ptr_array([m.handle for _, m in mats[:count]])
        check(lib().pai_qgemv_rmsnorm_f32_async(hs, count, bx.ptr, bg.ptr, 0.0,
                                                ptr_array([y.ptr for y in ys]), None),
              "pai_qgemv_rmsnorm_f32_async")
        check(lib().pai_rmsnorm_f32_async(bx.ptr, None, bg.ptr, bxn.ptr, k, 0.0, None),
              "pai_rmsnorm_f32_async")
        check(lib().pai_qgemm_f32_multi_async(hs, count, 1, bxn.ptr,
                                              ptr_array([y.ptr for y in ys2]),
                                              pa.FLAG_DEVICE_PTRS, None),
              "pai_qgemm_f32_multi_async")
        hm.synchronize()
        for i in range(count):
            blocks, _ = mats[i]
            ni = n + 32 * i
            got = ys[i].download(ni)
            want = ob.qgemm_seq(qtype, ni, k, blocks, xn.reshape(1, k)).reshape(ni)
            assert rel_l2(got, want) <= 1e-5, (count, i)
            assert rel_l2(got, ys2[i].download(ni)) <= 1e-6, (count, i)


@pytest.mark.parametrize("qtype,k,n", FUSED_CASES)
def test_fused_rmsnorm_gate_up(qtype, k, n):
    say(f"[gpu] fused rmsnorm+gate/up type={qtype} k={k} n={n}")
    rng = np.random.default_rng(3 * k + n)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    (gb, wg), (ub, wu) = packed(qtype, n, k, 0xA11 + qtype), packed(qtype, n, k, 0xB22 + qtype)
    bx, bg, bh = dev(x), dev(g), hm.DeviceBuffer(4 * n)
    check(lib().pai_qgemv_rmsnorm_gate_up_async(wg.handle, wu.handle, bx.ptr, bg.ptr, 0.0, bh.ptr,
                                                None), "pai_qgemv_rmsnorm_gate_up_async")
    hm.synchronize()
    xn = ob.rmsnorm(x, g).reshape(1, k)
    want = ob.silu_mul(ob.qgemm_seq(qtype, n, k, gb, xn), ob.qgemm_seq(qtype, n, k, ub, xn))
    assert rel_l2(bh.download(n), want.reshape(n)) <= 1e-5


@pytest.mark.parametrize("qtype,k,n", FUSED_CASES)
def test_projection_adds_to_residual(qtype, k, n):
    """y += x W^T: one f32 add of the finished product per output, as the
    reference's GEMM then ADD; called twice in a row (the decode step adds
    o and down to the same residual)."""
    say(f"[gpu] gemv+add type={qtype} k={k} n={n}")
    rng = np.random.default_rng(5 * k + n)
    x = rng.standard_normal(k).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    blocks, w = packed(qtype, n, k, 0xC33 + qtype)
    bx, by, bp = dev(x), dev(y0), hm.DeviceBuffer(4 * n)
    check(lib().pai_qgemv_add_f32_async(w.handle, bx.ptr, by.ptr, None), "pai_qgemv_add_f32_async")
    w.gemm_async(bx.ptr, bp.ptr, 1)
    hm.synchronize()
    prod = bp.download(n)
    assert rel_l2(prod, ob.qgemm_seq(qtype, n, k, blocks, x.reshape(1, k)).reshape(n)) <= 1e-5
    y1 = by.download(n)
    assert np.array_equal(y1.view(np.uint32), (y0 + prod).view(np.uint32))
    check(lib().pai_qgemv_add_f32_async(w.handle, bx.ptr, by.ptr, None), "pai_qgemv_add_f32_async")
    hm.synchronize()
    assert np.array_equal(by.download(n).view(np.uint32), (y1 + prod).view(np.uint32))


def test_fused_projection_argument_errors():
    """The fused projections reject misaligned pointers, mixed formats or
    K, too many matrices and a K beyond the fused RMSNorm's limit before
    any launch."""
    say("[gpu] fused projection argument errors")
    _, a = packed(pa.Q4_K, 64, 1024, 0xE01)
    _, b = packed(pa.Q4_0, 64, 1024, 0xE02)
    _, c = packed(pa.Q4_K, 64, 2048, 0xE03)
    _, big = packed(pa.Q4_K, 8, 16640, 0xE04)
    x, g, y = dev(np.ones(16640, np.float32)), dev(np.ones(16640, np.float32)), hm.DeviceBuffer(4 * 64)
    hs = lambda *ms: ptr_array([m.handle for m in ms])
    ys = lambda n: ptr_array([y.ptr] * n)
    f = lib().pai_qgemv_rmsnorm_f32_async
    assert f(hs(a), 1, x.ptr + 4, g.ptr, 0.0, ys(1), None) == -1        # x not 16-byte aligned
    assert f(hs(a), 1, x.ptr, g.ptr + 4, 0.0, ys(1), None) == -1        # gamma not aligned
    assert f(hs(a, b), 2, x.ptr, g.ptr, 0.0, ys(2), None) == -6         # formats differ
    assert f(hs(a, c), 2, x.ptr, g.ptr, 0.0, ys(2), None) == -6         # K differs
    assert f(hs(a, a, a, a), 4, x.ptr, g.ptr, 0.0, ys(4), None) == -1   # at most 3 matrices
    assert f(hs(big), 1, x.ptr, g.ptr, 0.0, ys(1), None) == -3          # K above 16384
    gu = lib().pai_qgemv_rmsnorm_gate_up_async
    _, a2 = packed(pa.Q4_K, 32, 1024, 0xE05)
    assert gu(a.handle, a2.handle, x.ptr, g.ptr, 0.0, y.ptr, None) == -6  # shapes differ
    assert gu(a.handle, b.handle, x.ptr, g.ptr, 0.0, y.ptr, None) == -6   # formats differ
    add = lib().pai_qgemv_add_f32_async
    assert add(a.handle, x.ptr + 4, y.ptr, None) == -1
    assert add(a.handle, x.ptr, y.ptr + 2, None) == -1


@pytest.mark.parametrize("hq,hk,hd,r2", [(32, 8, 128, 64), (4, 2, 64, 16), (2, 1, 256, 128)])
@pytest.mark.parametrize("pos", [0, 17, 63])
def test_rope_kv_append(hq, hk, hd, r2, pos):
    say(f"[gpu] rope hq={hq} hk={hk} hd={hd} r2={r2} pos={pos}")
    ctx = 64
    rng = np.random.default_rng(pos * 7 + hd)
    q = rng.standard_normal((hq, hd)).astype(np.float32)
    k = rng.standard_normal((hk, hd)).astype(np.float32)
    v = rng.standard_normal((hk, hd)).astype(np.float32)
    c, s = ob.rope_tables(ctx, r2, 2 * r2, 500000.0)
    bq, bk, bv, bqo = dev(q), dev(k), dev(v), hm.DeviceBuffer(q.nbytes)
    cache_bytes = hk * ctx * hd * 2
    bkc, bvc = dev(np.zeros(cache_bytes, np.uint8)), dev(np.zeros(cache_bytes, np.uint8))
    bc, bs = dev(c), dev(s)
    row = pos * r2 * 4
    check(lib().pai_rope_kv_append_async(bq.ptr, bk.ptr, bv.ptr, bqo.ptr, bkc.ptr, bvc.ptr,
                                         bc.ptr + row, bs.ptr + row, hq, hk, hd, r2, ctx, pos,
                                         None), "pai_rope_kv_append_async")
    hm.synchronize()
    want_q = ob.rope(q, hq, c[pos:pos + 1], s[pos:pos + 1], r2)
    assert np.array_equal(bqo.download((hq, hd)).view(np.uint32), want_q.view(np.uint32))
    want_k = ob.rope(k, hk, c[pos:pos + 1], s[pos:pos + 1], r2)
    kc = bkc.download((hk, ctx, hd), np.uint16)
    vc = bvc.download((hk, ctx, hd), np.uint16)
    assert np.array_equal(kc[:, pos], ob.f32_to_f16(want_k).reshape(hk, hd))
    assert np.array_equal(vc[:, pos], ob.f32_to_f16(v).reshape(hk, hd))
    others = np.ones(ctx, bool)
    others[pos] = False
    assert not kc[:, others].any() and not vc[:, others].any()


ATTN_CASES = [
    (32, 8, 128, 2048, [1, 63, 64, 65, 1000, 2048], 1.0),
    (32, 8, 128, 2048, [2048], 8.0),       # peaked softmax
    (8, 8, 64, 256, [1, 100, 256], 1.0),
    (16, 2, 256, 128, [1, 77, 128], 1.0),
    (8, 1, 128, 300, [300], 4.0),
    (12, 4, 64, 96, [96], 1.0),            # three q heads per KV head
    # contexts past 2048 positions (up to 66 chunks to merge), lengths on and
    # one past chunk boundaries
    (32, 8, 128, 4200, [129, 640, 2049, 4096, 4097, 4200], 1.0),
]


@pytest.mark.parametrize("hq,hk,hd,ctx,lens,qscale", ATTN_CASES)
def test_attention_decode(hq, hk, hd, ctx, lens, qscale):
    rng = np.random.default_rng(hq * 1000 + hd + ctx)
    kc = f16(rng.standard_normal((hk, ctx, hd)))
    vc = f16(rng.standard_normal((hk, ctx, hd)))
    bkc, bvc = dev(kc), dev(vc)
    bo = hm.DeviceBuffer(4 * hq * hd)
    ws = dev(np.zeros(lib().pai_attention_workspace_bytes(hq, hd, ctx), np.uint8))
    for length in lens:  # one workspace for all calls: each leaves it reusable
        say(f"[gpu] attention hq={hq} hk={hk} hd={hd} ctx={ctx} len={length} qscale={qscale}")
        q = (rng.standard_normal((hq, hd)) * qscale).astype(np.float32)
        bq = dev(q)
        check(lib().pai_attention_decode_async(bq.ptr, bkc.ptr, bvc.ptr, bo.ptr, ws.ptr, hq, hk,
                                               hd, ctx, length, None),
              "pai_attention_decode_async")
        hm.synchronize()
        got = bo.download((hq, hd))
        want = ob.attention_last(hq, hk, length, q, kc.astype(np.float32), vc.astype(np.float32))
        exact = attention_f64(q, kc, vc, hq, hk, length)
        for h in range(hq):
            e_gpu, e_orc = rel_l2(got[h], exact[h]), rel_l2(want[h], exact[h])
            ok = rel_l2(got[h], want[h]) <= TOL_ATTN or e_gpu <= 2 * e_orc
            assert ok, (length, h, rel_l2(got[h], want[h]), e_gpu, e_orc)


def attention_f64(q, kc, vc, hq, hk, length):
    """Softmax attention of one query per head in float64 (the exact value
    both f32 evaluations approximate)."""
    hd = q.shape[1]
    out = np.empty((hq, hd))
    for h in range(hq):
        K = kc[h * hk // hq, :length].astype(np.float64)
        V = vc[h * hk // hq, :length].astype(np.float64)
        sc = K @ q[h].astype(np.float64) / np.sqrt(hd)
        pr = np.exp(sc - sc.max())
        out[h] = (pr / pr.sum()) @ V
    return out


@pytest.mark.parametrize("hq,hk,hd,r2,pos", [(32, 8, 128, 64, 2047), (32, 8, 128, 64, 64),
                                         (8, 2, 64, 16, 0), (16, 2, 256, 128, 130)])
def test_attention_rope_fused_equals_two_ops(hq, hk, hd, r2, pos):
    """One launch (RoPE + append + attention) gives bit for bit what
    pai_rope_kv_append_async followed by pai_attention_decode_async gives,
    in the output and in both caches."""
    say(f"[gpu] fused rope+attention hq={hq} hk={hk} hd={hd} r2={r2} pos={pos}")
    ctx = max(pos + 1, 160)
    rng = np.random.default_rng(pos + hd)
    kc0 = f16(rng.standard_normal((hk, ctx, hd)))
    vc0 = f16(rng.standard_normal((hk, ctx, hd)))
    q = rng.standard_normal((hq, hd)).astype(np.float32)
    k = rng.standard_normal((hk, hd)).astype(np.float32)
    v = rng.standard_normal((hk, hd)).astype(np.float32)
    c, s = ob.rope_tables(ctx, r2, 2 * r2, 500000.0)
    bq, bk, bv, bc, bs = dev(q), dev(k), dev(v), dev(c), dev(s)
    row = pos * r2 * 4
    wsb = lib().pai_attention_workspace_bytes(hq, hd, ctx)
    outs, caches = [], []
    for fused in (False, True):
        bkc, bvc = dev(kc0), dev(vc0)
        ws = dev(np.zeros(wsb, np.uint8))
        bo = hm.DeviceBuffer(4 * hq * hd)
        if fused:
            check(lib().pai_attention_decode_rope_async(
                bq.ptr, bk.ptr, bv.ptr, bc.ptr + row, bs.ptr + row, r2, bkc.ptr, bvc.ptr, bo.ptr,
                ws.ptr, hq, hk, hd, ctx, pos, None), "pai_attention_decode_rope_async")
        else:
            bqr = hm.DeviceBuffer(q.nbytes)
            check(lib().pai_rope_kv_append_async(bq.ptr, bk.ptr, bv.ptr, bqr.ptr, bkc.ptr, bvc.ptr,
                                                 bc.ptr + row, bs.ptr + row, hq, hk, hd, r2, ctx,
                                                 pos, None), "pai_rope_kv_append_async")
            check(lib().pai_attention_decode_async(bqr.ptr, bkc.ptr, bvc.ptr, bo.ptr, ws.ptr, hq,
                                                   hk, hd, ctx, pos + 1, None),
                  "pai_attention_decode_async")
        hm.synchronize()
        outs.append(bo.download((hq, hd)))
        caches.append((bkc.download((hk, ctx, hd), np.uint16), bvc.download((hk, ctx, hd), np.uint16)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])


def test_argmax():
    ws = hm.DeviceBuffer(lib().pai_argmax_workspace_bytes())
    out = hm.DeviceBuffer(4)
    rng = np.random.default_rng(11)

    def run(x):
        bx = dev(np.asarray(x, np.float32))
        check(lib().pai_argmax_f32_async(bx.ptr, len(x), out.ptr, ws.ptr, None),
              "pai_argmax_f32_async")
        hm.synchronize()
        return int(out.download(1, np.uint32)[0])

    for n in (1, 1000, 65537, 128256):
        say(f"[gpu] argmax n={n}")
        x = rng.standard_normal(n).astype(np.float32)
        assert run(x) == ob.argmax_first(x)
        if n > 10:
            i, j = sorted(rng.choice(n, 2, replace=False))
            x[i] = x[j] = x.max() + 1  # tie: the first index
            assert run(x) == ob.argmax_first(x) == i
            x[rng.choice(n, 5)] = np.nan  # NaNs after index 0 never win
            x[0] = 0.0
            assert run(x) == ob.argmax_first(x)
            x[0] = np.nan  # NaN at 0 wins
            assert run(x) == ob.argmax_first(x) == 0
    assert run(np.full(300, -np.inf)) == 0
    assert run(np.full(300, np.nan)) == 0


# ---------------------------------------------------------------- model step
MODELS = {
    # 2 layers, head size 64, two q heads per KV head
    "small": (LlamaConfig(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, n_ff=512, vocab=1000,
                          ctx=96, n_rot=0, rope_theta=500000.0, norm_eps=0.0), 70),
    # head size 128 and four q heads per KV head (the 8B-model ratio)
    "hd128": (LlamaConfig(n_layer=1, n_embd=1024, n_head=8, n_head_kv=2, n_ff=1536, vocab=2048,
                          ctx=160, n_rot=0, rope_theta=500000.0, norm_eps=0.0), 130),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_decode_steps_match_oracle(name):
    cfg, prefill = MODELS[name]
    say(f"[gpu] decode model={name} prefill={prefill}")
    w = synthetic_weights(cfg, seed=0x5EED + len(name))
    d = cfg.as_dict()
    layers, head = dequantized_model(d, w)
    orc = ob.LlamaOracle(d, layers, head, kv_f16=True)
    m = upload(cfg, w)
    hd = cfg.n_embd // cfg.n_head
    rng = np.random.default_rng(prefill)
    for L in range(cfg.n_layer):
        k = f16(rng.standard_normal((prefill, cfg.n_head_kv, hd)))
        v = f16(rng.standard_normal((prefill, cfg.n_head_kv, hd)))
        m.kv_write(L, 0, k, v)
        orc.k_cache[L, :, :prefill] = k.astype(np.float32).transpose(1, 0, 2)
        orc.v_cache[L, :, :prefill] = v.astype(np.float32).transpose(1, 0, 2)
    token = 7
    for pos in range(prefill, prefill + 6):
        nxt, logits = m.decode(token, pos)
        want, want_next = orc.step(token, pos)
        err = rel_l2(logits, want)
        say(f"[gpu]   pos={pos} token={token} rel_l2={err:.2e} next={nxt}/{want_next}")
        assert err <= TOL_LOGITS, (pos, err)
        assert nxt == int(np.argmax(logits)) or not np.isfinite(logits).all()
        if nxt != want_next:
            top = np.sort(want)[-2:]
            assert top[1] - top[0] <= 1e-4 * abs(top[1]), (pos, nxt, want_next)
        # this step's keys and values are in both caches
        kd, vd = m.kv_cache(0)
        got_k = _download(kd, (cfg.n_head_kv, cfg.ctx, hd))[:, pos].astype(np.float32)
        got_v = _download(vd, (cfg.n_head_kv, cfg.ctx, hd))[:, pos].astype(np.float32)
        assert rel_l2(got_k, orc.k_cache[0, :, pos]) <= 1e-3
        assert rel_l2(got_v, orc.v_cache[0, :, pos]) <= 1e-3
        token = nxt
    m.free()


def _download(ptr: int, shape) -> np.ndarray:
    out = np.empty(shape, np.float16)
    hm.hip_check(hm.hip().hipMemcpy(out.ctypes.data, ptr, out.nbytes, hm.D2H), "hipMemcpy D2H")
    return out


def test_decode_async_chain_is_deterministic():
    """Steps chained on the device (token in and out of device memory) give
    the synchronous steps' tokens and bit-identical logits."""
    cfg, prefill = MODELS["small"]
    say("[gpu] decode async chain")
    w = synthetic_weights(cfg, seed=0xA5)
    m = upload(cfg, w)
    toks = [3]
    logits_sync = None
    for pos in range(4):
        nxt, logits_sync = m.decode(toks[-1], pos)
        toks.append(nxt)
    tok = hm.DeviceBuffer.from_array(np.array([3, 0], np.uint32))
    s = hm.Stream()
    for pos in range(4):
        # ping-pong: step pos reads slot pos % 2 and writes the other
        a, b = tok.ptr + 4 * (pos % 2), tok.ptr + 4 * ((pos + 1) % 2)
        m.decode_async(a, pos, b, s.handle)
    s.synchronize()
    got = tok.download(2, np.uint32)
    assert int(got[4 % 2]) == toks[-1]
    out = np.empty(cfg.vocab, np.float32)
    hm.hip_check(hm.hip().hipMemcpy(out.ctypes.data, m.logits_ptr(), out.nbytes, hm.D2H), "D2H")
    assert np.array_equal(out.view(np.uint32), logits_sync.view(np.uint32))
    s.destroy()
    m.free()
