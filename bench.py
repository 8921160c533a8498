#!/usr/bin/env python3
"""Quantized-weights GEMV/GEMM benchmark on one MI355X.

Headline (the JSON `value`): Q4_K decode GEMV, M=1 (the north-star
format), over the seven Llama-3-8B per-layer projections (q, o: 4096x4096; k, v: 1024x4096;
gate, up: 14336x4096; down: 4096x14336), issued as one layer's decode step:
q/k/v in one fused call (they share the attention input), o, gate/up in one
fused call (they share the FFN input), down -- four launches streaming the
seven matrices. Steps rotate over --layers distinct weight copies so the
working set (123 MB per layer) exceeds the 256 MB Infinity Cache. Weights
are f32 N(0, 0.02^2) from a fixed seed, quantized by libpai_hip's K-quant
encoder; activations are f32 N(0, 1), resident in HBM.

value    = algorithmic bytes (packed W + x + y, f32) of all timed steps
           / wall time between two stream synchronisations.
roofline = the GEMV kernel: the same bytes / the sum of its launch
           durations (HIP events around every launch, on the launch stream),
           against 8 TB/s.
cpu_baseline = the reference's AVX2+FMA GEMV (cpu/optimized/opt_ops.c,
           compiled from its sources into oracle/_ref; this repository's
           restatement when that build is absent) on the dequantized f32
           weights of the same seven projections, one host core.
extra    = the same step in Q4_0 (fused, as seven separate launches, and
           with silu(gate)*up fused into the gate/up launch); Q4_K at M in
           {8, 32}; Q8_0 4096x4096 GEMV; and the M=512 prefill GEMMs
           (gate Q4_K, down Q6_K, and gate+up with the fused silu*mul) in
           TFLOP/s against 2.5 PFLOP/s dense fp16; and the full decode step
           of a Llama-3-8B-shape model with an fp16 KV cache at context
           2048 (ms/token, and GB/s over its weight, cache and embedding
           bytes).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
PROJ = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
        ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
METRIC = "quant GEMV GB/s (%HBM peak) at 8B shapes; M=512 GEMM TFLOPS"
HEAD_QTYPE, HEAD_CONFIG = 12, 3  # Q4_K, the third configuration (M in {1, 8, 32}) at M = 1
HEAD_NAME = "Q4_K"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def seed_w(config: int, idx: int) -> int:
    return 0xC0DE0000 + 16 * config + idx


def call_bytes(pa, qtype: int, n: int, k: int, m: int = 1) -> int:
    return n * pa.qtype_bytes(qtype, k) + m * (k + n) * 4


class Layer:
    """One layer's seven packed projections on the device."""

    def __init__(self, pa, qtype: int, blocks: list):
        self.qtype = qtype
        self.w = [pa.QMat(qtype, n, k, b) for (_, n, k), b in zip(PROJ, blocks)]


def quantized_layer(pa, qtype: int, config: int) -> list:
    out = []
    for i, (_, n, k) in enumerate(PROJ):
        w = pa.normal_f32(seed_w(config, i), n * k, 0.0, 0.02).reshape(n, k)
        out.append(pa.quantize(qtype, w))
    return out


# The launches of one layer's decode step: projections that share their
# input run as one fused call (q/k/v on the attention input, gate/up on the
# FFN input); o and down stand alone.
FUSED_STEP = [("qkv", [0, 1, 2]), ("o", [3]), ("gate_up", [4, 5]), ("down", [6])]
SEPARATE_STEP = [(name, [i]) for i, (name, _, _) in enumerate(PROJ)]
# The same step with the FFN activation fused into the gate/up launch:
# h = silu(gate) * up is written instead of the two products.
SILU_STEP = [("qkv", [0, 1, 2]), ("o", [3]), ("gate_up_silu", [4, 5]), ("down", [6])]


def enqueue_entry(pa, layer, name, idx, m, xp, yp, sh):
    if name == "gate_up_silu":
        pa.gate_up_async(layer.w[idx[0]], layer.w[idx[1]], xp, yp[idx[0]], m, 0, sh)
    elif len(idx) == 1:
        layer.w[idx[0]].gemm_async(xp, yp[idx[0]], m, 0, sh)
    else:
        pa.gemm_multi_async([layer.w[i] for i in idx], xp, [yp[i] for i in idx], m, 0, sh)


def entry_bytes(pa, qtype, name, idx, m):
    """Algorithmic bytes of one plan entry: packed weights, x once, outputs."""
    if name == "gate_up_silu":
        n, k = PROJ[idx[0]][1], PROJ[idx[0]][2]
        return len(idx) * n * pa.qtype_bytes(qtype, k) + m * (k + n) * 4
    return sum(call_bytes(pa, qtype, PROJ[i][1], PROJ[i][2], m) for i in idx)


def run_layers(pa, hm, layers, m: int, steps: int, warmup: int, plan):
    """Time `steps` passes over the seven projections, rotating layers. The
    passes over all layer copies, in order, are captured once into one HIP
    graph (as a model's decode step over its layers would be), so a step is
    the launches of `plan` on one layer copy and there is no host work
    between steps. The timed region
    is bracketed by events on the launch stream, so the GPU time per step is
    the kernels' time plus the gaps between them inside the graph."""
    stream = hm.Stream()
    kmax = max(k for _, _, k in PROJ)
    x = hm.DeviceBuffer.from_array(pa.normal_f32(0xC0DE0000 ^ 0x5A5A, m * kmax))
    ys = [hm.DeviceBuffer(m * n * 4) for _, n, _ in PROJ]
    xp, yp = x.ptr, [y.ptr for y in ys]

    def enqueue(layer, sh):
        for name, idx in plan:
            enqueue_entry(pa, layer, name, idx, m, xp, yp, sh)

    nl = len(layers)
    for l in layers:  # eager pass first: per-matrix workspaces are allocated outside capture
        enqueue(l, stream.handle)
    stream.synchronize()
    graph = hm.Graph(stream, lambda sh: [enqueue(l, sh) for l in layers])
    rem = steps % nl  # a shorter graph over the first layers finishes the count
    tail = hm.Graph(stream, lambda sh: [enqueue(l, sh) for l in layers[:rem]]) if rem else None
    for _ in range(max(1, -(-warmup // nl))):
        graph.launch(stream)
    stream.synchronize()
    a, b = hm.Event(), hm.Event()
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(steps // nl):
        graph.launch(stream)
    if tail is not None:
        tail.launch(stream)
    b.record(stream)
    stream.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = a.elapsed_ms(b)
    graph.destroy()
    if tail is not None:
        tail.destroy()
    a.destroy(); b.destroy()
    for buf in [x, *ys]:
        buf.free()
    stream.destroy()
    return wall, gpu_ms / steps


def per_launch_times(pa, hm, layers, m: int, plan, reps: int = 50) -> dict:
    """Microseconds per launch of each entry of `plan` (events around `reps`
    back-to-back launches of that entry, rotating layers, on one stream)."""
    stream = hm.Stream()
    kmax = max(k for _, _, k in PROJ)
    x = hm.DeviceBuffer.from_array(pa.normal_f32(0xC0DE0000 ^ 0x5A5A, m * kmax))
    ys = [hm.DeviceBuffer(m * n * 4) for _, n, _ in PROJ]
    out = {}
    for name, idx in plan:
        def one(sh, r):
            enqueue_entry(pa, layers[r % len(layers)], name, idx, m, x.ptr,
                          [y.ptr for y in ys], sh)
        for r in range(len(layers)):  # eager first: workspaces are allocated outside capture
            one(stream.handle, r)
        stream.synchronize()
        g = hm.Graph(stream, lambda sh: [one(sh, r) for r in range(reps)])
        g.launch(stream)
        stream.synchronize()
        a, b = hm.Event(), hm.Event()
        a.record(stream)
        g.launch(stream)
        b.record(stream)
        b.synchronize()
        us = a.elapsed_ms(b) * 1e3 / reps
        nbytes = entry_bytes(pa, layers[0].qtype, name, idx, m)
        out[name] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
        a.destroy(); b.destroy(); g.destroy()
    for buf in [x, *ys]:
        buf.free()
    stream.destroy()
    return out


def gemv_config(pa, hm, qtype: int, config: int, m: int, nlayers: int, steps: int,
                warmup: int, plan=FUSED_STEP, launch_detail: bool = True) -> dict:
    blocks = quantized_layer(pa, qtype, config)
    layers = [Layer(pa, qtype, blocks) for _ in range(nlayers)]
    wall, gpu_ms = run_layers(pa, hm, layers, m, steps, warmup, plan)
    bytes_step = sum(entry_bytes(pa, qtype, name, idx, m) for name, idx in plan)
    res = {"qtype": qtype, "m": m, "layers": nlayers, "steps": steps,
           "launches_per_step": len(plan),
           "weight_set_MB": round(nlayers * sum(l.nbytes for l in layers[0].w) / 1e6, 1),
           "bytes_per_step": bytes_step, "ms_per_step": wall / steps * 1e3,
           "GBps": bytes_step * steps / wall / 1e9,
           "gpu_ms_per_step": gpu_ms, "gpu_GBps": bytes_step / (gpu_ms * 1e-3) / 1e9}
    if launch_detail:
        res["per_launch"] = per_launch_times(pa, hm, layers, m, plan)
    for l in layers:
        for w in l.w:
            w.free()
    return res


def timed_calls(hm, call, reps: int, warm: int) -> float:
    """Mean microseconds per call of `call(stream_handle, i)`: `reps` calls
    captured into one HIP graph, replayed between two events on one
    stream."""
    st = hm.Stream()
    call(st.handle, 0)  # eager call first: workspaces are allocated outside capture
    st.synchronize()
    warm_g = hm.Graph(st, lambda sh: [call(sh, i) for i in range(warm)])
    g = hm.Graph(st, lambda sh: [call(sh, i) for i in range(reps)])
    warm_g.launch(st)
    st.synchronize()
    a, b = hm.Event(), hm.Event()
    a.record(st)
    g.launch(st)
    b.record(st)
    b.synchronize()
    us = a.elapsed_ms(b) / reps * 1e3
    a.destroy(); b.destroy(); g.destroy(); warm_g.destroy(); st.destroy()
    return us


def q8_config1(pa, hm, steps: int) -> dict:
    n = k = 4096
    w = pa.normal_f32(seed_w(1, 0), n * k, 0.0, 0.02).reshape(n, k)
    blocks = pa.quantize(pa.Q8_0, w)
    copies = [pa.QMat(pa.Q8_0, n, k, blocks) for _ in range(32)]  # 570 MB
    x = hm.DeviceBuffer.from_array(pa.normal_f32(seed_w(1, 0) ^ 0x5A5A, k))
    y = hm.DeviceBuffer(n * 4)
    us = timed_calls(hm, lambda sh, i: copies[i % 32].gemm_async(x.ptr, y.ptr, 1, 0, sh),
                     steps, 64)
    b = call_bytes(pa, pa.Q8_0, n, k)
    for c in copies:
        c.free()
    return {"us_per_call": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)}


def host_pointer_step(pa, reps: int = 50) -> dict:
    """The seven headline-format projections through the synchronous host-pointer
    entry point (pai_qgemm_f32 without PAI_QGEMM_DEVICE_PTRS: x is copied
    to the device and y back over PCIe on every call), wall clock per
    step. Reported beside the HBM-resident figure, never as the value."""
    blocks = quantized_layer(pa, HEAD_QTYPE, HEAD_CONFIG)
    layer = Layer(pa, HEAD_QTYPE, blocks)
    kmax = max(k for _, _, k in PROJ)
    x = pa.normal_f32(0xC0DE0000 ^ 0x5A5A, kmax)
    xs = [x[:k] for _, _, k in PROJ]
    for w, xv in zip(layer.w, xs):
        w.gemm(xv)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for w, xv in zip(layer.w, xs):
            w.gemm(xv)
        times.append(time.perf_counter() - t0)
    for w in layer.w:
        w.free()
    med = float(np.median(times))
    b = sum(call_bytes(pa, HEAD_QTYPE, n, k) for _, n, k in PROJ)
    return {"us_per_step": round(med * 1e6, 1), "GBps": round(b / med / 1e9, 1),
            "calls_per_step": len(PROJ)}


def prefill(pa, hm, reps: int) -> dict:
    out = {}
    m = 512
    for name, qtype, (n, k), cfg in (("gate_q4_k", pa.Q4_K, (14336, 4096), 4),
                                     ("down_q6_k", pa.Q6_K, (4096, 14336), 4)):
        w = pa.normal_f32(seed_w(cfg, 0 if qtype == pa.Q4_K else 6), n * k, 0.0, 0.02)
        qm = pa.QMat(qtype, n, k, pa.quantize(qtype, w.reshape(n, k)))
        x = hm.DeviceBuffer.from_array(pa.normal_f32(seed_w(cfg, 9), m * k))
        y = hm.DeviceBuffer(m * n * 4)
        us = timed_calls(hm, lambda sh, i: qm.gemm_async(x.ptr, y.ptr, m, 0, sh), reps, 3)
        tflops = 2.0 * m * n * k / (us * 1e-6) / 1e12
        out[name] = {"us": round(us, 1), "TFLOPs": round(tflops, 1),
                     "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 3)}
        qm.free(); x.free(); y.free()
    # gate and up (Q4_K 14336 x 4096) with h = silu(gate) * up fused
    n, k = 14336, 4096
    mats = [pa.QMat(pa.Q4_K, n, k, pa.quantize(pa.Q4_K, pa.normal_f32(
        seed_w(4, i), n * k, 0.0, 0.02).reshape(n, k))) for i in (4, 5)]
    x = hm.DeviceBuffer.from_array(pa.normal_f32(seed_w(4, 9), m * k))
    h = hm.DeviceBuffer(m * n * 4)
    us = timed_calls(hm, lambda sh, i: pa.gate_up_async(mats[0], mats[1], x.ptr, h.ptr, m, 0, sh),
                     reps, 3)
    tflops = 2.0 * 2.0 * m * n * k / (us * 1e-6) / 1e12
    out["gate_up_silu_q4_k"] = {"us": round(us, 1), "TFLOPs": round(tflops, 1),
                                "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 3)}
    for w in mats:
        w.free()
    x.free(); h.free()
    g = out["gate_q4_k"]
    out["roofline"] = {"bound": "mfma", "achieved": g["TFLOPs"], "peak": MFMA_F16_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": g["frac_mfma_f16"], "traffic": None,
                       "workload": "gate Q4_K 14336x4096 at M=512 (one call: activation "
                                   "conversion + GEMM, HIP events around graph-captured calls)"}
    return out


DECODE_SHAPES = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
                 "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}


def decode_8b(pa, hm, steps: int, warmup: int, fill: int = 2048, threads: int = 8) -> dict:
    """One greedy decode step of a random-init Llama-3-8B-shape model
    (32 layers, hidden 4096, 32/8 heads, FFN 14336, vocab 128256, RoPE
    theta 500000) with the fp16 KV cache prefilled to `fill` positions.
    Q4_K weights, Q6_K ffn_down and output head, N(0, 0.02^2) per matrix
    from its own seed; norms 1; cache N(0, 1). Steps run on one stream,
    the token passed on the device from step to step (eager launches), and
    again as one captured step replayed (HIP graph)."""
    import concurrent.futures as cf
    from prosperoai_amd.llama import Llama, LlamaConfig
    cfg = LlamaConfig(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336,
                      vocab=128256, ctx=fill + warmup + steps + 2, n_rot=0,
                      rope_theta=500000.0, norm_eps=0.0)
    t0 = time.time()
    qt = {n: (pa.Q6_K if n == "down" else pa.Q4_K) for n in DECODE_SHAPES}

    def make(job):
        name, n, k, seed, qtype = job
        w = pa.normal_f32(seed, n * k, 0.0, 0.02).reshape(n, k)
        return job, pa.quantize(qtype, w, 1)

    jobs = [(nm, n, k, seed_w(5, 0) + 64 * L + i, qt[nm])
            for L in range(cfg.n_layer) for i, (nm, (n, k)) in enumerate(DECODE_SHAPES.items())]
    rows = 128256 // 8  # the two vocab matrices in 8 row bands each
    for name, qtype, base in (("token_embd", pa.Q4_K, 1 << 20), ("output", pa.Q6_K, 1 << 21)):
        jobs += [(f"{name}:{b}", rows, 4096, seed_w(5, 0) + base + b, qtype) for b in range(8)]
    m = Llama(cfg)
    mats, bands = {}, {}
    weight_bytes = 0
    with cf.ThreadPoolExecutor(threads) as ex:
        for (name, n, k, seed, qtype), blocks in ex.map(make, jobs):
            if ":" in name:
                bands[name] = (qtype, blocks)
                continue
            L = (seed - seed_w(5, 0)) // 64
            mats[(L, name)] = pa.QMat(qtype, n, k, blocks)
            weight_bytes += blocks.nbytes
            if all((L, nm) in mats for nm in DECODE_SHAPES):
                m.set_layer(L, {nm: mats[(L, nm)] for nm in DECODE_SHAPES},
                            np.ones(4096, np.float32), np.ones(4096, np.float32))
    head = {}
    for name in ("token_embd", "output"):
        qtype = bands[f"{name}:0"][0]
        blocks = np.concatenate([bands[f"{name}:{b}"][1] for b in range(8)])
        head[name] = pa.QMat(qtype, 128256, 4096, blocks)
        if name == "output":
            weight_bytes += blocks.nbytes
    bands.clear()
    m.set_output(head["token_embd"], head["output"], np.ones(4096, np.float32))
    rng = np.random.default_rng(seed_w(5, 15))
    for L in range(cfg.n_layer):
        k = rng.standard_normal((fill, 8, 128), dtype=np.float32).astype(np.float16)
        v = rng.standard_normal((fill, 8, 128), dtype=np.float32).astype(np.float16)
        m.kv_write(L, 0, k, v)
    setup_s = time.time() - t0
    log(f"decode 8B: model built in {setup_s:.1f} s")

    tok = hm.DeviceBuffer.from_array(np.array([1, 0], np.uint32))
    st = hm.Stream()

    def step(pos, sh):  # step pos reads slot pos % 2, writes the other
        m.decode_async(tok.ptr + 4 * (pos % 2), pos, tok.ptr + 4 * ((pos + 1) % 2), sh)

    for i in range(warmup):
        step(fill + i, st.handle)
    st.synchronize()
    a, b = hm.Event(), hm.Event()
    a.record(st)
    for i in range(steps):
        step(fill + warmup + i, st.handle)
    b.record(st)
    b.synchronize()
    eager_ms = a.elapsed_ms(b) / steps
    # one captured step at a fixed position, replayed
    pos_g = fill + warmup + steps
    g = hm.Graph(st, lambda sh: step(pos_g, sh))
    g.launch(st)
    st.synchronize()
    a.record(st)
    for _ in range(steps):
        g.launch(st)
    b.record(st)
    b.synchronize()
    graph_ms = a.elapsed_ms(b) / steps
    # the last step's token is the argmax of its logits, and they are finite
    logits = np.empty(cfg.vocab, np.float32)
    hm.hip_check(hm.hip().hipMemcpy(logits.ctypes.data, m.logits_ptr(), logits.nbytes, hm.D2H),
                 "logits")
    nxt = int(tok.download(2, np.uint32)[(pos_g + 1) % 2])
    ok = bool(np.isfinite(logits).all() and nxt == int(np.argmax(logits)))
    kv_bytes = 32 * 2 * 8 * 128 * 2 * (fill + warmup + steps // 2 + 1)  # mean cache read
    emb_row = pa.qtype_bytes(pa.Q4_K, 4096)
    step_bytes = weight_bytes + kv_bytes + emb_row
    out = {"ms_per_token": round(eager_ms, 4), "tokens_per_s": round(1e3 / eager_ms, 1),
           "GBps": round(step_bytes / (eager_ms * 1e-3) / 1e9, 1),
           "frac_hbm": round(step_bytes / (eager_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "graph_ms_per_token": round(graph_ms, 4),
           "graph_GBps": round(step_bytes / (graph_ms * 1e-3) / 1e9, 1),
           "bytes_per_token": step_bytes, "weight_bytes": weight_bytes, "kv_bytes": kv_bytes,
           "context": fill, "steps": steps, "argmax_ok": ok, "setup_s": round(setup_s, 1)}
    g.destroy(); a.destroy(); b.destroy(); st.destroy(); tok.free()
    m.free()
    for w in list(mats.values()) + list(head.values()):
        w.free()
    return out


def cpu_baseline(pa, budget_s: float) -> dict:
    """The reference's single-thread AVX2 GEMV on dequantized f32 weights of
    the seven headline-format projections (bounded number of passes)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_bind as ob
    r = ob.ref()
    kind = "reference" if r is not None else "port"
    blocks = quantized_layer(pa, HEAD_QTYPE, HEAD_CONFIG)
    mats = []
    for (_, n, k), b in zip(PROJ, blocks):
        if r is not None:
            mats.append(ob.ref_dequant(HEAD_QTYPE, b.tobytes(), n * k, row=k).reshape(n, k))
        else:
            mats.append(ob.dequant(HEAD_QTYPE, b, n * k).reshape(n, k))
    kmax = max(k for _, _, k in PROJ)
    x = pa.normal_f32(0xC0DE0000 ^ 0x5A5A, kmax)
    ys = [np.empty(n, np.float32) for _, n, _ in PROJ]
    gemv = r.pai_opt_gemv_f32 if r is not None else ob.oracle().orc_opt_gemv_avx2

    def one_pass():
        for (_, n, k), a, y in zip(PROJ, mats, ys):
            gemv(n, k, a.ctypes.data, x.ctypes.data, y.ctypes.data)

    for _ in range(2):
        one_pass()
    times = []
    t_start = time.perf_counter()
    while len(times) < 10 or (time.perf_counter() - t_start < budget_s and len(times) < 200):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    bytes_step = sum(call_bytes(pa, HEAD_QTYPE, n, k) for _, n, k in PROJ)
    med = float(np.median(times))

    def timed(fn, budget: float, least: int = 3) -> list:
        fn()
        ts, t_start = [], time.perf_counter()
        while len(ts) < least or (time.perf_counter() - t_start < budget and len(ts) < 100):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return ts

    # the same GEMV, rows split over every host core (a pthread wrapper
    # around the same AVX2 row kernel; the reference itself runs one thread)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))  # the host share of one GPU
    orc = ob.oracle()

    def mt_pass():
        for (_, n, k), a, y in zip(PROJ, mats, ys):
            orc.orc_opt_gemv_avx2_mt(n, k, a.ctypes.data, x.ctypes.data, y.ctypes.data, threads)

    mt_times = timed(mt_pass, min(5.0, budget_s / 3))
    mt_med = float(np.median(mt_times))
    # the reference's int8-weight GEMM at group size 32 (the Q8_0 analogue),
    # M=1 on the 4096 x 4096 shape of the Q8_0 configuration: w_q [K][N]
    w8 = None
    if r is not None:
        n8 = k8 = 4096
        rng = np.random.default_rng(8)
        wq = rng.integers(-127, 128, size=(k8, n8), dtype=np.int8)
        sc = (rng.random((k8 // 32, n8), dtype=np.float32) * 1e-3).astype(np.float32)
        x8 = pa.normal_f32(0x8808, k8)
        y8 = np.empty(n8, np.float32)
        w8_times = timed(lambda: r.pai_opt_gemm_w8_f32(1, n8, k8, x8.ctypes.data, wq.ctypes.data,
                                                       sc.ctypes.data, 32, y8.ctypes.data),
                         min(3.0, budget_s / 5))
        w8_med = float(np.median(w8_times))
        q8_bytes = call_bytes(pa, pa.Q8_0, n8, k8)
        w8 = {"GBps": round(q8_bytes / w8_med / 1e9, 2), "ms": round(w8_med * 1e3, 3),
              "cores": 1, "sample": f"{len(w8_times)} calls of pai_opt_gemm_w8_f32, M=1, "
                                    f"N=K=4096, group 32; GB/s counts the Q8_0 bytes of the "
                                    f"same shape"}
    return {"value": round(bytes_step / med / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": kind,
            "harness_parallel": {"value": round(bytes_step / mt_med / 1e9, 2), "unit": "GB/s",
                                 "cores": threads, "kind": "port",
                                 "sample": f"{len(mt_times)} passes, orc_opt_gemv_avx2_mt "
                                           f"(the AVX2 row kernel, rows split over {threads} "
                                           f"threads)"},
            "w8_gemm_q8_0_shape": w8,
            "sample": f"{len(times)} passes over the seven {HEAD_NAME} projections of one layer "
                      f"(pai_opt_gemv_f32 on dequantized f32 [N][K], 4 B/weight touched); "
                      f"median {med * 1e3:.1f} ms/pass, min {min(times) * 1e3:.1f} ms; "
                      f"GB/s counts the same packed bytes as the GPU value",
            "host_cpu": _cpu_model(), "host_nproc": os.cpu_count()}


def copy_calibration(hm, mib: int, reps: int = 4) -> None:
    """`reps` device-to-device copies of `mib` MiB (the runtime's copy
    kernel): a dispatch whose HBM traffic is known exactly (reads and
    writes mib MiB each), against which the FETCH_SIZE / WRITE_SIZE counters
    of a profiling run are scaled."""
    n = mib << 20
    src, dst = hm.DeviceBuffer(n), hm.DeviceBuffer(n)
    st = hm.Stream()
    for _ in range(reps):
        hm.hip_check(hm.hip().hipMemcpyAsync(dst.ptr, src.ptr, n, hm.D2D, st.handle),
                     "hipMemcpyAsync D2D")
    st.synchronize()
    st.destroy(); src.free(); dst.free()


def pmc_summary(fetch_csv: str, write_csv: str, copy_mib: int, kernel: str) -> dict:
    """Per-dispatch HBM traffic of `kernel` (a substring of the kernel
    name) from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; KiB per
    dispatch), each scaled by the ratio of known bytes to counted bytes of
    the copy dispatches (copy_calibration) in the same run."""
    import csv

    def read(path, counter):
        per = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            key = r["Dispatch_Id"]
            per.setdefault(key, [r["Kernel_Name"], 0.0])[1] += float(r["Counter_Value"])
        copies = [v for n, v in per.values() if "copyBuffer" in n]
        kern = [v for n, v in per.values() if kernel in n]
        if not copies or not kern:
            raise RuntimeError(f"{path}: {len(copies)} copy and {len(kern)} '{kernel}' dispatches")
        copy_bytes = float(copy_mib << 20)
        scale = copy_bytes / (np.mean(copies) * 1024.0)
        return np.mean(kern) * 1024.0, scale, len(kern), len(copies), float(np.mean(copies))

    f_b, f_s, nk, nc, f_c = read(fetch_csv, "FETCH_SIZE")
    w_b, w_s, _, _, w_c = read(write_csv, "WRITE_SIZE")
    return {"kernel": kernel, "dispatches": nk, "copy_dispatches": nc, "copy_MiB": copy_mib,
            "copy_fetch_KiB": round(f_c, 1), "copy_write_KiB": round(w_c, 1),
            "fetch_scale": round(f_s, 4), "write_scale": round(w_s, 4),
            "fetch_bytes_per_dispatch": round(f_b * f_s),
            "write_bytes_per_dispatch": round(w_b * w_s),
            "traffic_bytes_per_launch": round(f_b * f_s + w_b * w_s)}


def kernel_pmc_summary(paths: list) -> dict:
    """Per-kernel means of rocprofv3 --pmc CSVs (counter_collection): the
    dispatch count, the duration between each dispatch's start and end
    timestamps, and every counter's mean per dispatch. With
    SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE in the same pass, MFMA busy
    = SIMD cycles with an MFMA in flight / (GPU cycles x 1024 SIMDs), where
    GPU cycles = GRBM_GUI_ACTIVE / 8 (the counter is summed over the 8
    XCDs); with the MOPS counters, flops = MOPS x 512."""
    import csv
    out = {}
    for path in paths:
        per = {}
        for r in csv.DictReader(open(path)):
            d = per.setdefault(r["Dispatch_Id"], {"kernel": r["Kernel_Name"].split("(")[0],
                                                  "grid": int(r["Grid_Size"]),
                                                  "ns": int(r["End_Timestamp"]) -
                                                        int(r["Start_Timestamp"])})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for d in per.values():
            key = f"{d['kernel']} grid={d['grid']}"
            e = out.setdefault(key, {"file": path, "dispatches": 0, "sums": {}})
            if e["file"] != path:
                key = f"{key} [{Path(path).parent.name}]"
                e = out.setdefault(key, {"file": path, "dispatches": 0, "sums": {}})
            e["dispatches"] += 1
            for c, v in d.items():
                if c not in ("kernel", "grid"):
                    e["sums"][c] = e["sums"].get(c, 0.0) + v
    for e in out.values():
        mean = {c: v / e["dispatches"] for c, v in e.pop("sums").items()}
        e["mean_us"] = round(mean.pop("ns") / 1e3, 2)
        e["counters"] = {c: round(v, 1) for c, v in mean.items()}
        if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and "GRBM_GUI_ACTIVE" in mean:
            cyc = mean["GRBM_GUI_ACTIVE"] / 8.0
            e["gpu_cycles"] = round(cyc)
            e["clock_GHz"] = round(cyc / (e["mean_us"] * 1e3), 3)
            e["mfma_busy"] = round(mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * 1024.0), 4)
        mops = mean.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) + mean.get(
            "SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        if mops:
            e["mfma_flop"] = mops * 512.0
            e["TFLOPs"] = round(mops * 512.0 / (e["mean_us"] * 1e-6) / 1e12, 1)
            e["frac_mfma_f16"] = round(e["TFLOPs"] / MFMA_F16_PEAK_TFLOPS, 4)
    return out


def trace_summary(trace_csv: str, steps: int, warmup: int, layers: int) -> dict:
    """Kernel durations of the headline's timed region from a rocprofv3
    --kernel-trace CSV of a default run: the first headline GEMV dispatches are
    the eager pass over the layers and the warm-up graph replays, then come
    the timed steps (4 launches each, in step order qkv, o, gate_up, down)."""
    import csv
    rows = [r for r in csv.DictReader(open(trace_csv))
            if f"k_gemv<paik::{HEAD_NAME}" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    nl = len(FUSED_STEP)
    skip = nl * layers + nl * layers * max(1, -(-warmup // layers))
    timed = rows[skip:skip + nl * steps]
    if len(timed) != nl * steps:
        raise RuntimeError(f"{trace_csv}: {len(rows)} {HEAD_NAME} GEMV dispatches, "
                           f"expected {skip} + {nl * steps}")
    dur = np.array([int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in timed], float)
    out = {"dispatches": len(timed), "skipped": skip,
           "mean_ns": round(float(dur.mean()), 1),
           "span_ns_per_launch": round((int(timed[-1]["End_Timestamp"]) -
                                        int(timed[0]["Start_Timestamp"])) / len(timed), 1)}
    for i, (name, _) in enumerate(FUSED_STEP):
        d = dur[i::nl]
        out[name] = {"kernel": timed[i]["Kernel_Name"], "grid": int(timed[i]["Grid_Size_X"]),
                     "workgroup": int(timed[i]["Workgroup_Size_X"]),
                     "mean_ns": round(float(d.mean()), 1), "median_ns": round(float(np.median(d)), 1),
                     "min_ns": round(float(d.min()), 1)}
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--layers", type=int, default=6)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-launch-detail", action="store_true",
                    help="skip the per-launch timings of the headline step")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="end with device copies of this size (counter calibration)")
    ap.add_argument("--decode-only", type=int, metavar="STEPS", default=0,
                    help="run only the full-model decode step (Llama-3-8B shape, fp16 KV "
                         "cache at context 2048) for STEPS timed steps and print its JSON")
    ap.add_argument("--prefill-only", type=int, metavar="REPS", default=0,
                    help="run only the M=512 prefill GEMMs (REPS graph-captured calls per "
                         "shape) and print their JSON")
    ap.add_argument("--kernel-pmc-summary", nargs="+", metavar="PMC_CSV",
                    help="per-kernel durations and counter means of rocprofv3 --pmc CSVs, "
                         "then exit")
    ap.add_argument("--pmc-kernel", default=f"k_gemv<paik::{HEAD_NAME}",
                    help="kernel-name substring for --pmc-summary")
    ap.add_argument("--trace-summary", metavar="TRACE_CSV",
                    help="summarise the headline's timed-region GEMV dispatches of a "
                         "rocprofv3 --kernel-trace CSV of a run with the same --steps, "
                         "--warmup and --layers, then exit")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "this script with --calib-copy-mib, then exit")
    args = ap.parse_args()
    if args.trace_summary:
        print(json.dumps(trace_summary(args.trace_summary, args.steps, args.warmup, args.layers),
                         indent=1))
        return 0
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, args.calib_copy_mib or 64,
                                     args.pmc_kernel)))
        return 0
    if args.kernel_pmc_summary:
        print(json.dumps(kernel_pmc_summary(args.kernel_pmc_summary), indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the path has no multi-GPU sharding in this build)", file=sys.stderr)
        return 2

    import prosperoai_amd as pa
    from prosperoai_amd import hipmem as hm
    pa.init()
    if args.decode_only:
        print(json.dumps(decode_8b(pa, hm, args.decode_only, 5)), flush=True)
        return 0
    if args.prefill_only:
        print(json.dumps(prefill(pa, hm, args.prefill_only)), flush=True)
        if args.calib_copy_mib:
            copy_calibration(hm, args.calib_copy_mib)
        return 0
    log(f"{HEAD_NAME} M=1 x {args.layers} layers")

    head = gemv_config(pa, hm, HEAD_QTYPE, HEAD_CONFIG, 1, args.layers, args.steps, args.warmup,
                       launch_detail=not args.no_launch_detail)
    log(f"{HEAD_NAME} M=1 fused step: {head['GBps']:.1f} GB/s wall, {head['gpu_GBps']:.1f} GB/s GPU; "
        f"{head.get('per_launch')}")
    avg_us = head["gpu_ms_per_step"] * 1e3 / head["launches_per_step"]
    roof = {"bound": "hbm", "achieved": round(head["gpu_GBps"], 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(head["gpu_GBps"] / HBM_PEAK_GBS, 4),
            "traffic": None, "kernel": f"paik::k_gemv<paik::{HEAD_NAME}, U, 1, false, NW>",
            "launches_per_step": head["launches_per_step"],
            "bytes_per_launch": round(head["bytes_per_step"] / head["launches_per_step"]),
            "avg_launch_us": round(avg_us, 3)}
    traffic_file = ROOT / "profiles" / f"traffic_gemv_{HEAD_NAME.lower()}_decode_step.txt"
    if traffic_file.exists():  # measured by two counter runs of this script (see the file)
        for ln in traffic_file.read_text().splitlines():
            if ln.startswith("traffic_bytes_per_launch:"):
                roof["traffic"] = int(ln.split(":", 1)[1])

    extra = {}
    if not args.no_extra:
        try:
            extra["q4_0_m1"] = gemv_config(pa, hm, pa.Q4_0, 2, 1, args.layers, 300, 20)
            log(f"Q4_0 M=1: {extra['q4_0_m1']['gpu_GBps']:.1f} GB/s GPU; "
                f"{extra['q4_0_m1']['per_launch']}")
            extra["q4_0_m1_separate"] = gemv_config(pa, hm, pa.Q4_0, 2, 1, args.layers, 300, 20,
                                                    plan=SEPARATE_STEP)
            log(f"Q4_0 M=1 separate: {extra['q4_0_m1_separate']['gpu_GBps']:.1f} GB/s GPU")
            extra["q4_0_m1_silu_fused"] = gemv_config(pa, hm, pa.Q4_0, 2, 1, args.layers, 300,
                                                      20, plan=SILU_STEP)
            log(f"Q4_0 M=1 with silu*mul fused: "
                f"{extra['q4_0_m1_silu_fused']['gpu_GBps']:.1f} GB/s GPU; "
                f"{extra['q4_0_m1_silu_fused']['per_launch']}")
            for m in (8, 32):
                extra[f"q4_k_m{m}"] = gemv_config(pa, hm, pa.Q4_K, 3, m, args.layers, 100, 5)
                log(f"Q4_K M={m}: {extra[f'q4_k_m{m}']['gpu_GBps']:.1f} GB/s GPU")
            extra["q8_0_4096x4096_m1"] = q8_config1(pa, hm, 300)
            extra["q4_k_m1_host_pointers"] = host_pointer_step(pa)
            log(f"{HEAD_NAME} M=1 host pointers: {extra['q4_k_m1_host_pointers']}")
            extra["prefill_m512"] = prefill(pa, hm, 20)
            log(f"prefill: {extra['prefill_m512']}")
            extra["decode_8b_ctx2048"] = decode_8b(pa, hm, 20, 5)
            log(f"decode 8B: {extra['decode_8b_ctx2048']}")
        except Exception as e:  # extras never hide the headline
            extra["error"] = repr(e)
    if args.calib_copy_mib:
        copy_calibration(hm, args.calib_copy_mib)
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(pa, args.cpu_budget)
            log(f"cpu baseline: {cpu['value']} GB/s ({cpu['kind']})")
        except Exception as e:
            cpu = {"error": repr(e)}

    line = {
        "metric": METRIC, "value": round(head["GBps"], 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{HEAD_NAME} GEMV M=1, Llama-3-8B projections q,k,v,o,gate,up,down "
                               "as one layer's decode step (q/k/v fused, o, gate/up fused, "
                               f"down: 4 launches), {args.layers} rotating layer copies",
                   "weights": f"{HEAD_NAME} (144 B / 256), f32 N(0,0.02^2) seeded, libpai_hip "
                              f"K-quant encoder",
                   "activations": "f32 N(0,1) resident in HBM",
                   "weight_set_MB": head["weight_set_MB"],
                   "frac_hbm_wall": round(head["GBps"] / HBM_PEAK_GBS, 4),
                   "per_launch": head.get("per_launch")},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
