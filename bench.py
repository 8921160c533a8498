#!/usr/bin/env python3
"""Quantized-weights GEMV/GEMM benchmark on one MI355X.

Headline (the JSON `value`): Q4_0 decode GEMV, M=1, over the seven
Llama-3-8B per-layer projections (q, o: 4096x4096; k, v: 1024x4096;
gate, up: 14336x4096; down: 4096x14336). One step = the seven projections
of one layer on one activation vector; steps rotate over --layers distinct
weight copies so the working set (123 MB per layer) exceeds the 256 MB
Infinity Cache. Weights are f32 N(0, 0.02^2) from a fixed seed, quantized
by libpai_hip's encoder; activations are f32 N(0, 1), resident in HBM.

value    = algorithmic bytes (packed W + x + y, f32) of all timed steps
           / wall time between two device synchronisations.
roofline = the GEMV kernel: the same bytes / the sum of its launch
           durations (HIP events around every launch, on the launch stream),
           against 8 TB/s.
cpu_baseline = the reference's AVX2+FMA GEMV (cpu/optimized/opt_ops.c,
           compiled from its sources into oracle/_ref; this repository's
           restatement when that build is absent) on the dequantized f32
           weights of the same seven projections, one host core.
extra    = the other configurations: Q8_0 4096x4096 GEMV, Q4_K GEMV at
           M in {1, 8, 32}, and the M=512 prefill GEMMs (gate Q4_K,
           down Q6_K) in TFLOP/s against 2.5 PFLOP/s dense fp16.
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


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def seed_w(config: int, idx: int) -> int:
    return 0xC0DE0000 + 16 * config + idx


def call_bytes(pa, qtype: int, n: int, k: int, m: int = 1) -> int:
    return n * pa.qtype_bytes(qtype, k) + m * (k + n) * 4


class Layer:
    """One layer's seven packed projections on the device."""

    def __init__(self, pa, qtype: int, blocks: list):
        self.w = [pa.QMat(qtype, n, k, b) for (_, n, k), b in zip(PROJ, blocks)]


def quantized_layer(pa, qtype: int, config: int) -> list:
    out = []
    for i, (_, n, k) in enumerate(PROJ):
        w = pa.normal_f32(seed_w(config, i), n * k, 0.0, 0.02).reshape(n, k)
        out.append(pa.quantize(qtype, w))
    return out


def run_layers(pa, hm, layers, m: int, steps: int, warmup: int, per_launch_events: bool):
    """Time `steps` passes over the seven projections, rotating layers.
    Every launch goes to one HIP stream; the per-launch events are recorded
    on that stream."""
    stream = hm.Stream()
    sh = stream.handle
    kmax = max(k for _, _, k in PROJ)
    x = hm.DeviceBuffer.from_array(pa.normal_f32(0xC0DE0000 ^ 0x5A5A, m * kmax))
    ys = [hm.DeviceBuffer(m * n * 4) for _, n, _ in PROJ]
    xp, yp = x.ptr, [y.ptr for y in ys]

    def step(s, evs=None):
        layer = layers[s % len(layers)]
        for j, w in enumerate(layer.w):
            if evs is not None:
                evs[2 * j].record(stream)
            w.gemm_async(xp, yp[j], m, 0, sh)
            if evs is not None:
                evs[2 * j + 1].record(stream)

    for s in range(warmup):
        step(s)
    evs = None
    if per_launch_events:
        evs = [[hm.Event() for _ in range(2 * len(PROJ))] for _ in range(steps)]
    stream.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        step(s, evs[s] if evs else None)
    stream.synchronize()
    wall = time.perf_counter() - t0
    per_proj_ms = None
    if evs:
        per_proj_ms = np.zeros(len(PROJ))
        for e in evs:
            for j in range(len(PROJ)):
                per_proj_ms[j] += e[2 * j].elapsed_ms(e[2 * j + 1])
        per_proj_ms /= steps
        for e in evs:
            for ev in e:
                ev.destroy()
    for b in [x, *ys]:
        b.free()
    stream.destroy()
    return wall, per_proj_ms


def gemv_config(pa, hm, qtype: int, config: int, m: int, nlayers: int, steps: int,
                warmup: int, per_launch_events: bool = True) -> dict:
    blocks = quantized_layer(pa, qtype, config)
    layers = [Layer(pa, qtype, blocks) for _ in range(nlayers)]
    wall, per_ms = run_layers(pa, hm, layers, m, steps, warmup, per_launch_events)
    bytes_step = sum(call_bytes(pa, qtype, n, k, m) for _, n, k in PROJ)
    res = {"qtype": qtype, "m": m, "layers": nlayers, "steps": steps,
           "weight_set_MB": round(nlayers * sum(l.nbytes for l in layers[0].w) / 1e6, 1),
           "bytes_per_step": bytes_step, "ms_per_step": wall / steps * 1e3,
           "GBps": bytes_step * steps / wall / 1e9}
    if per_ms is not None:
        kern_ms = float(per_ms.sum())
        res["kernel_GBps"] = bytes_step / (kern_ms * 1e-3) / 1e9
        res["per_projection"] = {
            name: {"us": round(float(t) * 1e3, 2),
                   "GBps": round(call_bytes(pa, qtype, n, k, m) / (t * 1e-3) / 1e9, 1)}
            for (name, n, k), t in zip(PROJ, per_ms)}
    for l in layers:
        for w in l.w:
            w.free()
    return res


def timed_calls(hm, call, reps: int, warm: int) -> float:
    """Mean microseconds per call of `call(stream_handle, i)` between two
    events on one stream."""
    st = hm.Stream()
    for i in range(warm):
        call(st.handle, i)
    a, b = hm.Event(), hm.Event()
    a.record(st)
    for i in range(reps):
        call(st.handle, i)
    b.record(st)
    b.synchronize()
    us = a.elapsed_ms(b) / reps * 1e3
    a.destroy(); b.destroy(); st.destroy()
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
    return out


def cpu_baseline(pa, budget_s: float) -> dict:
    """The reference's single-thread AVX2 GEMV on dequantized f32 weights of
    the seven Q4_0 projections (bounded number of passes)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_bind as ob
    r = ob.ref()
    kind = "reference" if r is not None else "port"
    blocks = quantized_layer(pa, pa.Q4_0, 2)
    mats = []
    for (_, n, k), b in zip(PROJ, blocks):
        if r is not None:
            mats.append(ob.ref_dequant(pa.Q4_0, b.tobytes(), n * k, row=k).reshape(n, k))
        else:
            mats.append(ob.dequant(pa.Q4_0, b, n * k).reshape(n, k))
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
    bytes_step = sum(call_bytes(pa, pa.Q4_0, n, k) for _, n, k in PROJ)
    med = float(np.median(times))
    return {"value": round(bytes_step / med / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{len(times)} passes over the seven Q4_0 projections of one layer "
                      f"(pai_opt_gemv_f32 on dequantized f32 [N][K], 4 B/weight touched); "
                      f"median {med * 1e3:.1f} ms/pass, min {min(times) * 1e3:.1f} ms; "
                      f"GB/s counts the same packed bytes as the GPU value",
            "host_cpu": _cpu_model(), "host_nproc": os.cpu_count()}


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
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the path has no multi-GPU sharding in this build)", file=sys.stderr)
        return 2

    import prosperoai_amd as pa
    from prosperoai_amd import hipmem as hm
    pa.init()
    log(f"Q4_0 M=1 x {args.layers} layers")

    head = gemv_config(pa, hm, pa.Q4_0, 2, 1, args.layers, args.steps, args.warmup)
    log(f"Q4_0 M=1: {head['GBps']:.1f} GB/s wall, {head.get('kernel_GBps', 0):.1f} GB/s kernels")
    roof = {"bound": "hbm", "achieved": round(head["kernel_GBps"], 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(head["kernel_GBps"] / HBM_PEAK_GBS, 4),
            "traffic": None, "kernel": "paik::k_gemv<Q4_0,1>",
            "bytes_per_launch": round(head["bytes_per_step"] / len(PROJ)),
            "avg_launch_us": round(head["bytes_per_step"] / len(PROJ)
                                   / (head["kernel_GBps"] * 1e9) * 1e6, 3)}
    traffic_file = ROOT / "profiles" / "traffic_gemv_q4_0.json"
    if traffic_file.exists():
        roof["traffic"] = json.loads(traffic_file.read_text()).get("bytes_per_launch")

    extra = {}
    if not args.no_extra:
        try:
            extra["q4_k_m1"] = gemv_config(pa, hm, pa.Q4_K, 3, 1, args.layers, 300, 20)
            log(f"Q4_K M=1: {extra['q4_k_m1']['kernel_GBps']:.1f} GB/s kernels")
            for m in (8, 32):
                extra[f"q4_k_m{m}"] = gemv_config(pa, hm, pa.Q4_K, 3, m, args.layers, 100, 5,
                                                  per_launch_events=False)
                log(f"Q4_K M={m}: {extra[f'q4_k_m{m}']['GBps']:.1f} GB/s")
            extra["q8_0_4096x4096_m1"] = q8_config1(pa, hm, 300)
            extra["prefill_m512"] = prefill(pa, hm, 20)
            log(f"prefill: {extra['prefill_m512']}")
        except Exception as e:  # extras never hide the headline
            extra["error"] = repr(e)
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
        "config": {"workload": "Q4_0 GEMV M=1, Llama-3-8B projections q,k,v,o,gate,up,down "
                               f"(one layer per step, {args.layers} rotating layer copies)",
                   "weights": "Q4_0 (18 B / 32), f32 N(0,0.02^2) seeded, libpai_hip encoder",
                   "activations": "f32 N(0,1) resident in HBM",
                   "weight_set_MB": head["weight_set_MB"],
                   "frac_hbm_wall": round(head["GBps"] / HBM_PEAK_GBS, 4),
                   "per_projection": head.get("per_projection")},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
