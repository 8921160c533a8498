"""Python view of include/pai_llama.h: the decode-step operators and the
device-resident LLaMA model (pai_llama_t), for tests and benchmarks.

The reference generates in sequence mode, re-running the whole graph per
token (models/model.c:453-507); pai_llama_decode computes one new position
against an fp16 KV cache. Every kernel runs through libpai_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import check, lib
from .qmat import Q4_K, Q6_K, QMat, normal_f32, quantize


class LlamaConfig(C.Structure):
    """pai_llama_config_t."""
    _fields_ = [(n, C.c_uint32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "n_ff",
                                          "vocab", "ctx", "n_rot")] + [
        ("rope_theta", C.c_float), ("norm_eps", C.c_float)]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class Llama:
    """A pai_llama_t: borrowed QMat weights (kept alive here), fp16 KV cache."""

    def __init__(self, cfg: LlamaConfig):
        self.cfg = cfg
        self.hd = cfg.n_embd // cfg.n_head
        self._h = C.c_void_p()
        self._keep = []
        check(lib().pai_llama_create(C.byref(self._h), C.byref(cfg)), "pai_llama_create")

    @property
    def handle(self) -> int:
        return self._h.value

    def set_layer(self, layer: int, w: dict, attn_norm: np.ndarray, ffn_norm: np.ndarray) -> None:
        """w: QMats q, k, v, o, gate, up, down."""
        an = np.ascontiguousarray(attn_norm, np.float32)
        fn = np.ascontiguousarray(ffn_norm, np.float32)
        mats = [w[n] for n in ("q", "k", "v", "o", "gate", "up", "down")]
        self._keep.extend(mats)
        check(lib().pai_llama_set_layer(self._h, layer, *[m.handle for m in mats], an.ctypes.data,
                                        fn.ctypes.data), "pai_llama_set_layer")

    def set_output(self, token_embd: QMat, output: QMat, output_norm: np.ndarray) -> None:
        on = np.ascontiguousarray(output_norm, np.float32)
        self._keep.extend([token_embd, output])
        check(lib().pai_llama_set_output(self._h, token_embd.handle, output.handle,
                                         on.ctypes.data), "pai_llama_set_output")

    def kv_write(self, layer: int, pos0: int, k16: np.ndarray, v16: np.ndarray) -> None:
        """k16, v16: fp16 [npos][n_head_kv][hd]."""
        k = np.ascontiguousarray(k16, np.float16)
        v = np.ascontiguousarray(v16, np.float16)
        check(lib().pai_llama_kv_write(self._h, layer, pos0, k.shape[0], k.ctypes.data,
                                       v.ctypes.data), "pai_llama_kv_write")

    def decode(self, token: int, pos: int, want_logits: bool = True):
        nxt = C.c_uint32()
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        check(lib().pai_llama_decode(self._h, token, pos, C.byref(nxt),
                                     logits.ctypes.data if want_logits else None),
              "pai_llama_decode")
        return nxt.value, logits

    def decode_async(self, token_ptr: int, pos: int, next_ptr: int, stream: int = 0) -> None:
        check(lib().pai_llama_decode_async(self._h, token_ptr, pos, next_ptr, stream or None),
              "pai_llama_decode_async")

    def logits_ptr(self) -> int:
        return lib().pai_llama_logits(self._h)

    def kv_cache(self, layer: int):
        k, v = C.c_void_p(), C.c_void_p()
        check(lib().pai_llama_kv_cache(self._h, layer, C.byref(k), C.byref(v)),
              "pai_llama_kv_cache")
        return k.value, v.value

    def free(self) -> None:
        if self._h.value:
            lib().pai_llama_free(self._h)
            self._h = C.c_void_p()
        self._keep = []

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class SyntheticWeights:
    """Native GGUF blocks of a random-init model (host), and their types."""
    layers: list   # per layer: {name: (qtype, blocks [N][row_bytes])} + norms
    head: dict     # token_embd, output: (qtype, blocks); output_norm


def synthetic_weights(cfg: LlamaConfig, seed: int, types: dict | None = None,
                      norms_one: bool = False, threads: int = 0) -> SyntheticWeights:
    """Weights drawn N(0, 0.02^2) from `seed` and quantized by the build's
    encoders: Q4_K everywhere except Q6_K for ffn_down and the output head
    (override per name with `types`). Norm weights are 1 when norms_one,
    otherwise drawn N(1, 0.1^2)."""
    t = {"q": Q4_K, "k": Q4_K, "v": Q4_K, "o": Q4_K, "gate": Q4_K, "up": Q4_K, "down": Q6_K,
         "token_embd": Q4_K, "output": Q6_K}
    t.update(types or {})
    E, F, KV = cfg.n_embd, cfg.n_ff, cfg.n_head_kv * (cfg.n_embd // cfg.n_head)
    shapes = {"q": (E, E), "k": (KV, E), "v": (KV, E), "o": (E, E), "gate": (F, E),
              "up": (F, E), "down": (E, F)}
    s = seed

    def draw(name, n, k):
        nonlocal s
        s += 1
        w = normal_f32(s, n * k, 0.0, 0.02).reshape(n, k)
        return t[name], quantize(t[name], w, threads)

    def norm(sd, n):
        if norms_one:
            return np.ones(n, np.float32)
        return normal_f32(sd, n, 1.0, 0.1)

    layers = []
    for L in range(cfg.n_layer):
        d = {}
        for name, (n, k) in shapes.items():
            d[name] = draw(name, n, k)
        s += 1
        d["attn_norm"] = norm(s, E)
        s += 1
        d["ffn_norm"] = norm(s, E)
        layers.append(d)
    head = {}
    for name in ("token_embd", "output"):
        head[name] = draw(name, cfg.vocab, E)
    s += 1
    head["output_norm"] = norm(s, E)
    return SyntheticWeights(layers, head)


def upload(cfg: LlamaConfig, w: SyntheticWeights) -> Llama:
    """A Llama holding device copies of the synthetic weights."""
    m = Llama(cfg)
    E, F, KV = cfg.n_embd, cfg.n_ff, cfg.n_head_kv * (cfg.n_embd // cfg.n_head)
    shapes = {"q": (E, E), "k": (KV, E), "v": (KV, E), "o": (E, E), "gate": (F, E),
              "up": (F, E), "down": (E, F)}
    for L, d in enumerate(w.layers):
        mats = {n: QMat(d[n][0], *shapes[n], d[n][1]) for n in shapes}
        m.set_layer(L, mats, d["attn_norm"], d["ffn_norm"])
    te, out = w.head["token_embd"], w.head["output"]
    m.set_output(QMat(te[0], cfg.vocab, E, te[1]), QMat(out[0], cfg.vocab, E, out[1]),
                 w.head["output_norm"])
    return m
