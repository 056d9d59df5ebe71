"""Python handle on the native Qwen3 engine (include/cactus_engine.h)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._native import NativeError, engine

LAYER_FIELDS = ["input_norm", "q_w", "q_s", "k_w", "k_s", "v_w", "v_s", "o_w", "o_s", "q_norm",
                "k_norm", "post_norm", "gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s"]


class QwenConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("num_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim", "vocab", "group_size")] + \
               [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
                ("max_seq", ctypes.c_uint32), ("prefill_chunk", ctypes.c_uint32)]


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in LAYER_FIELDS]


class Timing(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_double), ("first_decode_ms", ctypes.c_double),
                ("decode_ms", ctypes.c_double), ("prefill_tokens", ctypes.c_uint32),
                ("decode_tokens", ctypes.c_uint32)]


def qwen3_0p6b(max_seq: int = 4352) -> dict:
    """Qwen3-0.6B architecture (engine/engine.h:43-59), group-32 weights."""
    return dict(num_layers=28, hidden=1024, ffn=3072, heads=16, kv_heads=8, head_dim=128,
                vocab=151936, group_size=32, eps=1e-6, rope_theta=1e6, max_seq=max_seq,
                prefill_chunk=256)


def layer_shapes(c: dict) -> dict:
    H, F, hd, gs = c["hidden"], c["ffn"], c["head_dim"], c["group_size"]
    nq, nkv = c["heads"] * hd, c["kv_heads"] * hd
    return {
        "input_norm": ((H,), np.uint16), "post_norm": ((H,), np.uint16),
        "q_norm": ((hd,), np.uint16), "k_norm": ((hd,), np.uint16),
        "q_w": ((nq, H), np.int8), "q_s": ((nq, H // gs), np.uint16),
        "k_w": ((nkv, H), np.int8), "k_s": ((nkv, H // gs), np.uint16),
        "v_w": ((nkv, H), np.int8), "v_s": ((nkv, H // gs), np.uint16),
        "o_w": ((H, nq), np.int8), "o_s": ((H, nq // gs), np.uint16),
        "gate_w": ((F, H // 2), np.uint8), "gate_s": ((F, H // gs), np.uint16),
        "up_w": ((F, H // 2), np.uint8), "up_s": ((F, H // gs), np.uint16),
        "down_w": ((H, F // 2), np.uint8), "down_s": ((H, F // gs), np.uint16),
    }


def random_weights(cfg: dict, seed: int):
    """The host weights Qwen(cfg, seed=seed) uploads (cactus_qwen_random_weights;
    no device call): (layers, embedding, output_norm) as numpy arrays."""
    lib = engine()
    c = QwenConfig(**cfg)
    shapes = layer_shapes(cfg)
    layers = [{k: np.zeros(s, t) for k, (s, t) in shapes.items()} for _ in range(cfg["num_layers"])]
    arr = (LayerWeights * cfg["num_layers"])()
    for i, L in enumerate(layers):
        for k in LAYER_FIELDS:
            setattr(arr[i], k, L[k].ctypes.data)
    emb = np.zeros((cfg["vocab"], cfg["hidden"]), np.uint16)
    on = np.zeros(cfg["hidden"], np.uint16)
    rc = lib.cactus_qwen_random_weights(ctypes.byref(c), ctypes.c_uint64(seed), arr, emb.ctypes.data,
                                        on.ctypes.data)
    if rc != 0:
        raise NativeError(rc, lib.cactus_engine_last_error().decode(errors="replace"))
    return layers, emb, on


class Qwen:
    """Qwen3-architecture model on the GPU (mirrors Model init/prefill/decode)."""

    def __init__(self, cfg: dict, layers: list[dict] | None = None, embedding=None,
                 output_norm=None, seed: int | None = None):
        self.lib = engine()
        self.cfg = dict(cfg)
        self.c = QwenConfig(**self.cfg)
        h = ctypes.c_void_p()
        if layers is None:
            self._check(self.lib.cactus_qwen_create_random(ctypes.byref(self.c), seed or 0, ctypes.byref(h)))
        else:
            self._keep = [{k: np.ascontiguousarray(v) for k, v in L.items()} for L in layers]
            arr = (LayerWeights * len(layers))()
            for i, L in enumerate(self._keep):
                for k in LAYER_FIELDS:
                    setattr(arr[i], k, L[k].ctypes.data)
            emb = np.ascontiguousarray(embedding)
            on = np.ascontiguousarray(output_norm)
            self._check(self.lib.cactus_qwen_create(ctypes.byref(self.c), arr, emb.ctypes.data, on.ctypes.data,
                                                    ctypes.byref(h)))
        self.h = h.value

    @classmethod
    def from_folder(cls, folder, context_size: int) -> "Qwen":
        """Model::init(model_folder, context_size) over a folder of CACT
        tensor files and config.txt (cactus_qwen_create_from_folder)."""
        self = cls.__new__(cls)
        self.lib = engine()
        self.h = None
        c = QwenConfig()
        path = str(folder).encode()
        self._check(self.lib.cactus_qwen_read_config(path, ctypes.byref(c)))
        c.max_seq = context_size
        h = ctypes.c_void_p()
        self._check(self.lib.cactus_qwen_create_from_folder(path, context_size, ctypes.byref(h)))
        self.c = c
        self.cfg = {name: getattr(c, name) for name, _ in QwenConfig._fields_}
        self.h = h.value
        return self

    def _check(self, rc):
        if rc != 0:
            raise NativeError(rc, self.lib.cactus_engine_last_error().decode(errors="replace"))

    def set_decode_mode(self, mode: int):
        self._check(self.lib.cactus_qwen_set_decode_mode(self.h, mode))

    def set_attention_mode(self, mode: int):
        """0: exact attention (bit-identical); 1: tolerance mode for every
        attention node -- split-K kernels for decode steps and FP16-MFMA
        flash attention for prefill chunks, each within 1e-3 + 1e-2 |ref| of
        the reference per output (the softmax where the reference's block
        rescale overflows); greedy tokens may then differ from the
        reference's."""
        self._check(self.lib.cactus_qwen_set_attention_mode(self.h, mode))

    def reset(self):
        self._check(self.lib.cactus_qwen_reset(self.h))

    def set_kv_window(self, window: int, sink: int):
        """KVCache::set_window_size: keep the first `sink` and the latest
        window - sink tokens (0 = no window)."""
        self._check(self.lib.cactus_qwen_set_kv_window(self.h, window, sink))

    def set_sampling(self, temperature: float, top_p: float, top_k: int, seed: int = 0):
        """Model::decode's temperature / top_p / top_k; all zero = greedy."""
        self._check(self.lib.cactus_qwen_set_sampling(self.h, ctypes.c_float(temperature), ctypes.c_float(top_p),
                                                      top_k, seed))

    def total_len(self) -> int:
        n = ctypes.c_size_t()
        self._check(self.lib.cactus_qwen_total_len(self.h, ctypes.byref(n)))
        return n.value

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self._check(self.lib.cactus_qwen_prefill(self.h, t.ctypes.data, t.size))

    def decode(self, token: int) -> int:
        out = ctypes.c_uint32()
        self._check(self.lib.cactus_qwen_decode(self.h, int(token), ctypes.byref(out)))
        return out.value

    def generate(self, prompt, max_new: int):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max_new, np.uint32)
        t = Timing()
        self._check(self.lib.cactus_qwen_generate(self.h, p.ctypes.data, p.size, max_new, out.ctypes.data,
                                                  ctypes.byref(t)))
        return out, t

    def last_hidden(self) -> np.ndarray:
        rows = ctypes.c_size_t()
        H = self.cfg["hidden"]
        buf = np.zeros((8192, H), np.uint16)
        self._check(self.lib.cactus_qwen_last_hidden(self.h, buf.ctypes.data, buf.shape[0], ctypes.byref(rows)))
        return buf[:rows.value].copy()

    def last_logits(self) -> np.ndarray:
        out = np.zeros(self.cfg["vocab"], np.uint16)
        self._check(self.lib.cactus_qwen_last_logits(self.h, out.ctypes.data))
        return out

    def last_entropy(self) -> float:
        e = ctypes.c_float()
        self._check(self.lib.cactus_qwen_last_entropy(self.h, ctypes.byref(e)))
        return e.value

    def cache_len(self) -> int:
        n = ctypes.c_size_t()
        self._check(self.lib.cactus_qwen_cache_len(self.h, ctypes.byref(n)))
        return n.value

    def read_kv(self, layer: int):
        n = self.cache_len()
        kvh, hd = self.cfg["kv_heads"], self.cfg["head_dim"]
        ng = (hd + 127) // 128
        k = np.zeros((n, kvh, hd), np.int8)
        v = np.zeros_like(k)
        ks = np.zeros((n, kvh, ng), np.float32)
        vs = np.zeros_like(ks)
        self._check(self.lib.cactus_qwen_read_kv(self.h, layer, k.ctypes.data, v.ctypes.data, ks.ctypes.data,
                                                 vs.ctypes.data))
        return k, v, ks, vs

    def read_weights(self):
        shapes = layer_shapes(self.cfg)
        L = self.cfg["num_layers"]
        layers = [{k: np.zeros(s, t) for k, (s, t) in shapes.items()} for _ in range(L)]
        arr = (LayerWeights * L)()
        for i in range(L):
            for k in LAYER_FIELDS:
                setattr(arr[i], k, layers[i][k].ctypes.data)
        emb = np.zeros((self.cfg["vocab"], self.cfg["hidden"]), np.uint16)
        on = np.zeros(self.cfg["hidden"], np.uint16)
        self._check(self.lib.cactus_qwen_read_weights(self.h, arr, emb.ctypes.data, on.ctypes.data))
        return layers, emb, on

    def close(self):
        if getattr(self, "h", None):
            self.lib.cactus_qwen_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
