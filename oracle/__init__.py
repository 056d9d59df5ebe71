"""ctypes binding of the CPU restatement (oracle/_build/libcactus_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libcactus_oracle.so"

_lib = None

P = ctypes.c_void_p
SZ = ctypes.c_size_t
F = ctypes.c_float
I = ctypes.c_int

_SIGS = {
    "orc_h2f": (F, [ctypes.c_uint16]),
    "orc_f2h": (ctypes.c_uint16, [F]),
    "orc_d2h": (ctypes.c_uint16, [ctypes.c_double]),
    "orc_hadd": (ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16]),
    "orc_hmul": (ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint16]),
    "orc_hfma": (ctypes.c_uint16, [ctypes.c_uint16] * 3),
    "orc_expf": (F, [F]),
    "orc_fast_exp": (F, [F]),
    "orc_poly_exp_weight": (F, [F, F]),
    "orc_fp16_max_abs": (F, [P, SZ]),
    "orc_fp16_to_int8": (None, [P, P, SZ, F]),
    "orc_quantize_activations": (None, [P, P, P, SZ, SZ]),
    "orc_matmul_int8": (None, [P, P, P, P, P, SZ, SZ, SZ, SZ]),
    "orc_matmul_int4": (None, [P, P, P, P, P, SZ, SZ, SZ, SZ]),
    "orc_group_sums_int8": (None, [P, P, P, SZ, SZ, SZ, SZ]),
    "orc_unpack_int4_to_int8": (None, [P, P, SZ]),
    "orc_matmul_int8_mt": (None, [P, P, P, P, P, SZ, SZ, SZ, SZ, I]),
    "orc_set_threads": (None, [I]),
    "orc_matmul_f16": (None, [P, P, P, SZ, SZ, SZ]),
    "orc_attention_f16": (None, [P, P, P, P, SZ, SZ, SZ, SZ, SZ, SZ, F, P, SZ, SZ, I]),
    "orc_attention_hybrid_int8_fp16": (None, [P, P, P, P, P, P, P, P, SZ, SZ, SZ, SZ, SZ, SZ,
                                              SZ, F, SZ, I, SZ]),
    "orc_quantize_kv_fp16_to_int8": (None, [P, P, P, SZ, SZ, SZ, SZ]),
    "orc_rms_norm_f16": (None, [P, P, P, SZ, SZ, F]),
    "orc_rope_tables": (None, [P, P, SZ, SZ, F]),
    "orc_rope_f16": (None, [P, P, SZ, SZ, SZ, SZ, SZ, F]),
    "orc_softmax_f16": (None, [P, P, SZ, SZ]),
    "orc_silu_f16": (None, [P, P, SZ]),
    "orc_add_f16": (None, [P, P, P, SZ]),
    "orc_multiply_f16": (None, [P, P, P, SZ]),
    "orc_embedding_f16": (I, [P, P, P, SZ, SZ, SZ]),
    "orc_argmax_f16": (ctypes.c_uint32, [P, SZ]),
    "orc_qwen_create": (P, [P, P, P, P]),
    "orc_qwen_destroy": (None, [P]),
    "orc_qwen_reset": (None, [P]),
    "orc_qwen_prefill": (I, [P, P, SZ, SZ]),
    "orc_qwen_decode": (ctypes.c_uint32, [P, ctypes.c_uint32, P]),
    "orc_qwen_last_hidden": (P, [P, P]),
    "orc_qwen_cache_len": (SZ, [P]),
    "orc_qwen_kv": (None, [P, SZ, P, P, P, P]),
    "orc_qwen_set_window": (I, [P, SZ, SZ]),
    "orc_mt19937_nth": (ctypes.c_uint32, [ctypes.c_uint32, SZ]),
    "orc_sample_uniform": (F, [ctypes.c_uint32]),
    "orc_logits_entropy_f16": (F, [P, SZ]),
    "orc_sample_f16": (ctypes.c_uint32, [P, SZ, F, F, SZ, F, P, P]),
    "orc_sample_f32": (ctypes.c_uint32, [P, SZ, F, F, SZ, P, P, SZ, F]),
    "orc_fast_tanh": (F, [F]),
    "orc_gelu_f16": (None, [P, P, SZ]),
    "orc_gelu_erf_f16": (None, [P, P, SZ]),
    "orc_layer_norm_f16": (None, [P, P, P, P, SZ, SZ, F]),
    "orc_conv1d_causal_depthwise_f16": (None, [P, P, P, SZ, SZ, SZ, SZ, SZ]),
    "orc_conv1d_f16_k3": (None, [P, P, P, SZ, SZ, SZ, SZ, SZ]),
    "orc_kv_create": (P, [SZ, SZ, SZ, SZ]),
    "orc_kv_destroy": (None, [P]),
    "orc_kv_set_window": (I, [P, SZ, SZ]),
    "orc_kv_reset": (None, [P]),
    "orc_kv_update": (I, [P, P, P, SZ]),
    "orc_kv_len": (SZ, [P]),
    "orc_kv_total": (SZ, [P]),
    "orc_kv_layer": (None, [P, SZ, P, P, P, P]),
}


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- numpy conveniences (fp16 arrays travel as uint16 bit patterns) ----------
def f16bits(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float16)).view(np.uint16)


def bits2f(u: np.ndarray) -> np.ndarray:
    return np.asarray(u, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_activations(x16: np.ndarray):
    M, K = x16.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib().orc_quantize_activations(ptr(x16), ptr(q), ptr(s), M, K)
    return q, s


def matmul_int8(A, As, B, Bs, gs):
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), np.uint16)
    lib().orc_matmul_int8(ptr(A), ptr(As), ptr(B), ptr(Bs), ptr(C), M, K, N, gs)
    return C


def matmul_int4(A, As, Bp, Bs, gs):
    M, K = A.shape
    N = Bp.shape[0]
    C = np.empty((M, N), np.uint16)
    lib().orc_matmul_int4(ptr(A), ptr(As), ptr(Bp), ptr(Bs), ptr(C), M, K, N, gs)
    return C


def group_sums_int8(A, B, gs):
    M, K = A.shape
    N = B.shape[0]
    acc = np.empty((M, N, K // gs), np.int32)
    lib().orc_group_sums_int8(ptr(A), ptr(B), ptr(acc), M, K, N, gs)
    return acc


def matmul_f16(a, bT):
    M, K = a.shape
    N = bT.shape[0]
    c = np.empty((M, N), np.uint16)
    lib().orc_matmul_f16(ptr(a), ptr(bT), ptr(c), M, K, N)
    return c


def attention_f16(q, k, v, scale, mask=None, pos_off=0, window=0, causal=True):
    B, S, Hq, d = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    o = np.empty_like(q)
    lib().orc_attention_f16(ptr(q), ptr(k), ptr(v), ptr(o), B, S, Skv, Hq, Hkv, d, scale,
                            ptr(mask), pos_off, window, 1 if causal else 0)
    return o


def attention_hybrid(q, kc, vc, ks, vs, kn, vn, scale, pos_off, causal=True, qgs=128):
    B, S, Hq, d = q.shape
    cache_len = kc.shape[1] if kc is not None else 0
    new_len = kn.shape[1] if kn is not None else 0
    Hkv = (kc if kc is not None else kn).shape[2]
    o = np.empty_like(q)
    lib().orc_attention_hybrid_int8_fp16(ptr(q), ptr(kc), ptr(vc), ptr(ks), ptr(vs), ptr(kn),
                                         ptr(vn), ptr(o), B, S, cache_len, new_len, Hq, Hkv, d,
                                         scale, pos_off, 1 if causal else 0, qgs)
    return o


def quantize_kv(src, gs=128):
    S, H, d = src.shape
    ng = (d + gs - 1) // gs
    dst = np.empty((S, H, d), np.int8)
    sc = np.empty((S, H, ng), np.float32)
    lib().orc_quantize_kv_fp16_to_int8(ptr(src), ptr(dst), ptr(sc), S, H, d, gs)
    return dst, sc


def rms_norm(x, w, eps):
    rows, dims = x.shape
    y = np.empty_like(x)
    lib().orc_rms_norm_f16(ptr(x), ptr(w), ptr(y), rows, dims, eps)
    return y


def rope(x, start_pos, theta):
    B, S, H, d = x.shape
    y = np.empty_like(x)
    lib().orc_rope_f16(ptr(x), ptr(y), B, S, H, d, start_pos, theta)
    return y


def softmax(x):
    rows, V = x.shape
    y = np.empty_like(x)
    lib().orc_softmax_f16(ptr(x), ptr(y), rows, V)
    return y


def silu(x):
    y = np.empty_like(x)
    lib().orc_silu_f16(ptr(x), ptr(y), x.size)
    return y


def add(a, b):
    y = np.empty_like(a)
    lib().orc_add_f16(ptr(a), ptr(b), ptr(y), a.size)
    return y


def multiply(a, b):
    y = np.empty_like(a)
    lib().orc_multiply_f16(ptr(a), ptr(b), ptr(y), a.size)
    return y


def argmax(logits):
    return int(lib().orc_argmax_f16(ptr(logits), logits.size))


# ---- Qwen3 forward restatement ---------------------------------------------
QWEN_LAYER_FIELDS = ["input_norm", "q_w", "q_s", "k_w", "k_s", "v_w", "v_s", "o_w", "o_s", "q_norm",
                     "k_norm", "post_norm", "gate_w", "gate_s", "up_w", "up_s", "down_w", "down_s"]


class _Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("num_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim", "vocab", "group_size")] + \
               [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("max_seq", ctypes.c_uint32)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in QWEN_LAYER_FIELDS]


def fast_tanh(x: float) -> float:
    return float(lib().orc_fast_tanh(x))


def gelu(x16):
    y = np.empty_like(x16)
    lib().orc_gelu_f16(ptr(x16), ptr(y), x16.size)
    return y


def gelu_erf(x16):
    y = np.empty_like(x16)
    lib().orc_gelu_erf_f16(ptr(x16), ptr(y), x16.size)
    return y


def layer_norm(x16, w16, b16, eps):
    rows, F = x16.shape
    y = np.empty_like(x16)
    lib().orc_layer_norm_f16(ptr(x16), ptr(w16), ptr(b16), ptr(y), rows, F, eps)
    return y


def conv1d_causal_depthwise(x16, w16, dilation):
    """x [N][L][C], w [C][K] -> y [N][L][C]"""
    N, L, C = x16.shape
    K = w16.shape[1]
    y = np.empty_like(x16)
    lib().orc_conv1d_causal_depthwise_f16(ptr(x16), ptr(w16), ptr(y), N, L, C, K, dilation)
    return y


def conv1d_k3(x16, w16, stride):
    """x [N][C_in][L], w [C_out][C_in][3] -> y [N][C_out][(L-1)/stride + 1]"""
    N, Cin, L = x16.shape
    Cout = w16.shape[0]
    y = np.empty((N, Cout, (L - 1) // stride + 1), np.uint16)
    lib().orc_conv1d_f16_k3(ptr(x16), ptr(w16), ptr(y), N, L, Cin, Cout, stride)
    return y


def mt19937_nth(seed: int, n: int) -> int:
    return int(lib().orc_mt19937_nth(seed, n))


def logits_entropy(logits) -> float:
    x = np.ascontiguousarray(logits, dtype=np.uint16)
    return float(lib().orc_logits_entropy_f16(x.ctypes.data, x.size))


def sample_uniform(seed: int) -> float:
    return float(lib().orc_sample_uniform(seed))


def sample_f32(logits, temperature, top_p, top_k, seed, bias=None):
    """cactus_sample_f32 with the draw of mt19937(seed); bias: {token: value}
    or a list of (token, value) pairs applied in order."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    pairs = list(bias.items()) if isinstance(bias, dict) else list(bias or [])
    bi = np.array([t for t, _ in pairs], np.uint32)
    bv = np.array([v for _, v in pairs], np.float32)
    return int(lib().orc_sample_f32(x.ctypes.data, x.size, temperature, top_p, top_k,
                                    bv.ctypes.data if pairs else None, bi.ctypes.data if pairs else None,
                                    len(pairs), sample_uniform(seed)))


class OracleSampler:
    """cactus_sample_f16 with its process-wide token history held here."""

    def __init__(self):
        self.hist = np.zeros(128, np.uint32)
        self.n = ctypes.c_size_t(0)

    def history(self):
        return self.hist[:self.n.value].copy()

    def sample(self, logits, temperature, top_p, top_k, seed):
        x = np.ascontiguousarray(logits, dtype=np.uint16)
        u = sample_uniform(seed)
        return int(lib().orc_sample_f16(x.ctypes.data, x.size, temperature, top_p, top_k, u,
                                        self.hist.ctypes.data, ctypes.byref(self.n)))


def _kv_arrays(ptrs, n, kvh, hd, ng):
    def arr(p, dt, shape):
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(dt)), (int(np.prod(shape)),)).reshape(
            shape).copy()
    return (arr(ptrs[0], ctypes.c_int8, (n, kvh, hd)), arr(ptrs[1], ctypes.c_int8, (n, kvh, hd)),
            arr(ptrs[2], ctypes.c_float, (n, kvh, ng)), arr(ptrs[3], ctypes.c_float, (n, kvh, ng)))


class OracleKV:
    """orc_kv_* (kv_oracle.c): the engine's INT8 KV cache with sliding window
    and sinks (engine_cache.cpp)."""

    def __init__(self, layers, max_seq, kv_heads, head_dim):
        self.layers, self.kvh, self.hd = layers, kv_heads, head_dim
        self.h = lib().orc_kv_create(layers, max_seq, kv_heads, head_dim)

    def set_window(self, window, sink):
        assert lib().orc_kv_set_window(self.h, window, sink) == 0

    def reset(self):
        lib().orc_kv_reset(self.h)

    def update(self, k_layers, v_layers) -> int:
        """k_layers / v_layers: per layer fp16 bits [seq][kv_heads][head_dim]."""
        ks = [np.ascontiguousarray(k, dtype=np.uint16) for k in k_layers]
        vs = [np.ascontiguousarray(v, dtype=np.uint16) for v in v_layers]
        kp = (ctypes.c_void_p * self.layers)(*[k.ctypes.data for k in ks])
        vp = (ctypes.c_void_p * self.layers)(*[v.ctypes.data for v in vs])
        return int(lib().orc_kv_update(self.h, kp, vp, ks[0].shape[0]))

    def len(self):
        return int(lib().orc_kv_len(self.h))

    def total(self):
        return int(lib().orc_kv_total(self.h))

    def layer(self, l, n=None):
        """(codes k, codes v, scales k, scales v) of the first n tokens (default: len)."""
        n = self.len() if n is None else n
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        lib().orc_kv_layer(self.h, l, *[ctypes.byref(p) for p in ptrs])
        return _kv_arrays(ptrs, n, self.kvh, self.hd, (self.hd + 127) // 128)

    def close(self):
        if self.h:
            lib().orc_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class OracleQwen:
    """orc_qwen_* (qwen_oracle.c): the reference's Qwen3 block and engine flow."""

    def __init__(self, cfg: dict, layers, embedding, output_norm):
        L = lib()
        self.cfg = cfg
        c = _Cfg(**{k: cfg[k] for k in ("num_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim",
                                        "vocab", "group_size", "eps", "rope_theta", "max_seq")})
        self._keep = [{k: np.ascontiguousarray(v) for k, v in Lw.items()} for Lw in layers]
        self._emb = np.ascontiguousarray(embedding)
        self._on = np.ascontiguousarray(output_norm)
        arr = (_Layer * len(layers))()
        for i, Lw in enumerate(self._keep):
            for k in QWEN_LAYER_FIELDS:
                setattr(arr[i], k, Lw[k].ctypes.data)
        self.h = L.orc_qwen_create(ctypes.byref(c), arr, self._emb.ctypes.data, self._on.ctypes.data)

    def reset(self):
        lib().orc_qwen_reset(self.h)

    def set_window(self, window: int, sink: int):
        assert lib().orc_qwen_set_window(self.h, window, sink) == 0

    def prefill(self, tokens, chunk=256):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        rc = lib().orc_qwen_prefill(self.h, t.ctypes.data, t.size, chunk)
        assert rc == 0

    def decode(self, token, logits=None):
        return int(lib().orc_qwen_decode(self.h, int(token), None if logits is None else logits.ctypes.data))

    def generate(self, prompt, max_new, chunk=256):
        """The FFI order: prefill prompt[:-1], then decode from prompt[-1]."""
        if len(prompt) > 1:
            self.prefill(prompt[:-1], chunk)
        out, tok = [], int(prompt[-1])
        for _ in range(max_new):
            tok = self.decode(tok)
            out.append(tok)
        return np.array(out, np.uint32)

    def last_hidden(self):
        rows = ctypes.c_size_t()
        p = lib().orc_qwen_last_hidden(self.h, ctypes.byref(rows))
        n = rows.value * self.cfg["hidden"]
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint16)), (n,)).reshape(
            rows.value, self.cfg["hidden"]).copy()

    def cache_len(self):
        return int(lib().orc_qwen_cache_len(self.h))

    def read_kv(self, layer):
        n = self.cache_len()
        kvh, hd = self.cfg["kv_heads"], self.cfg["head_dim"]
        ng = (hd + 127) // 128
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        lib().orc_qwen_kv(self.h, layer, *[ctypes.byref(p) for p in ptrs])
        return _kv_arrays(ptrs, n, kvh, hd, ng)

    def close(self):
        if self.h:
            lib().orc_qwen_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
