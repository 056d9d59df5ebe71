"""Seeded synthetic inputs shared by the parity tests, the smoke test and the
bench (shapes and distributions of the workloads the kernels are quoted on)."""
from __future__ import annotations

import numpy as np


def f16(x) -> np.ndarray:
    """float array -> fp16 bit patterns (uint16)."""
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).astype(np.float16)).view(np.uint16)


def grouped_int8_weights(rng, N, K, gs):
    """INT8 codes U{-127..127}, fp16 group scales |N(0,0.02)|/127."""
    B = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    Bs = f16(np.abs(rng.normal(0, 0.02, size=(N, K // gs))) / 127.0)
    return B, Bs


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """[N][K] int codes in [-8,7] -> [N][K/2] bytes, low nibble = even k
    (the packing of tests/test_kernel.cpp:323-330 and tensor_io.py:225-229)."""
    lo = codes[:, 0::2].astype(np.uint8) & 0x0F
    hi = codes[:, 1::2].astype(np.uint8) & 0x0F
    return np.ascontiguousarray(lo | (hi << 4))


def grouped_int4_weights(rng, N, K, gs, sd=0.02):
    """INT4 codes U{-7..7}, fp16 group scales |N(0,sd)|/7."""
    codes = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    Bs = f16(np.abs(rng.normal(0, sd, size=(N, K // gs))) / 7.0)
    return codes, pack_int4(codes), Bs


def activations(rng, M, K):
    return f16(rng.normal(0, 1, size=(M, K)))


def qwen_small_config(**over):
    """Reduced Qwen3-architecture config the oracle runs in seconds."""
    c = dict(num_layers=2, hidden=256, ffn=768, heads=4, kv_heads=2, head_dim=128, vocab=2048,
             group_size=32, eps=1e-6, rope_theta=1e6, max_seq=640, prefill_chunk=256)
    c.update(over)
    return c


def qwen_weights(rng, c, down_sd=0.1, emb_sd=0.005):
    """Random-init weights of the architecture: INT8 g-grouped attention
    projections, packed INT4 MLP, fp16 norms 1+N(0,0.02).  Group scales are
    |N(0,0.02)|/qmax except the down projection's |N(0,down_sd)|/7, and
    embeddings are N(0,emb_sd): with those two at 0.02 the decode of these
    random models repeats its input token forever (a residual stream still
    dominated by the tied embedding row predicts that row's own token)."""
    H, F, hd, gs = c["hidden"], c["ffn"], c["head_dim"], c["group_size"]
    nq, nkv = c["heads"] * hd, c["kv_heads"] * hd
    layers = []
    for _ in range(c["num_layers"]):
        L = {}
        L["input_norm"] = f16(1 + rng.normal(0, 0.02, H))
        L["post_norm"] = f16(1 + rng.normal(0, 0.02, H))
        L["q_norm"] = f16(1 + rng.normal(0, 0.02, hd))
        L["k_norm"] = f16(1 + rng.normal(0, 0.02, hd))
        for name, (n, k) in {"q": (nq, H), "k": (nkv, H), "v": (nkv, H), "o": (H, nq)}.items():
            L[name + "_w"], L[name + "_s"] = grouped_int8_weights(rng, n, k, gs)
        for name, (n, k) in {"gate": (F, H), "up": (F, H), "down": (H, F)}.items():
            _, L[name + "_w"], L[name + "_s"] = grouped_int4_weights(rng, n, k, gs,
                                                                     down_sd if name == "down" else 0.02)
        layers.append(L)
    emb = f16(rng.normal(0, emb_sd, (c["vocab"], H)))
    out_norm = f16(1 + rng.normal(0, 0.02, H))
    return layers, emb, out_norm
