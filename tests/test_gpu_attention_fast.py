"""Tolerance-mode (split-K) decode attention against the oracle.

cactus_hip_attention_f16_fast and cactus_hip_attention_hybrid_int8_fp16_fast
compute the reference's softmax attention (kernel_attention.cpp:10-255,
257-482) with a different fp32 summation order, so the bar is the
tolerance of fp16 outputs: |gpu - ref| <= 1e-3 + 1e-2 |ref| per element,
written in `close` below.  Shapes: config 4 (16 query / 8 KV heads,
head_dim 128, 4096 context, RoPE theta 1e6 applied at positions 4095 for
q and 0..4095 for k) in its FP16 and INT8-cache forms, split edges (1, 255,
256, 257 keys), GQA 1/2/4, head_dim 64, batch 2, a sliding window, two new
rows, a causal cut inside the keys, peaked scores, and shapes the fast
path hands to the exact kernels (FP16 prefill rows, head_dim 40, a mask),
which must then be bit-identical to the oracle.  Prefill rows of the hybrid
form run the FP16-MFMA flash kernel (chunk shapes of a 4096-token prefill,
with and without key splits and their combine).
"""
import ctypes
import math
import sys

import numpy as np
import pytest

from _data import f16

pytestmark = pytest.mark.gpu

ABS_TOL, REL_TOL = 1e-3, 1e-2


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def close(got, ref, what):
    g = np.asarray(got, np.uint16).view(np.float16).astype(np.float64)
    r = np.asarray(ref, np.uint16).view(np.float16).astype(np.float64)
    err = np.abs(g - r)
    bad = np.flatnonzero(err.ravel() > ABS_TOL + REL_TOL * np.abs(r).ravel())
    assert bad.size == 0, f"{what}: {bad.size}/{r.size} outside tolerance, first at {bad[:5]}: " \
                          f"got {g.ravel()[bad[:5]]} ref {r.ravel()[bad[:5]]}"
    return float(err.max())


class Dev:
    def __init__(self, cm):
        self.cm = cm
        self.bufs = []

    def put(self, arr):
        b = self.cm.DeviceBuffer.from_numpy(np.ascontiguousarray(arr))
        self.bufs.append(b)
        return b.ptr

    def empty(self, n):
        b = self.cm.DeviceBuffer(n)
        self.bufs.append(b)
        return b

    def get(self, buf, dtype, shape):
        self.cm.call("cactus_hip_stream_sync", None)
        return buf.to_numpy(dtype, shape)

    def get_ptr(self, ptr, dtype, shape):
        out = np.empty(shape, dtype)
        self.cm.call("cactus_hip_stream_sync", None)
        self.cm.call("cactus_hip_memcpy_d2h", out.ctypes.data, ptr, out.nbytes, None)
        return out


@pytest.fixture
def dev(hip_ready):
    d = Dev(hip_ready)
    yield d
    for b in d.bufs:
        b.free()


def _roped(orc, x, start):
    """RoPE (theta 1e6) of [B, S, H, d] rows at positions start.. (a9)."""
    return orc.rope(x, start, 1e6)


@pytest.mark.parametrize("B,Skv,Hq,Hkv,d,pos,window,qmul", [
    (1, 4096, 16, 8, 128, 4095, 0, 1.0),    # config 4, FP16 KV
    (1, 1, 16, 8, 128, 0, 0, 1.0),
    (1, 255, 4, 2, 128, 254, 0, 1.0),
    (1, 256, 4, 4, 64, 255, 0, 1.0),
    (1, 257, 8, 2, 128, 256, 0, 1.0),
    (2, 700, 4, 1, 64, 699, 0, 1.0),
    (1, 1000, 4, 2, 128, 600, 0, 1.0),     # causal cut: keys past the query position
    (1, 900, 4, 2, 128, 899, 300, 1.0),    # sliding window
    (1, 3000, 16, 8, 128, 2999, 0, 30.0),  # peaked scores
    (1, 20000, 8, 2, 128, 19999, 0, 1.0),  # 79 splits of 4 query heads: the many-split combine
])
def test_attention_f16_fast(dev, orc, B, Skv, Hq, Hkv, d, pos, window, qmul):
    say("attention_f16_fast", B, Skv, Hq, Hkv, d, pos, window, qmul)
    rng = np.random.default_rng(Skv + d + Hq)
    q = _roped(orc, f16(rng.normal(0, 1, (B, 1, Hq, d)) * qmul), pos)
    k = _roped(orc, f16(rng.normal(0, 1, (B, Skv, Hkv, d))), 0)
    v = f16(rng.normal(0, 1, (B, Skv, Hkv, d)))
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_f16(q, k, v, scale, pos_off=pos, window=window)
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_attention_f16_fast", dev.put(q), dev.put(k), dev.put(v), o.ptr, B, 1, Skv, Hq, Hkv, d,
                ctypes.c_float(scale), None, pos, window, 1, None)
    close(dev.get(o, np.uint16, q.shape), ref, "attention_f16_fast")


@pytest.mark.parametrize("B,cache,new,Hq,Hkv,d,qmul", [
    (1, 4095, 1, 16, 8, 128, 1.0),     # config 4, INT8 cache + the new FP16 row
    (1, 0, 1, 16, 8, 128, 1.0),
    (1, 255, 1, 4, 2, 128, 1.0),
    (1, 256, 1, 4, 1, 64, 1.0),
    (1, 511, 2, 8, 2, 128, 1.0),       # two new rows
    (2, 1000, 1, 8, 2, 64, 1.0),
    (1, 3000, 1, 16, 8, 128, 30.0),    # peaked scores
    (1, 9000, 1, 16, 8, 128, 1.0),     # 36 splits: the many-split combine
])
def test_attention_hybrid_fast(dev, orc, B, cache, new, Hq, Hkv, d, qmul):
    say("attention_hybrid_fast", B, cache, new, Hq, Hkv, d, qmul)
    rng = np.random.default_rng(cache + new + d + 7)
    pos = cache + new - 1
    kf = _roped(orc, f16(rng.normal(0, 1, (B, max(cache, 1), Hkv, d))), 0)
    vf = f16(rng.normal(0, 1, (B, max(cache, 1), Hkv, d)))
    kc = np.zeros((B, max(cache, 1), Hkv, d), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((B, max(cache, 1), Hkv, 1), np.float32)
    vs = np.zeros_like(ks)
    for b in range(B):
        kc[b], ks[b] = orc.quantize_kv(kf[b])
        vc[b], vs[b] = orc.quantize_kv(vf[b])
    # one scale table for every batch row (kernel_attention.cpp:353,424)
    kc, vc, ks, vs = (np.ascontiguousarray(x[:, :cache]) for x in (kc, vc, ks[:1], vs[:1]))
    kn = _roped(orc, f16(rng.normal(0, 1, (B, new, Hkv, d))), cache)
    vn = f16(rng.normal(0, 1, (B, new, Hkv, d)))
    q = _roped(orc, f16(rng.normal(0, 1, (B, 1, Hq, d)) * qmul), pos)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_hybrid(q, kc if cache else None, vc if cache else None, ks if cache else None,
                               vs if cache else None, kn, vn, scale, pos_off=pos)
    o = dev.empty(q.nbytes)
    P = (lambda a: dev.put(a) if cache else None)
    dev.cm.call("cactus_hip_attention_hybrid_int8_fp16_fast", dev.put(q), P(kc), P(vc), P(ks), P(vs), dev.put(kn),
                dev.put(vn), o.ptr, B, 1, cache, new, Hq, Hkv, d, ctypes.c_float(scale), pos, 1, 128, None)
    close(dev.get(o, np.uint16, q.shape), ref, "attention_hybrid_fast")


def test_fast_entries_hand_other_shapes_to_the_exact_kernels(dev, orc):
    """Prefill rows, head_dim 40 and a mask run the exact kernels:
    bit-identical to the oracle."""
    rng = np.random.default_rng(5)
    for S, Skv, d, masked in [(8, 64, 128, False), (1, 50, 40, False), (1, 45, 64, True)]:
        say("attention_f16_fast -> exact", S, Skv, d, masked)
        q = f16(rng.normal(0, 1, (1, S, 4, d)))
        k = f16(rng.normal(0, 1, (1, Skv, 2, d)))
        v = f16(rng.normal(0, 1, (1, Skv, 2, d)))
        mask = f16((rng.random((1, S, Skv)) > 0.3).astype(np.float32)) if masked else None
        scale = 1.0 / math.sqrt(d)
        pos = Skv - S
        ref = orc.attention_f16(q, k, v, scale, mask=mask, pos_off=pos)
        o = dev.empty(q.nbytes)
        dev.cm.call("cactus_hip_attention_f16_fast", dev.put(q), dev.put(k), dev.put(v), o.ptr, 1, S, Skv, 4, 2, d,
                    ctypes.c_float(scale), dev.put(mask) if masked else None, pos, 0, 1, None)
        got = dev.get(o, np.uint16, q.shape)
        assert (got == ref).all(), (S, Skv, d, masked)


@pytest.mark.parametrize("cache,Hq,Hkv,d", [
    (4095, 16, 8, 128), (4096, 16, 8, 128), (4097, 16, 8, 128),   # split edges of the config-4 shape
    (127, 4, 2, 128), (128, 4, 2, 128), (129, 4, 2, 64), (300, 4, 4, 64), (0, 4, 2, 128),
    (255, 4, 2, 128), (256, 4, 2, 128), (511, 4, 2, 64),                 # 256-key split edges
])
def test_decode_prep_attention_fast(dev, orc, cache, Hq, Hkv, d):
    """The fused decode step's attention in tolerance mode against the exact
    fused entry point on the same cache and step state: the prepared key and
    value appended to the cache (codes and scales) bit-identical, the output
    within tolerance; run twice on one workspace (the split counters reset
    themselves)."""
    say("decode_prep_attention_fast", cache, Hq, Hkv, d)
    rng = np.random.default_rng(cache * 3 + d + Hq)
    cap = cache + 70
    kc, ks = orc.quantize_kv(_roped(orc, f16(rng.normal(0, 1, (1, cap, Hkv, d))), 0)[0])
    vc, vs = orc.quantize_kv(f16(rng.normal(0, 1, (cap, Hkv, d))))
    q_raw = f16(rng.normal(0, 1, (Hq, d)))
    k_raw = f16(rng.normal(0, 1, (Hkv, d)))
    v_raw = f16(rng.normal(0, 1, (Hkv, d)))
    qn = f16(rng.normal(1, 0.2, d))
    kn = f16(rng.normal(1, 0.2, d))
    eps, theta, scale = 1e-6, 1e6, 1.0 / math.sqrt(d)
    state = dev.put(np.array([0, cache, cache, 0], np.uint32))
    raw = [dev.put(x) for x in (q_raw, k_raw, v_raw, qn, kn)]
    ws_bytes = dev.cm.hip().cactus_hip_decode_attention_fast_workspace(Hq, Hkv, d, cap)
    ws = dev.empty(ws_bytes)
    dev.cm.call("cactus_hip_memset", ws.ptr, 0, ws_bytes, None)
    outs, rows = [], []
    for fast in (False, True, True):
        bufs = [dev.put(kc), dev.put(vc), dev.put(ks), dev.put(vs)]
        o = dev.empty(q_raw.nbytes)
        if fast:
            dev.cm.call("cactus_hip_decode_prep_attention_fast", *raw, ctypes.c_float(eps), Hq, Hkv, d,
                        ctypes.c_float(theta), state, *bufs, cap, None, ctypes.c_float(scale), o.ptr, ws.ptr, ws_bytes,
                        None)
        else:
            dev.cm.call("cactus_hip_decode_prep_attention", *raw, ctypes.c_float(eps), Hq, Hkv, d,
                        ctypes.c_float(theta), state, *bufs, cap, None, ctypes.c_float(scale), o.ptr, None)
        outs.append(dev.get(o, np.uint16, (Hq, d)))
        rows.append([dev.get_ptr(b, dt, shp)[cache] for b, dt, shp in
                     zip(bufs, (np.int8, np.int8, np.float32, np.float32),
                         ((cap, Hkv, d), (cap, Hkv, d), (cap, Hkv, 1), (cap, Hkv, 1)))])
    for i in (1, 2):
        for x, y in zip(rows[0], rows[i]):
            assert (x == y).all(), "appended cache row"
        close(outs[i], outs[0], "decode_prep_attention_fast")
    assert (outs[1] == outs[2]).all(), "second launch on the same workspace"


@pytest.mark.parametrize("B,cache,new,Hq,Hkv,d,qmul,pos", [
    (1, 3840, 256, 16, 8, 128, 1.0, None),   # the last 256-row chunk of a 4096-token prefill
    (1, 0, 256, 16, 8, 128, 1.0, None),      # the first chunk: new rows only
    (1, 700, 100, 8, 2, 128, 1.0, None),     # GQA 4, ragged row count
    (2, 129, 37, 4, 4, 64, 1.0, None),       # batch 2, head_dim 64, GQA 1
    (1, 1000, 256, 16, 8, 128, 6.0, None),   # peaked scores
    (1, 3, 5, 4, 2, 128, 1.0, None),         # tiny
    (1, 500, 64, 16, 8, 128, 1.0, 530),      # position past the cache length (a windowed cache)
    (1, 0, 40, 4, 2, 128, 1.0, 17),          # no cache, rows from position 17
])
def test_attention_hybrid_prefill_fast(dev, orc, B, cache, new, Hq, Hkv, d, qmul, pos):
    """Prefill rows (S = new rows at positions pos..pos+new-1, pos the
    cache length unless given; the causal limit of row r is key index
    pos + r) through the FP16-MFMA flash kernel, against the oracle's hybrid
    attention within 1e-3 + 1e-2 |ref|.  The peaked case keeps the score
    spread below ~88: the reference rescales by expf(previous block max -
    this block max) (kernel_attention.cpp:395-403), which overflows when a
    later block's maximum lies that far below an earlier one, and then
    writes a zero row (:465-469); the tolerance mode computes the softmax
    itself there."""
    say("attention_hybrid_prefill_fast", B, cache, new, Hq, Hkv, d, qmul, pos)
    pos = cache if pos is None else pos
    rng = np.random.default_rng(cache * 5 + new + d)
    kf = _roped(orc, f16(rng.normal(0, 1, (B, max(cache, 1), Hkv, d))), 0)
    vf = f16(rng.normal(0, 1, (B, max(cache, 1), Hkv, d)))
    kc = np.zeros((B, max(cache, 1), Hkv, d), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((B, max(cache, 1), Hkv, 1), np.float32)
    vs = np.zeros_like(ks)
    for b in range(B):
        kc[b], ks[b] = orc.quantize_kv(kf[b])
        vc[b], vs[b] = orc.quantize_kv(vf[b])
    kc, vc, ks, vs = (np.ascontiguousarray(x[:, :cache]) for x in (kc, vc, ks[:1], vs[:1]))
    kn = _roped(orc, f16(rng.normal(0, 1, (B, new, Hkv, d))), pos)
    vn = f16(rng.normal(0, 1, (B, new, Hkv, d)))
    q = _roped(orc, f16(rng.normal(0, 1, (B, new, Hq, d)) * qmul), pos)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_hybrid(q, kc if cache else None, vc if cache else None, ks if cache else None,
                               vs if cache else None, kn, vn, scale, pos_off=pos)
    o = dev.empty(q.nbytes)
    P = (lambda a: dev.put(a) if cache else None)
    dev.cm.call("cactus_hip_attention_hybrid_int8_fp16_fast", dev.put(q), P(kc), P(vc), P(ks), P(vs), dev.put(kn),
                dev.put(vn), o.ptr, B, new, cache, new, Hq, Hkv, d, ctypes.c_float(scale), pos, 1, 128, None)
    err = close(dev.get(o, np.uint16, q.shape), ref, "attention_hybrid_prefill_fast")
    print(f"[prefill fast] max abs error {err:.2e}", flush=True)
