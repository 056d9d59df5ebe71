"""Frozen vectors of the kernel layer (tests/golden/golden.npz, written by
tests/golden/make_golden.py from the oracle).

* CPU: the oracle still reproduces every stored output bit for bit.
* GPU: the HIP entry points reproduce them through the C ABI, with no oracle
  involved at run time.
"""
import ctypes
import math
from pathlib import Path

import numpy as np
import pytest

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


def _same(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    bad = np.flatnonzero(got.reshape(-1).view(np.uint8) != want.reshape(-1).view(np.uint8))
    assert bad.size == 0, f"{what}: {bad.size} differing bytes"


def test_oracle_reproduces_golden(orc):
    c, s = orc.quantize_activations(G["qa_x"])
    _same(c, G["qa_codes"], "quantize codes")
    _same(s, G["qa_scales"], "quantize scales")
    for p, gs, fn in (("mm8", 32, orc.matmul_int8), ("mm8p", 64, orc.matmul_int8), ("mm4", 32, orc.matmul_int4)):
        q, sc = orc.quantize_activations(G[p + "_x"])
        _same(fn(q, sc, G[p + "_B"], G[p + "_Bs"], gs), G[p + "_C"], p)
    _same(orc.attention_f16(G["af_q"], G["af_k"], G["af_v"], 1.0 / math.sqrt(64), pos_off=35), G["af_o"],
          "attention_f16")
    _same(orc.attention_hybrid(G["ah_q"], G["ah_kc"][None], G["ah_vc"][None], G["ah_ks"][None], G["ah_vs"][None],
                               G["ah_kn"], G["ah_vn"], 1.0 / math.sqrt(64), pos_off=70), G["ah_o"],
          "attention_hybrid")
    c, s = orc.quantize_kv(G["kv_x"])
    _same(c, G["kv_codes"], "kv codes")
    _same(s, G["kv_scales"], "kv scales")
    _same(orc.rms_norm(G["rms_x"], G["rms_w"], 1e-6), G["rms_y"], "rms_norm")
    _same(orc.rope(G["rope_x"], 100, 1e6), G["rope_y"], "rope")
    _same(orc.softmax(G["sm_x"]), G["sm_y"], "softmax")
    _same(orc.silu(G["ew_a"]), G["ew_silu"], "silu")
    _same(orc.add(G["ew_a"], G["ew_b"]), G["ew_add"], "add")
    _same(orc.multiply(G["ew_a"], G["ew_b"]), G["ew_mul"], "multiply")
    assert orc.argmax(G["am_x"]) == int(G["am_i"][0]) == 17


@pytest.mark.gpu
def test_hip_reproduces_golden(hip_ready):
    cm = hip_ready
    keep = []

    def put(a):
        b = cm.DeviceBuffer.from_numpy(np.ascontiguousarray(a))
        keep.append(b)
        return b.ptr

    def out(like):
        b = cm.DeviceBuffer(np.asarray(like).nbytes)
        keep.append(b)
        return b

    def get(b, like):
        like = np.asarray(like)
        cm.call("cactus_hip_stream_sync", None)
        return b.to_numpy(like.dtype, like.shape)

    x = G["qa_x"]
    c, s = out(G["qa_codes"]), out(G["qa_scales"])
    cm.call("cactus_hip_quantize_activations", put(x), c.ptr, s.ptr, x.shape[0], x.shape[1], None)
    _same(get(c, G["qa_codes"]), G["qa_codes"], "quantize codes")
    _same(get(s, G["qa_scales"]), G["qa_scales"], "quantize scales")
    for p, gs, name in (("mm8", 32, "cactus_hip_matmul_int8_f16act"), ("mm8p", 64, "cactus_hip_matmul_int8_f16act"),
                        ("mm4", 32, "cactus_hip_matmul_int4_f16act")):
        x, Cw = G[p + "_x"], G[p + "_C"]
        C = out(Cw)
        cm.call(name, put(x), put(G[p + "_B"]), put(G[p + "_Bs"]), C.ptr, x.shape[0], x.shape[1], Cw.shape[1], gs,
                None)
        _same(get(C, Cw), Cw, p)
    q = G["af_q"]
    o = out(G["af_o"])
    cm.call("cactus_hip_attention_f16", put(q), put(G["af_k"]), put(G["af_v"]), o.ptr, 1, 5, 40, 4, 2, 64,
            ctypes.c_float(1.0 / math.sqrt(64)), None, 35, 0, 1, None)
    _same(get(o, G["af_o"]), G["af_o"], "attention_f16")
    o = out(G["ah_o"])
    cm.call("cactus_hip_attention_hybrid_int8_fp16", put(G["ah_q"]), put(G["ah_kc"]), put(G["ah_vc"]),
            put(G["ah_ks"]), put(G["ah_vs"]), put(G["ah_kn"]), put(G["ah_vn"]), o.ptr, 1, 3, 70, 3, 4, 2, 64,
            ctypes.c_float(1.0 / math.sqrt(64)), 70, 1, 128, None)
    _same(get(o, G["ah_o"]), G["ah_o"], "attention_hybrid")
    x = G["kv_x"]
    c, s = out(G["kv_codes"]), out(G["kv_scales"])
    cm.call("cactus_hip_quantize_kv_fp16_to_int8", put(x), c.ptr, s.ptr, 5, 2, 128, 128, None)
    _same(get(c, G["kv_codes"]), G["kv_codes"], "kv codes")
    _same(get(s, G["kv_scales"]), G["kv_scales"], "kv scales")
    y = out(G["rms_y"])
    cm.call("cactus_hip_rms_norm_f16", put(G["rms_x"]), put(G["rms_w"]), y.ptr, 4, 256, ctypes.c_float(1e-6), None)
    _same(get(y, G["rms_y"]), G["rms_y"], "rms_norm")
    y = out(G["rope_y"])
    cm.call("cactus_hip_rope_f16", put(G["rope_x"]), y.ptr, 1, 3, 2, 64, 100, ctypes.c_float(1e6), None)
    _same(get(y, G["rope_y"]), G["rope_y"], "rope")
    y = out(G["sm_y"])
    cm.call("cactus_hip_softmax_f16", put(G["sm_x"]), y.ptr, 1, 3, 100, None)
    _same(get(y, G["sm_y"]), G["sm_y"], "softmax")
    a, b = put(G["ew_a"]), put(G["ew_b"])
    for name, key, args in (("cactus_hip_silu_f16", "ew_silu", (a,)), ("cactus_hip_add_f16", "ew_add", (a, b)),
                            ("cactus_hip_multiply_f16", "ew_mul", (a, b))):
        y = out(G[key])
        cm.call(name, *args, y.ptr, 300, None)
        _same(get(y, G[key]), G[key], key)
    t = out(G["am_i"])
    cm.call("cactus_hip_sample_f16", put(G["am_x"]), t.ptr, 1000, ctypes.c_float(0.0), ctypes.c_float(0.0), 0, 0,
            None)
    _same(get(t, G["am_i"]), G["am_i"], "greedy token")
    for b in keep:
        b.free()
