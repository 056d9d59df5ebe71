"""Writes tests/golden/golden.npz: seeded inputs of the kernel-layer entry
points and the oracle's outputs for them.

The reference stores no vectors of its own (its kernel tests draw unseeded
random data), so these fixtures are the oracle's, frozen: the CPU test
requires the oracle to keep reproducing them, and the GPU test requires the
HIP path to reproduce them through the C ABI without consulting the oracle.

    python tests/golden/make_golden.py     (rewrites golden.npz)
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

import oracle as orc  # noqa: E402
from _data import activations, f16, grouped_int4_weights, grouped_int8_weights  # noqa: E402

OUT = HERE / "golden.npz"


def cases() -> dict:
    rng = np.random.default_rng(20261201)
    g = {}
    # a1: per-row activation quantization, ragged K and special values
    x = activations(rng, 3, 1001)
    x[0, :4] = f16([0.0, -0.0, 65504.0, -3.5])
    g["qa_x"] = x
    g["qa_codes"], g["qa_scales"] = orc.quantize_activations(x)
    # a2: grouped INT8 matmul, FP16 activations (slice of the M=1 K=640 N=2048 g32 GEMV)
    x = activations(rng, 1, 640)
    B, Bs = grouped_int8_weights(rng, 64, 640, 32)
    q, s = orc.quantize_activations(x)
    g["mm8_x"], g["mm8_B"], g["mm8_Bs"] = x, B, Bs
    g["mm8_C"] = orc.matmul_int8(q, s, B, Bs, 32)
    # a2 at a prefill size (the MFMA path)
    x = activations(rng, 40, 256)
    B, Bs = grouped_int8_weights(rng, 96, 256, 64)
    q, s = orc.quantize_activations(x)
    g["mm8p_x"], g["mm8p_B"], g["mm8p_Bs"] = x, B, Bs
    g["mm8p_C"] = orc.matmul_int8(q, s, B, Bs, 64)
    # a3: packed INT4
    x = activations(rng, 2, 256)
    _, packed, Bs = grouped_int4_weights(rng, 64, 256, 32)
    q, s = orc.quantize_activations(x)
    g["mm4_x"], g["mm4_B"], g["mm4_Bs"] = x, packed, Bs
    g["mm4_C"] = orc.matmul_int4(q, s, packed, Bs, 32)
    # a5: FP16 attention, causal, GQA 2
    q = f16(rng.normal(0, 1, (1, 5, 4, 64)))
    k = f16(rng.normal(0, 1, (1, 40, 2, 64)))
    v = f16(rng.normal(0, 1, (1, 40, 2, 64)))
    g["af_q"], g["af_k"], g["af_v"] = q, k, v
    g["af_o"] = orc.attention_f16(q, k, v, 1.0 / math.sqrt(64), pos_off=35)
    # a6 + a7: hybrid attention over an INT8 cache
    kc, ks = orc.quantize_kv(f16(rng.normal(0, 1, (70, 2, 64))))
    vc, vs = orc.quantize_kv(f16(rng.normal(0, 1, (70, 2, 64))))
    kn = f16(rng.normal(0, 1, (1, 3, 2, 64)))
    vn = f16(rng.normal(0, 1, (1, 3, 2, 64)))
    q = f16(rng.normal(0, 1, (1, 3, 4, 64)))
    g["ah_q"], g["ah_kc"], g["ah_vc"], g["ah_ks"], g["ah_vs"], g["ah_kn"], g["ah_vn"] = q, kc, vc, ks, vs, kn, vn
    g["ah_o"] = orc.attention_hybrid(q, kc[None], vc[None], ks[None], vs[None], kn, vn, 1.0 / math.sqrt(64),
                                     pos_off=70)
    x = f16(rng.normal(0, 1, (5, 2, 128)))
    g["kv_x"] = x
    g["kv_codes"], g["kv_scales"] = orc.quantize_kv(x)
    # a8-a14
    x = f16(rng.normal(0, 1, (4, 256)))
    w = f16(1 + rng.normal(0, 0.05, 256))
    g["rms_x"], g["rms_w"] = x, w
    g["rms_y"] = orc.rms_norm(x, w, 1e-6)
    x = f16(rng.normal(0, 1, (1, 3, 2, 64)))
    g["rope_x"] = x
    g["rope_y"] = orc.rope(x, 100, 1e6)
    x = f16(rng.normal(0, 2, (3, 100)))
    g["sm_x"] = x
    g["sm_y"] = orc.softmax(x)
    x = f16(rng.normal(0, 3, 300))
    y = f16(rng.normal(0, 1, 300))
    g["ew_a"], g["ew_b"] = x, y
    g["ew_silu"], g["ew_add"], g["ew_mul"] = orc.silu(x), orc.add(x, y), orc.multiply(x, y)
    logits = f16(rng.normal(0, 1, 1000))
    logits[[17, 901]] = f16([5.0, 5.0])
    g["am_x"] = logits
    g["am_i"] = np.array([orc.argmax(logits)], np.uint32)
    return g


def main() -> None:
    np.savez_compressed(OUT, **cases())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
