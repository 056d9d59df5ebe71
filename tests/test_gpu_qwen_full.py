"""The full-shape Qwen3-0.6B-architecture run against the oracle's frozen run
of the same workload (tests/golden/qwen3_0p6b_generate.npz, written by
tests/golden/make_qwen_golden.py; no oracle at run time).

Workload: 28 layers, hidden 1024, MLP 3072, 16/8 heads, head_dim 128,
vocab 151936, group-32 INT8 attention projections and packed INT4 MLP,
FP16 tied embeddings and norms, random-init weights of seed 6, a 4096-token
prompt (seed 7) prefilled as prompt[:-1] in 256-token chunks, then 128
greedy steps from prompt[-1] (engine_model.cpp:170-297,
cactus_complete.cpp:196-204) -- the run bench.py times.

Required bit for bit, in decode mode 0 (node graph) and mode 1 (fused
kernels replayed as a HIP graph): every token id, every step's fp16 logits
row (SHA-256), every layer's final INT8 KV cache (SHA-256) and, in mode 0,
the last final hidden state.  Mode 1 is also run through generate(), the
bench's own path (all 128 steps queued on the device with no host round
trip).  The weights make 128 distinct ids (a CPU test checks the fixture),
so token identity is not one repeated id.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

pytestmark = pytest.mark.gpu

FIXTURE = HERE / "golden" / "qwen3_0p6b_generate.npz"


def say(*a):
    print("[case]", *a, flush=True)


def sha(*arrays) -> bytes:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.digest()


@pytest.fixture(scope="module")
def full():
    import cactus_amd
    from cactus_amd.engine import Qwen
    from make_qwen_golden import WEIGHT_SEED, workload
    cactus_amd.call("cactus_hip_init", 0)
    fx = dict(np.load(FIXTURE))
    cfg, prompt = workload()
    say("qwen3-0.6b full shape: create (seed 6)")
    m = Qwen(cfg, seed=WEIGHT_SEED)
    yield m, fx, cfg, prompt
    m.close()


def _first_diff(fx, step, lg):
    ids = fx["top16_ids"][step]
    return {"step": step, "oracle_top_ids": ids[:4].tolist(), "oracle_top_bits": fx["top16_bits"][step][:4].tolist(),
            "gpu_bits_at_those_ids": lg[ids[:4]].tolist()}


def _check_kv(m, fx, cfg):
    assert m.cache_len() == int(fx["cache_len"])
    for layer in range(cfg["num_layers"]):
        assert sha(*m.read_kv(layer)) == fx["kv_sha256"][layer].tobytes(), f"kv cache layer {layer}"


@pytest.mark.parametrize("mode", [0, 1])
def test_qwen3_full_shape_step_by_step(full, mode):
    m, fx, cfg, prompt = full
    say("qwen3-0.6b full shape, step by step, mode", mode)
    m.reset()
    m.set_decode_mode(mode)
    m.prefill(prompt[:-1])
    tok = int(prompt[-1])
    for i in range(len(fx["tokens"])):
        tok = m.decode(tok)
        lg = m.last_logits()
        assert sha(lg) == fx["logits_sha256"][i].tobytes(), _first_diff(fx, i, lg)
        assert tok == int(fx["tokens"][i]), (i, tok, int(fx["tokens"][i]))
    _check_kv(m, fx, cfg)
    if mode == 0:
        assert sha(m.last_hidden()) == fx["hidden_sha256"].tobytes()


def test_qwen3_full_shape_generate_fused(full):
    """The bench's path: generate() in mode 1 (prefill, then all steps on the
    device)."""
    m, fx, cfg, prompt = full
    say("qwen3-0.6b full shape, generate, mode 1")
    m.reset()
    m.set_decode_mode(1)
    toks, _ = m.generate(prompt, len(fx["tokens"]))
    assert toks.tolist() == fx["tokens"].tolist()
    assert sha(m.last_logits()) == fx["logits_sha256"][-1].tobytes()
    _check_kv(m, fx, cfg)


def test_qwen3_full_shape_tolerance_mode(full):
    """Tolerance-mode attention (split-K decode attention and the MFMA
    prefill attention, each within 1e-3 + 1e-2 |ref| of the reference per
    fp16 output, tested kernel by kernel in test_gpu_attention_fast.py) at
    model level.  The exact mode is first checked against the fixture; then
    the tolerance mode is prefilled and run teacher-forced on the fixture's
    tokens, and its logits compared step by step with the exact mode's.  This
    random 28-layer model amplifies single-ulp attention differences.  Both
    runs are deterministic; measured on MI355X: relative L2 of the logits
    0.090-0.167 per step (mean 0.117; already 0.126 at step 0, from the
    prefill) and the argmax equal on 89 of 128 steps.  The bounds sit ~20%
    above the measured errors (every step <= 0.20, the mean <= 0.14) and ~10%
    below the measured agreement (at least 80 of 128 argmax equal); garbage
    attention lands near 1 and agrees on almost no step.  The free-running token prefix that matches the oracle
    is printed, not required: it is 3 steps."""
    m, fx, cfg, prompt = full
    toks = fx["tokens"]
    say("qwen3-0.6b full shape, exact vs tolerance attention")
    m.reset()
    m.set_decode_mode(1)
    m.set_attention_mode(0)
    m.prefill(prompt[:-1])
    ref = []
    tok = int(prompt[-1])
    for i in range(len(toks)):
        t = m.decode(tok)
        lg = m.last_logits()
        assert sha(lg) == fx["logits_sha256"][i].tobytes(), i
        ref.append(lg.view(np.float16).astype(np.float64))
        tok = int(toks[i])
        assert t == tok
    m.reset()
    m.set_attention_mode(1)
    try:
        m.prefill(prompt[:-1])
        tok = int(prompt[-1])
        rel, agree = [], 0
        for i in range(len(toks)):
            t = m.decode(tok)
            g = m.last_logits().view(np.float16).astype(np.float64)
            rel.append(float(np.linalg.norm(g - ref[i]) / np.linalg.norm(ref[i])))
            agree += int(t == int(toks[i]))
            tok = int(toks[i])
        m.reset()
        free, _ = m.generate(prompt, len(toks))
    finally:
        m.set_attention_mode(0)
    prefix = int(np.argmax(free != toks)) if (free != toks).any() else len(toks)
    print(f"[tolerance mode] max relative L2 of logits {max(rel):.4f}, argmax agreement {agree}/{len(toks)}, "
          f"free-running tokens equal to the oracle's for the first {prefix} steps", flush=True)
    print(f"[tolerance mode] mean relative L2 {float(np.mean(rel)):.4f}", flush=True)
    assert max(rel) <= 0.20, rel
    assert float(np.mean(rel)) <= 0.14, rel
    assert agree * 128 >= 80 * len(toks), agree
