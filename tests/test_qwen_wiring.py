"""Pins the oracle's Qwen3 model (OracleQwen, oracle/qwen_oracle.c) by an
independent composition of the individually pinned oracle ops, written
from the reference's graph construction:

  QwenModel::build_attention / build_mlp / build_transformer_block / forward
                                         models/model_qwen.cpp:51-172
  attention scale 1/sqrt(head_dim)       engine/engine_model.cpp:125-129
  Model::prefill chunking                engine/engine_model.cpp:170-219
  Model::decode (greedy, tied LM head)   engine/engine_model.cpp:221-297
  KV append after each execute (INT8)    engine/engine_cache.cpp:234-267
  matmul node = row quantization + grouped matmul   graph/graph_ops_nn.cpp:129-231
  attention node (causal, no window)     graph/graph_ops_nn.cpp:302-338,
                                         graph/graph.h:291-292
  hybrid node (always causal, group 128) graph/graph_ops_nn.cpp:340-371

Every op used here is pinned on its own in test_oracle_pins.py; this file
pins how they are wired.  The second half plants wiring mistakes of the
kinds a shared misreading would make (q/k norm after RoPE, a zero position
offset for later chunks, FP16 attention over the whole history instead of
the hybrid node, the residual taken after the norm, the MLP reading the
un-normed stream, the KV cache holding pre-RoPE keys) into this composition
and requires each to disagree with OracleQwen, so the comparison is shown
to see every one of them.  CPU only; runs in seconds.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as orc
from _data import qwen_small_config, qwen_weights


class Composed:
    """The Qwen3 forward and engine flow composed from pinned oracle ops.
    `plant` names one deliberate wiring mistake (None = the reference)."""

    def __init__(self, cfg, layers, emb, out_norm, plant=None):
        self.c, self.layers, self.emb, self.on = cfg, layers, emb, out_norm
        self.plant = plant
        self.scale = np.float32(1.0) / np.sqrt(np.float32(cfg["head_dim"]))
        L = cfg["num_layers"]
        self.kc = [[] for _ in range(L)]   # per layer: list of [S, Hkv, d] int8 blocks
        self.vc = [[] for _ in range(L)]
        self.ks = [[] for _ in range(L)]
        self.vs = [[] for _ in range(L)]
        self.fp_k = [[] for _ in range(L)]   # fp16 history (only for the planted FP16-attention mistake)
        self.fp_v = [[] for _ in range(L)]
        self.total = 0
        self.hidden = None

    def _mm8(self, x, w, s):
        q, qs = orc.quantize_activations(x)
        return orc.matmul_int8(q, qs, w, s, self.c["group_size"])

    def _mm4(self, x, w, s):
        q, qs = orc.quantize_activations(x)
        return orc.matmul_int4(q, qs, w, s, self.c["group_size"])

    def forward(self, tokens):
        c, P = self.c, self.plant
        S = len(tokens)
        Hq, Hkv, hd, eps, th = c["heads"], c["kv_heads"], c["head_dim"], c["eps"], c["rope_theta"]
        pos = 0 if (P == "zero_offset") else self.total
        h = np.ascontiguousarray(self.emb[np.asarray(tokens, np.int64)])
        new_k, new_v = [], []
        for l, L in enumerate(self.layers):
            x = orc.rms_norm(h, L["input_norm"], eps)
            q = self._mm8(x, L["q_w"], L["q_s"])
            k = self._mm8(x, L["k_w"], L["k_s"])
            v = self._mm8(x, L["v_w"], L["v_s"]).reshape(1, S, Hkv, hd)
            if P == "rope_before_norm":
                q = orc.rope(q.reshape(1, S, Hq, hd), pos, th)
                k = orc.rope(k.reshape(1, S, Hkv, hd), pos, th)
                q = orc.rms_norm(q.reshape(S * Hq, hd), L["q_norm"], eps).reshape(1, S, Hq, hd)
                k = orc.rms_norm(k.reshape(S * Hkv, hd), L["k_norm"], eps).reshape(1, S, Hkv, hd)
            else:
                q = orc.rms_norm(q.reshape(S * Hq, hd), L["q_norm"], eps).reshape(1, S, Hq, hd)
                k = orc.rms_norm(k.reshape(S * Hkv, hd), L["k_norm"], eps).reshape(1, S, Hkv, hd)
                k_pre = k
                q = orc.rope(q, pos, th)
                k = orc.rope(k, pos, th)
            if not self.kc[l]:
                at = orc.attention_f16(q, k, v, self.scale, pos_off=pos)
            elif P == "fp16_history":
                kk = np.concatenate(self.fp_k[l] + [k[0]])[None]
                vv = np.concatenate(self.fp_v[l] + [v[0]])[None]
                at = orc.attention_f16(q, kk, vv, self.scale, pos_off=pos)
            else:
                kc = np.concatenate(self.kc[l])[None]
                vc = np.concatenate(self.vc[l])[None]
                ks = np.concatenate(self.ks[l])[None]
                vs = np.concatenate(self.vs[l])[None]
                at = orc.attention_hybrid(q, kc, vc, ks, vs, k, v, self.scale, pos)
            new_k.append(k_pre[0] if P == "cache_pre_rope" else k[0])
            new_v.append(v[0])
            o = self._mm8(np.ascontiguousarray(at.reshape(S, Hq * hd)), L["o_w"], L["o_s"])
            if P == "residual_after_norm":
                h = orc.add(x, o)
            else:
                h = orc.add(h, o)
            x2 = h if P == "mlp_unnormed" else orc.rms_norm(h, L["post_norm"], eps)
            g = self._mm4(x2, L["gate_w"], L["gate_s"])
            u = self._mm4(x2, L["up_w"], L["up_s"])
            m = orc.multiply(orc.silu(g), u)
            h = orc.add(h, self._mm4(m, L["down_w"], L["down_s"]))
        self.hidden = orc.rms_norm(h, self.on, eps)
        # KVCache::update_from_graph after the graph executes: quantize the
        # post-RoPE keys and the values per token, append
        for l in range(len(self.layers)):
            kq, ksc = orc.quantize_kv(np.ascontiguousarray(new_k[l]))
            vq, vsc = orc.quantize_kv(np.ascontiguousarray(new_v[l]))
            self.kc[l].append(kq)
            self.ks[l].append(ksc)
            self.vc[l].append(vq)
            self.vs[l].append(vsc)
            self.fp_k[l].append(new_k[l])
            self.fp_v[l].append(new_v[l])
        self.total += S
        return self.hidden

    def prefill(self, tokens, chunk):
        n = len(tokens)
        if n <= chunk:
            self.forward(tokens)
            return
        full = (n - 1) // chunk
        for i in range(full):
            self.forward(tokens[i * chunk:(i + 1) * chunk])
        self.forward(tokens[full * chunk:])

    def decode(self, token):
        hN = self.forward([token])
        logits = orc.matmul_f16(np.ascontiguousarray(hN[-1:]), self.emb)[0]
        return orc.argmax(logits), logits

    def kv(self, l):
        return (np.concatenate(self.kc[l]), np.concatenate(self.vc[l]),
                np.concatenate(self.ks[l]), np.concatenate(self.vs[l]))


def _model(seed=5):
    cfg = qwen_small_config(num_layers=2, max_seq=256, prefill_chunk=32)
    rng = np.random.default_rng(seed)
    w = qwen_weights(rng, cfg)
    prompt = rng.integers(0, cfg["vocab"], 75).astype(np.uint32)
    return cfg, w, prompt


def _run(plant=None, steps=5):
    """Both models over a 3-chunk prefill (32 + 32 + 10 tokens) and decode
    steps; returns the first point where they differ, or None."""
    cfg, w, prompt = _model()
    ref = orc.OracleQwen(cfg, *w)
    mine = Composed(cfg, *w, plant=plant)
    chunk = cfg["prefill_chunk"]
    ref.prefill(prompt[:-1], chunk)
    mine.prefill(prompt[:-1], chunk)
    if not (mine.hidden == ref.last_hidden()).all():
        return "prefill hidden"
    tok_r = tok_m = int(prompt[-1])
    lg = np.zeros(cfg["vocab"], np.uint16)
    for s in range(steps):
        tok_r = ref.decode(tok_r, lg)
        tok_m, lg_m = mine.decode(tok_m)
        if tok_r != tok_m or not (lg == lg_m).all():
            return f"decode step {s} logits"
        if not (mine.hidden == ref.last_hidden()).all():
            return f"decode step {s} hidden"
    for l in range(cfg["num_layers"]):
        for a, b in zip(mine.kv(l), ref.read_kv(l)):
            if not (a == b).all():
                return f"kv layer {l}"
    return None


def test_oracle_qwen_matches_composition_of_pinned_ops():
    assert _run() is None


def test_composition_decodes_distinct_tokens():
    """The weights above do not collapse to one repeated id, so token
    identity carries information."""
    cfg, w, prompt = _model()
    mine = Composed(cfg, *w)
    mine.prefill(prompt[:-1], cfg["prefill_chunk"])
    tok, seen = int(prompt[-1]), []
    for _ in range(5):
        tok, _ = mine.decode(tok)
        seen.append(tok)
    assert len(set(seen)) >= 4, seen


@pytest.mark.parametrize("plant", ["rope_before_norm", "zero_offset", "fp16_history", "residual_after_norm",
                                   "mlp_unnormed", "cache_pre_rope"])
def test_planted_wiring_mistake_is_seen(plant):
    assert _run(plant) is not None, f"planted mistake {plant} went unnoticed"
