"""Writes tests/golden/qwen3_0p6b_generate.npz: the oracle's run of the
full-shape Qwen3-0.6B-architecture workload.

Workload (the same one bench.py times): 28 layers, hidden 1024, MLP 3072,
16/8 heads, head_dim 128, vocab 151936, group-32 INT8 attention projections
and packed INT4 MLP, FP16 embeddings (tied LM head) and norms; random-init
weights of seed 6 (cactus_qwen_random_weights, generated on the host, no
device); a 4096-token prompt of ids U[0, 151936) from numpy seed 7; the
reference's FFI flow (engine_model.cpp:170-219 prefill of prompt[:-1] in
256-token chunks, cactus_complete.cpp:196-204 decode from prompt[-1]), then
128 greedy decode steps (engine_model.cpp:221-297).

Stored: the 128 token ids; per decode step the SHA-256 of the fp16 logits
row and its 16 largest entries (ids and bit patterns, for diagnosis); per
layer the SHA-256 of the final INT8 KV cache (codes K, codes V, scales K,
scales V, in that order); the SHA-256 of the last forward's final hidden
state; and the SHA-256 of the weights, so a change of the generator is
caught on the CPU.

The oracle runs its row and head loops on threads (orc_set_threads); each
output element is computed by the same sequential code whatever the thread
count, so the results do not depend on it.

    python tests/golden/make_qwen_golden.py [--threads 8]
"""
from __future__ import annotations

import argparse
import hashlib
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
sys.path.insert(0, str(HERE.parent))

OUT = HERE / "qwen3_0p6b_generate.npz"
PROMPT_LEN, NEW_TOKENS, WEIGHT_SEED, PROMPT_SEED = 4096, 128, 6, 7


def workload():
    """(cfg, prompt) of the full-shape run."""
    from cactus_amd.engine import qwen3_0p6b
    cfg = qwen3_0p6b(max_seq=PROMPT_LEN + NEW_TOKENS + 64)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], PROMPT_LEN).astype(np.uint32)
    return cfg, prompt


def sha(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), np.uint8).copy()


def weights_digest(layers, emb, on) -> np.ndarray:
    from cactus_amd.engine import LAYER_FIELDS
    return sha(*[L[k] for L in layers for k in LAYER_FIELDS], emb, on)


def top16(logits: np.ndarray):
    """16 largest logits (ids ascending within equal values), as fp16 bits."""
    v = logits.view(np.float16).astype(np.float32)
    idx = np.lexsort((np.arange(v.size), -v))[:16]
    return idx.astype(np.uint32), logits[idx]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    args = ap.parse_args()
    import oracle
    from cactus_amd.engine import random_weights
    oracle.lib().orc_set_threads(args.threads)
    cfg, prompt = workload()
    t0 = time.time()
    layers, emb, on = random_weights(cfg, WEIGHT_SEED)
    wd = weights_digest(layers, emb, on)
    print(f"weights ready ({time.time() - t0:.1f} s)", flush=True)
    orc = oracle.OracleQwen(cfg, layers, emb, on)
    chunk = cfg["prefill_chunk"]
    body = prompt[:-1]
    t1 = time.time()
    # Model::prefill's chunking (engine_model.cpp:203-218), one chunk per call
    # so progress shows; the oracle's own chunker gives the same calls
    n_full = (len(body) - 1) // chunk
    starts = [i * chunk for i in range(n_full)] + [n_full * chunk]
    for i, s in enumerate(starts):
        e = s + chunk if i < n_full else len(body)
        orc.prefill(body[s:e], chunk=e - s)
        print(f"prefill chunk {i + 1}/{len(starts)} ({e} tokens, {time.time() - t1:.0f} s)", flush=True)
    prefill_s = time.time() - t1
    toks = np.zeros(NEW_TOKENS, np.uint32)
    dig = np.zeros((NEW_TOKENS, 32), np.uint8)
    top_ids = np.zeros((NEW_TOKENS, 16), np.uint32)
    top_bits = np.zeros((NEW_TOKENS, 16), np.uint16)
    lg = np.zeros(cfg["vocab"], np.uint16)
    tok = int(prompt[-1])
    t2 = time.time()
    for i in range(NEW_TOKENS):
        tok = orc.decode(tok, lg)
        toks[i] = tok
        dig[i] = sha(lg)
        top_ids[i], top_bits[i] = top16(lg)
        if i % 8 == 7:
            print(f"decode step {i + 1}/{NEW_TOKENS} ({time.time() - t2:.0f} s)", flush=True)
    decode_s = time.time() - t2
    kv = np.stack([sha(*orc.read_kv(l)) for l in range(cfg["num_layers"])])
    hidden = sha(orc.last_hidden())
    np.savez_compressed(
        OUT, tokens=toks, logits_sha256=dig, top16_ids=top_ids, top16_bits=top_bits, kv_sha256=kv,
        hidden_sha256=hidden, weights_sha256=wd, cache_len=np.uint64(orc.cache_len()),
        prompt_len=np.uint32(PROMPT_LEN), weight_seed=np.uint32(WEIGHT_SEED), prompt_seed=np.uint32(PROMPT_SEED),
        oracle_seconds=np.array([prefill_s, decode_s]), oracle_threads=np.uint32(args.threads))
    print(f"wrote {OUT}: {len(set(toks.tolist()))} distinct ids in {NEW_TOKENS} steps; "
          f"oracle prefill {prefill_s:.0f} s, decode {decode_s:.0f} s on {args.threads} threads", flush=True)


if __name__ == "__main__":
    main()
