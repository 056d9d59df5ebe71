"""End-to-end parity of the Qwen3-architecture engine against the oracle:
identical greedy token ids, bit-identical final hidden states and INT8 KV
cache, over the reference's FFI flow (chunked prefill of prompt[:-1], then
decode from the last prompt token)."""
import sys

import numpy as np
import pytest

from _data import qwen_small_config, qwen_weights

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _run_both(cfg, prompt, steps, mode=0, weights=None, seed=None):
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    if weights is None:
        gpu = Qwen(cfg, seed=seed)
        layers, emb, on = gpu.read_weights()
    else:
        layers, emb, on = weights
        gpu = Qwen(cfg, layers, emb, on)
    if mode:
        gpu.set_decode_mode(mode)
    toks, _ = gpu.generate(prompt, steps)
    orc = oracle.OracleQwen(cfg, layers, emb, on)
    ref = orc.generate(prompt, steps, cfg["prefill_chunk"])
    return gpu, orc, toks, ref


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("prompt_len,steps", [(300, 16), (40, 8), (1, 4)])
def test_qwen_small_generate_matches_oracle(prompt_len, steps, mode):
    """mode 0: node-by-node graph decode; mode 1: fused kernels replayed as
    one HIP graph per token with the step state on the device."""
    say("qwen small", prompt_len, steps, "mode", mode)
    cfg = qwen_small_config()
    rng = np.random.default_rng(prompt_len)
    w = qwen_weights(rng, cfg)
    prompt = rng.integers(0, cfg["vocab"], prompt_len).astype(np.uint32)
    gpu, orc, toks, ref = _run_both(cfg, prompt, steps, mode=mode, weights=w)
    assert list(toks) == list(ref)
    assert gpu.cache_len() == orc.cache_len() == prompt_len - 1 + steps
    if mode == 0:
        assert (gpu.last_hidden() == orc.last_hidden()).all()
    for layer in range(cfg["num_layers"]):
        for a, b in zip(gpu.read_kv(layer), orc.read_kv(layer)):
            assert (a == b).all(), f"kv cache layer {layer}"


def test_qwen_random_init_and_logits():
    """Host random init (the bench's weights) read back and replayed by the
    oracle; logits of the last step bit-identical."""
    say("qwen random init")
    cfg = qwen_small_config(num_layers=3, vocab=4096, max_seq=400)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 270).astype(np.uint32)
    gpu, orc, toks, ref = _run_both(cfg, prompt, 6, seed=1234)
    assert list(toks) == list(ref)
    import oracle
    lg = np.zeros(cfg["vocab"], np.uint16)
    t_gpu = gpu.decode(int(toks[-1]))
    t_orc = orc.decode(int(ref[-1]), lg)
    assert t_gpu == t_orc
    assert (gpu.last_logits() == lg).all()


def test_qwen_fused_decode_continues_after_reset():
    """Fused decode, reset, a second prompt: the captured graph reads the
    new step state and cache length from the device."""
    say("qwen fused reset")
    cfg = qwen_small_config()
    rng = np.random.default_rng(11)
    w = qwen_weights(rng, cfg)
    p1 = rng.integers(0, cfg["vocab"], 70).astype(np.uint32)
    p2 = rng.integers(0, cfg["vocab"], 130).astype(np.uint32)
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    gpu = Qwen(cfg, *w)
    gpu.set_decode_mode(1)
    orc = oracle.OracleQwen(cfg, *w)
    for p, n in ((p1, 9), (p2, 12)):
        gpu.reset()
        orc.reset()
        toks, _ = gpu.generate(p, n)
        ref = orc.generate(p, n, cfg["prefill_chunk"])
        assert list(toks) == list(ref)
        # single steps through the same graph
        t_gpu = gpu.decode(int(toks[-1]))
        lg = np.zeros(cfg["vocab"], np.uint16)
        t_orc = orc.decode(int(ref[-1]), lg)
        assert t_gpu == t_orc
    for layer in range(cfg["num_layers"]):
        for a, b in zip(gpu.read_kv(layer), orc.read_kv(layer)):
            assert (a == b).all(), f"kv cache layer {layer}"


def test_qwen_prefill_rejects_out_of_range_token():
    """A prompt id at or past the vocabulary is refused with the reference's
    embedding error (graph_ops_tensor.cpp:256-263) before anything runs, and
    the model stays usable: the next prompt matches the oracle."""
    say("qwen out-of-range token")
    cfg = qwen_small_config()
    rng = np.random.default_rng(12)
    w = qwen_weights(rng, cfg)
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    gpu = Qwen(cfg, *w)
    bad = np.array([3, cfg["vocab"], 5], np.uint32)
    with pytest.raises(Exception, match="Embedding index out of bounds"):
        gpu.prefill(bad)
    gpu.reset()
    p = rng.integers(0, cfg["vocab"], 40).astype(np.uint32)
    toks, _ = gpu.generate(p, 4)
    ref = oracle.OracleQwen(cfg, *w).generate(p, 4, cfg["prefill_chunk"])
    assert list(toks) == list(ref)


def test_qwen_overlapped_prefill_rejects_bad_id_in_last_chunk():
    """A prompt long enough for the overlapped (three-stream) prefill whose
    out-of-range id sits in its last chunk: refused before any chunk is
    queued, the cache is left as it was, and a following prompt on the same
    model -- prefill onto the first prompt's cache, then greedy decode --
    matches the oracle bit for bit."""
    say("qwen overlapped prefill, bad id in the last chunk")
    cfg = qwen_small_config(prefill_chunk=32)
    rng = np.random.default_rng(21)
    w = qwen_weights(rng, cfg)
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    gpu = Qwen(cfg, *w)
    orc = oracle.OracleQwen(cfg, *w)
    first = rng.integers(0, cfg["vocab"], 70).astype(np.uint32)
    gpu.prefill(first)
    orc.prefill(first, 32)
    bad = rng.integers(0, cfg["vocab"], 100).astype(np.uint32)
    bad[-3] = cfg["vocab"] + 2
    with pytest.raises(Exception, match="Embedding index out of bounds"):
        gpu.prefill(bad)
    assert gpu.cache_len() == orc.cache_len() == 70
    good = rng.integers(0, cfg["vocab"], 100).astype(np.uint32)
    gpu.prefill(good)
    orc.prefill(good, 32)
    assert (gpu.last_hidden() == orc.last_hidden()).all(), "final hidden states"
    for layer in range(cfg["num_layers"]):
        for a, b in zip(gpu.read_kv(layer), orc.read_kv(layer)):
            assert (a == b).all(), f"kv cache layer {layer}"
    tok = int(rng.integers(0, cfg["vocab"]))
    for _ in range(4):
        t_gpu, t_orc = gpu.decode(tok), orc.decode(tok)
        assert t_gpu == t_orc
        tok = t_gpu


@pytest.mark.parametrize("chunk,lens", [(64, (150,)), (64, (200,)), (32, (70, 130))])
def test_qwen_overlapped_prefill_matches_oracle(chunk, lens):
    """Multi-chunk prompts run their chunks overlapped on three streams (chunk
    c + 1's layer-l attention ordered after chunk c's layer-l KV append):
    three and four chunks (the first on the third and on the second stream),
    and a second prompt prefilled onto a cache that already holds the first
    -- final hidden states, KV caches and the following greedy tokens
    bit-identical to the oracle's serial chunked prefill."""
    say("qwen overlapped prefill", chunk, lens)
    cfg = qwen_small_config(prefill_chunk=chunk)
    rng = np.random.default_rng(chunk + sum(lens))
    w = qwen_weights(rng, cfg)
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    gpu = Qwen(cfg, *w)
    orc = oracle.OracleQwen(cfg, *w)
    for n in lens:
        p = rng.integers(0, cfg["vocab"], n).astype(np.uint32)
        gpu.prefill(p)
        orc.prefill(p, chunk)
        assert (gpu.last_hidden() == orc.last_hidden()).all(), "final hidden states"
    assert gpu.cache_len() == orc.cache_len() == sum(lens)
    for layer in range(cfg["num_layers"]):
        for a, b in zip(gpu.read_kv(layer), orc.read_kv(layer)):
            assert (a == b).all(), f"kv cache layer {layer}"
    tok = int(rng.integers(0, cfg["vocab"]))
    for _ in range(4):
        t_gpu, t_orc = gpu.decode(tok), orc.decode(tok)
        assert t_gpu == t_orc
        tok = t_gpu


def test_qwen_tolerance_prefill_close_to_oracle():
    """Tolerance-mode prefill (the FP16-MFMA flash attention, 64-row chunks
    overlapped on three streams) of a 230-token prompt against the oracle's
    exact prefill, on a 4-layer model whose MLP down projection is small
    (group scales |N(0, 0.001)|/7), so that a layer passes on its attention's
    difference without the random MLP amplifying it.  Layer 0's KV cache,
    computed before any attention, must be bit-identical.  Measured on
    MI355X for the later layers: 69-85% of the INT8 codes equal, 97.5-99.9%
    within one step, no code more than 5 steps off, final hidden state 0.69%
    relative L2 from the oracle's.  Bounds with a margin: >= 60% equal,
    >= 96% within one step, <= 8 steps, <= 1.5%.  A wrong stream order,
    scale table or chunk offset moves whole rows and lands far outside."""
    say("qwen tolerance prefill vs oracle")
    cfg = qwen_small_config(prefill_chunk=64, num_layers=4)
    rng = np.random.default_rng(91)
    w = qwen_weights(rng, cfg, down_sd=0.001)
    import cactus_amd
    from cactus_amd.engine import Qwen
    import oracle
    cactus_amd.call("cactus_hip_init", 0)
    gpu = Qwen(cfg, *w)
    gpu.set_attention_mode(1)
    orc = oracle.OracleQwen(cfg, *w)
    p = rng.integers(0, cfg["vocab"], 230).astype(np.uint32)
    try:
        gpu.prefill(p)
    finally:
        gpu.set_attention_mode(0)
    orc.prefill(p, 64)
    assert gpu.cache_len() == orc.cache_len() == len(p)
    for a, b in zip(gpu.read_kv(0), orc.read_kv(0)):
        assert (a == b).all(), "kv cache layer 0"
    for layer in range(1, cfg["num_layers"]):
        kg, vg, _, _ = gpu.read_kv(layer)
        ko, vo, _, _ = orc.read_kv(layer)
        for nm, g_, o_ in (("k", kg, ko), ("v", vg, vo)):
            d = np.abs(g_.astype(np.int16) - o_.astype(np.int16))
            eq, one, step = float(np.mean(d == 0)), float(np.mean(d <= 1)), int(np.max(d))
            print(f"[tolerance prefill] layer {layer} {nm}: codes equal {eq:.4f}, within one step {one:.4f}, "
                  f"largest step {step}", flush=True)
            assert eq >= 0.60 and one >= 0.96 and step <= 8, (layer, nm, eq, one, step)
    hg = gpu.last_hidden().view(np.float16).astype(np.float64)
    ho = orc.last_hidden().view(np.float16).astype(np.float64)
    rel = float(np.linalg.norm(hg - ho) / np.linalg.norm(ho))
    print(f"[tolerance prefill] final hidden relative L2 {rel:.2e}", flush=True)
    assert rel <= 0.015, rel
