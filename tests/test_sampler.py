"""The FP16 sampler (kernel_nn.cpp:446-651).

CPU: the oracle (oracle/sample_oracle.c) on known answers that follow from
the reference's code by hand: MT19937's values fixed by the C++ standard,
greedy unchanged, the repetition penalty (x 1/1.1 for positive, x 1.1 for
negative logits, once per history entry) flipping a top-1 choice on a
computed schedule, temperature on two-token distributions with known
probabilities, the reference's top-p cut (the entry that crosses top_p is
removed too) on 0.5/0.3/0.2, and the 128-entry history.

GPU: cactus_hip_sample_f16 against the oracle over consecutive draws that
share the history: identical tokens and identical histories for
temperature / top-k / top-p mixes on 151936-entry and tied logits.
"""
import ctypes
import math

import numpy as np
import pytest

from _data import f16


def say(*a):
    print("[case]", *a, flush=True)


def _seed_where(orc, lo, hi):
    """a seed whose draw u lies in (lo, hi)"""
    for s in range(1, 10000):
        u = orc.sample_uniform(s)
        if lo < u < hi:
            return s
    raise AssertionError("no seed")


# ------------------------------------------------------------------ CPU
def test_mt19937_standard_values(orc):
    """[rand.predef]: the 10000th output of default-seeded std::mt19937 is
    4123659995; its first is 3499211612."""
    assert orc.mt19937_nth(5489, 1) == 3499211612
    assert orc.mt19937_nth(5489, 10000) == 4123659995
    x = orc.mt19937_nth(7, 1)
    assert orc.sample_uniform(7) == np.float32(np.float32(x) / np.float32(2.0 ** 32))


def test_greedy_is_argmax_and_keeps_no_history(orc):
    s = orc.OracleSampler()
    x = f16([0.5, 2.0, 2.0, -1.0])
    assert s.sample(x, 0.0, 0.0, 0, 3) == 1
    assert len(s.history()) == 0


@pytest.mark.parametrize("logits,want", [([2.0, 1.95], [0, 1, 0, 1, 0]), ([-1.0, -1.05], [0, 1, 0, 1, 0])])
def test_repetition_penalty_schedule(orc, logits, want):
    """top-1 after the penalty: 2.0 -> 2.0*fp16(1/1.1) = 1.818 < 1.95 flips
    to token 1, then 1.95 -> 1.773 < 1.818 flips back, ...; negative logits
    are multiplied by fp16(1.1) instead."""
    s = orc.OracleSampler()
    got = [s.sample(f16(logits), 1.0, 0.0, 1, 11) for _ in range(len(want))]
    assert got == want
    assert list(s.history()) == want


@pytest.mark.parametrize("T,p0", [(1.0, 0.25), (0.5, 0.1)])
def test_temperature_two_tokens(orc, T, p0):
    """logits (0, ln 3): p = (1/4, 3/4) at T = 1 and (1/10, 9/10) at T = 1/2;
    draws well inside either side of p0 pick token 0 or 1."""
    x = f16([0.0, math.log(3.0)])
    s0, s1 = _seed_where(orc, 0.02, p0 - 0.03), _seed_where(orc, p0 + 0.03, 0.98)
    assert orc.OracleSampler().sample(x, T, 0.0, 0, s0) == 0
    assert orc.OracleSampler().sample(x, T, 0.0, 0, s1) == 1


def test_top_p_removes_the_crossing_entry(orc):
    """p = (0.5, 0.3, 0.2): top_p 0.7 -> the running sum 0.8 at the second
    entry crosses, which is removed too: only token 0 is left; top_p 0.85 ->
    tokens 0 and 1 stay with (0.625, 0.375)."""
    x = f16(np.log([0.5, 0.3, 0.2]))
    for seed in (1, 2, 3, 4, 5):
        assert orc.OracleSampler().sample(x, 1.0, 0.7, 3, seed) == 0
    s0, s1 = _seed_where(orc, 0.05, 0.58), _seed_where(orc, 0.68, 0.95)
    assert orc.OracleSampler().sample(x, 1.0, 0.85, 3, s0) == 0
    assert orc.OracleSampler().sample(x, 1.0, 0.85, 3, s1) == 1


def test_history_keeps_the_last_128(orc):
    s = orc.OracleSampler()
    rng = np.random.default_rng(3)
    got = []
    for i in range(135):
        x = f16(rng.normal(0, 1, 300))
        got.append(s.sample(x, 1.0, 0.0, 1, i + 1))
    assert list(s.history()) == got[-128:]


def test_all_masked_returns_zero_without_history(orc):
    s = orc.OracleSampler()
    x = np.full(8, 0xFC00, np.uint16)   # every logit -inf
    assert s.sample(x, 1.0, 0.0, 0, 5) == 0
    assert len(s.history()) == 0


# ------------------------------------------------------------------ GPU
def _gpu_sampler(cm):
    out = cm.DeviceBuffer(4)

    def run(logits, T, top_p, top_k, seed):
        d = cm.DeviceBuffer.from_numpy(np.ascontiguousarray(logits, dtype=np.uint16))
        rc = cm.hip().cactus_hip_sample_f16(d.ptr, out.ptr, logits.size, ctypes.c_float(T), ctypes.c_float(top_p),
                                            top_k, seed, None)
        if rc:
            d.free()
            return rc, None
        cm.call("cactus_hip_stream_sync", None)
        t = int(out.to_numpy(np.uint32, (1,))[0])
        d.free()
        return 0, t

    def history():
        buf = np.zeros(128, np.uint32)
        n = ctypes.c_size_t()
        cm.call("cactus_hip_sample_history", buf.ctypes.data, ctypes.byref(n), None)
        return buf[:n.value].copy()

    return run, history


CONFIGS = [
    # (temperature, top_p, top_k)
    (0.6, 0.95, 20),
    (1.0, 0.9, 50),
    (1.7, 0.5, 4096),
    (0.8, 0.0, 40),
    (1.0, 0.0, 1),
    (0.7, 0.0, 0),
    (0.0, 0.8, 10),
    (1.0, 0.9, 0),       # top-p over the whole vocabulary
    (2.5, 0.95, 0),      # flat: most of the vocabulary reaches top-p
    (1.2, 0.8, 20000),   # top-k above the LDS sort
]


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [151936, 1000])
@pytest.mark.parametrize("cfg", CONFIGS)
def test_sampler_matches_oracle(hip_ready, orc, vocab, cfg):
    """40 consecutive draws with the history carried: the device sampler and
    the oracle pick the same tokens and keep the same history.  Every draw
    has fresh logits; every fifth repeats the previous ones so the
    repetition penalty decides."""
    cm = hip_ready
    T, top_p, top_k = cfg
    run, history = _gpu_sampler(cm)
    cm.call("cactus_hip_sample_history_reset", None)
    s = orc.OracleSampler()
    rng = np.random.default_rng(vocab + int(T * 10) + top_k)
    say("sampler", vocab, cfg)
    x = None
    for step in range(40):
        if x is None or step % 5:
            x = f16(rng.normal(0, 2.5, vocab))
        seed = int(rng.integers(1, 2**31))
        rc, got = run(x, T, top_p, top_k, seed)
        assert rc == 0
        want = s.sample(x, T, top_p, top_k, seed)
        assert got == want, (step, got, want)
    assert (history() == s.history()).all()


@pytest.mark.gpu
def test_sampler_ties(hip_ready, orc):
    """Logits on a coarse grid (many exact ties): top-k keeps every tie of
    the k-th value; the top-p order of ties is the oracle's (ascending
    token)."""
    cm = hip_ready
    run, history = _gpu_sampler(cm)
    cm.call("cactus_hip_sample_history_reset", None)
    s = orc.OracleSampler()
    rng = np.random.default_rng(21)
    say("sampler ties")
    for step in range(30):
        x = f16(np.round(rng.normal(0, 2, 5000) * 2) / 2)
        seed = int(rng.integers(1, 2**31))
        for cfg in ((1.0, 0.9, 30), (0.5, 0.0, 7), (1.3, 0.6, 100)):
            rc, got = run(x, *cfg, seed)
            assert rc == 0
            assert got == s.sample(x, *cfg, seed), (step, cfg)
    assert (history() == s.history()).all()


@pytest.mark.gpu
def test_sampler_large_top_p(hip_ready, orc):
    """More top-p candidates than the LDS sort holds (16384): top-p with
    top_k 0 on 151936 logits, a flat row of 20000 ties (top-k 10 keeps every
    tie), ties straddling the cut on a coarse grid and a draw past a
    repetition-penalised token: the oracle's token every time, never an
    invalid id."""
    cm = hip_ready
    run, history = _gpu_sampler(cm)
    cm.call("cactus_hip_sample_history_reset", None)
    s = orc.OracleSampler()
    rng = np.random.default_rng(41)
    cases = [(f16(rng.normal(0, 1, 151936)), (1.0, 0.9, 0)),
             (f16(np.zeros(20000)), (1.0, 0.9, 10)),
             (f16(np.zeros(20000)), (1.0, 0.3, 0)),
             (f16(np.round(rng.normal(0, 1, 151936) * 4) / 4), (1.0, 0.7, 0)),
             (f16(np.round(rng.normal(0, 1, 60000) * 2) / 2), (3.0, 0.5, 40000))]
    for i, (x, cfg) in enumerate(cases):
        for rep in range(3):
            say("sampler large top-p", i, cfg, rep)
            seed = int(rng.integers(1, 2**31))
            rc, got = run(x, *cfg, seed)
            assert rc == 0
            assert got < x.size
            assert got == s.sample(x, *cfg, seed), (i, cfg, rep)
    assert (history() == s.history()).all()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_qwen_sampled_decode_matches_oracle(hip_ready, orc, mode):
    """Model::decode with temperature 0.8, top-p 0.9, top-k 40 and a fixed
    seed: the engine's tokens equal the oracle model's logits drawn through
    the oracle sampler step by step (the history carried across steps)."""
    from _data import qwen_small_config, qwen_weights
    from cactus_amd.engine import Qwen
    cm = hip_ready
    cfg = qwen_small_config(vocab=1024)
    rng = np.random.default_rng(31 + mode)
    w = qwen_weights(rng, cfg)
    prompt = rng.integers(0, cfg["vocab"], 50).astype(np.uint32)
    say("qwen sampled decode mode", mode)
    gpu = Qwen(cfg, *w)
    gpu.set_decode_mode(mode)
    gpu.set_sampling(0.8, 0.9, 40, 1234)
    cm.call("cactus_hip_sample_history_reset", None)
    toks, _ = gpu.generate(prompt, 12)
    m = orc.OracleQwen(cfg, *w)
    s = orc.OracleSampler()
    m.prefill(prompt[:-1], cfg["prefill_chunk"])
    tok, want = int(prompt[-1]), []
    logits = np.zeros(cfg["vocab"], np.uint16)
    for _ in range(12):
        m.decode(tok, logits)
        tok = s.sample(logits, 0.8, 0.9, 40, 1234)
        want.append(tok)
    assert list(toks) == want
    # the sampling path ran (greedy decoding records no history)
    _, history = _gpu_sampler(cm)
    assert list(history()) == list(s.history()) and len(s.history()) == 12


# ------------------------------------------------------------------ entropy
def test_entropy_closed_forms(orc):
    """engine_model.cpp:255-290: uniform logits -> 1; two live tokens (the
    rest -inf) -> log 2 / log V; one live token -> 0."""
    V = 1000
    assert orc.logits_entropy(f16(np.full(V, 0.37))) == np.float32(1.0)
    two = np.full(V, 0xFC00, np.uint16)
    two[[3, 700]] = f16([1.5, 1.5])
    assert abs(orc.logits_entropy(two) - math.log(2) / math.log(V)) < 1e-7
    one = np.full(V, 0xFC00, np.uint16)
    one[5] = f16([2.0])[0]
    assert orc.logits_entropy(one) == 0.0


def _ulps(a, b):
    return abs(int(np.float32(a).view(np.int32)) - int(np.float32(b).view(np.int32)))


@pytest.mark.gpu
@pytest.mark.parametrize("V,sd", [(151936, 2.0), (151936, 0.02), (1000, 5.0)])
def test_entropy_matches_oracle(hip_ready, orc, V, sd):
    """Floating point: within 2 float ulp of the oracle's sequential double
    sums (the device sums in a tree)."""
    cm = hip_ready
    x = f16(np.random.default_rng(V + int(sd * 100)).normal(0, sd, V))
    d = cm.DeviceBuffer.from_numpy(x)
    e = cm.DeviceBuffer(4)
    say("entropy", V, sd)
    cm.call("cactus_hip_logits_entropy_f16", d.ptr, V, e.ptr, None)
    got = float(e.to_numpy(np.float32, (1,))[0])
    assert _ulps(got, orc.logits_entropy(x)) <= 2, (got, orc.logits_entropy(x))


@pytest.mark.gpu
def test_qwen_last_entropy(hip_ready, orc):
    """The decode step's entropy (mode 0 keeps the logits) against the
    oracle's entropy of the oracle model's logits."""
    from _data import qwen_small_config, qwen_weights
    from cactus_amd.engine import Qwen
    cfg = qwen_small_config(vocab=1024)
    rng = np.random.default_rng(41)
    w = qwen_weights(rng, cfg)
    prompt = rng.integers(0, cfg["vocab"], 30).astype(np.uint32)
    say("qwen last entropy")
    gpu = Qwen(cfg, *w)
    gpu.prefill(prompt[:-1])
    gpu.decode(int(prompt[-1]))
    m = orc.OracleQwen(cfg, *w)
    m.prefill(prompt[:-1], cfg["prefill_chunk"])
    logits = np.zeros(cfg["vocab"], np.uint16)
    m.decode(int(prompt[-1]), logits)
    assert (gpu.last_logits() == logits).all()
    assert _ulps(gpu.last_entropy(), orc.logits_entropy(logits)) <= 2
