"""The FP32 sampler (kernel_nn.cpp:253-444): the variant with the logit bias
and min-p.

CPU: the oracle (orc_sample_f32 in oracle/sample_oracle.c) on answers that
follow from the reference's code by hand: the greedy branch takes the first
maximum and ignores the bias; the bias is added and kept (the FP16 sampler
drops it); min-p 0.15 removes a token whose probability is below 0.15 of the
largest and keeps one above it; the top-p cut on 0.5/0.3/0.2 (the crossing
entry is removed, position 0 never is); top-k keeps ties; an infinite
maximum or an all-masked vector returns 0; and over many seeds the draw
reproduces the filtered distribution (a chi-square bound).

GPU: cactus_hip_sample_f32 against the oracle on 151936- and 1000-entry
logits for temperature / top-k / top-p mixes with and without a bias,
tied logits, and the refusals.
"""
import ctypes
import math

import numpy as np
import pytest


def say(*a):
    print("[case]", *a, flush=True)


def _seed_where(orc, lo, hi):
    """a seed whose draw u lies in (lo, hi)"""
    for s in range(1, 20000):
        u = orc.sample_uniform(s)
        if lo < u < hi:
            return s
    raise AssertionError("no seed")


def f32(x):
    return np.asarray(x, np.float32)


# ------------------------------------------------------------------ CPU
def test_greedy_first_maximum_ignores_bias(orc):
    x = f32([1.0, 3.0, 2.0, 3.0])
    assert orc.sample_f32(x, 0.0, 0.0, 0, 5) == 1
    assert orc.sample_f32(x, 0.0, 0.0, 0, 5, {0: 10.0}) == 1


def test_bias_is_kept(orc):
    """Three equal logits and +10 on token 2: after min-p only token 2 is
    left (e^-10 of the largest probability), whatever the draw."""
    x = f32([0.0, 0.0, 0.0])
    for seed in (1, 2, 3, 99, 12345):
        assert orc.sample_f32(x, 1.0, 0.0, 0, seed, {2: 10.0}) == 2
    # a bias entry per occurrence, in order: -5 then +15 on token 1
    assert orc.sample_f32(x, 1.0, 0.0, 0, 7, [(1, -5.0), (1, 15.0)]) == 1


@pytest.mark.parametrize("ratio,survives", [(0.16, True), (0.14, False)])
def test_min_p_threshold(orc, ratio, survives):
    """Two tokens with probabilities in the ratio r : 1.  A draw above the
    first token's share picks token 1 only if r >= 0.15 keeps it."""
    x = f32([0.0, math.log(ratio)])
    p0 = 1.0 / (1.0 + ratio)
    seed = _seed_where(orc, p0 + 0.01, 1.0)
    assert orc.sample_f32(x, 1.0, 0.0, 0, seed) == (1 if survives else 0)
    seed = _seed_where(orc, 0.0, p0 - 0.01)
    assert orc.sample_f32(x, 1.0, 0.0, 0, seed) == 0


def test_top_p_cut(orc):
    """0.5 / 0.3 / 0.2 (all above min-p): top_p 0.6 leaves token 0 only,
    0.9 leaves tokens 0 and 1, 0.4 (crossing at position 0) token 0."""
    x = f32(np.log([0.5, 0.3, 0.2]))
    hi = _seed_where(orc, 0.97, 1.0)
    mid = _seed_where(orc, 0.7, 0.75)
    assert orc.sample_f32(x, 1.0, 0.6, 0, hi) == 0
    assert orc.sample_f32(x, 1.0, 0.4, 0, hi) == 0
    assert orc.sample_f32(x, 1.0, 0.9, 0, hi) == 1        # renormalised over 0.5 + 0.3
    assert orc.sample_f32(x, 1.0, 0.9, 0, mid) == 1       # u > 0.5 / 0.8
    # the running sum reaches ~1.0 > 0.99 at position 2: removed as well
    assert orc.sample_f32(x, 1.0, 0.99, 0, hi) == 1
    assert orc.sample_f32(x, 1.0, 0.0, 0, hi) == 2        # top-p off


def test_top_k_keeps_ties(orc):
    x = f32([3.0, 5.0, 5.0, 1.0])
    lo = _seed_where(orc, 0.0, 0.45)
    hi = _seed_where(orc, 0.55, 1.0)
    assert orc.sample_f32(x, 1.0, 0.0, 1, lo) == 1
    assert orc.sample_f32(x, 1.0, 0.0, 1, hi) == 2


def test_infinities(orc):
    assert orc.sample_f32(f32([0.0, np.inf, 1.0]), 1.0, 0.0, 0, 3) == 0
    assert orc.sample_f32(f32([-np.inf] * 4), 1.0, 0.0, 0, 3) == 0
    assert orc.sample_f32(f32([-np.inf, 2.0, -np.inf]), 1.0, 0.0, 0, 3) == 1


def test_draw_follows_the_distribution(orc):
    """p = (0.25, 0.25, 0.5) after every filter: 3000 seeds, chi-square with
    2 degrees of freedom below 13.8 (p = 0.001)."""
    x = f32(np.log([1.0, 1.0, 2.0]))
    counts = np.zeros(3)
    for seed in range(1, 3001):
        counts[orc.sample_f32(x, 1.0, 0.0, 0, seed)] += 1
    expect = 3000 * np.array([0.25, 0.25, 0.5])
    assert ((counts - expect) ** 2 / expect).sum() < 13.8


# ------------------------------------------------------------------ GPU
def _gpu_sampler_f32(cm):
    out = cm.DeviceBuffer(4)

    def run(logits, T, top_p, top_k, seed, bias=None):
        pairs = list(bias.items()) if isinstance(bias, dict) else list(bias or [])
        bi = np.array([t for t, _ in pairs], np.uint32)
        bv = np.array([v for _, v in pairs], np.float32)
        d = cm.DeviceBuffer.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
        rc = cm.hip().cactus_hip_sample_f32(d.ptr, out.ptr, logits.size, ctypes.c_float(T), ctypes.c_float(top_p),
                                            top_k, seed, bv.ctypes.data if pairs else None,
                                            bi.ctypes.data if pairs else None, len(pairs), None)
        if rc:
            d.free()
            return rc, None
        cm.call("cactus_hip_stream_sync", None)
        t = int(out.to_numpy(np.uint32, (1,))[0])
        d.free()
        return 0, t

    return run


CONFIGS = [
    # (temperature, top_p, top_k)
    (0.6, 0.95, 20),
    (1.0, 0.9, 0),
    (1.7, 0.5, 4096),
    (0.8, 0.0, 40),
    (1.0, 0.0, 1),
    (0.7, 0.0, 0),
    (0.0, 0.8, 10),
    (0.0, 0.0, 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [151936, 1000])
@pytest.mark.parametrize("cfg", CONFIGS)
def test_sampler_f32_matches_oracle(hip_ready, orc, vocab, cfg):
    """30 draws on fresh logits, every third with a logit bias of 1-40
    entries (duplicates included): the device picks the oracle's token."""
    cm = hip_ready
    T, top_p, top_k = cfg
    run = _gpu_sampler_f32(cm)
    rng = np.random.default_rng(vocab + int(T * 10) + top_k + 7)
    say("sampler_f32", vocab, cfg)
    for step in range(30):
        x = f32(rng.normal(0, 2.5, vocab))
        bias = None
        if step % 3 == 0:
            n = int(rng.integers(1, 41))
            bias = [(int(rng.integers(0, vocab)), float(rng.normal(0, 4))) for _ in range(n)]
            bias.append(bias[0])
        seed = int(rng.integers(1, 2**31))
        rc, got = run(x, T, top_p, top_k, seed, bias)
        assert rc == 0
        want = orc.sample_f32(x, T, top_p, top_k, seed, bias)
        assert got == want, (step, got, want)


@pytest.mark.gpu
def test_sampler_f32_ties_and_signed_zero(hip_ready, orc):
    """Logits on a coarse grid (many exact ties, +0 and -0 among them)."""
    cm = hip_ready
    run = _gpu_sampler_f32(cm)
    rng = np.random.default_rng(23)
    say("sampler_f32 ties")
    for step in range(20):
        x = f32(np.round(rng.normal(0, 2, 5000) * 2) / 2)
        x[rng.integers(0, 5000, 50)] = -0.0
        seed = int(rng.integers(1, 2**31))
        for cfg in ((1.0, 0.9, 30), (0.5, 0.0, 7), (1.3, 0.6, 0), (2.0, 0.0, 0)):
            rc, got = run(x, *cfg, seed)
            assert rc == 0
            assert got == orc.sample_f32(x, *cfg, seed), (step, cfg)


@pytest.mark.gpu
def test_sampler_f32_edges_and_refusals(hip_ready, orc):
    """Infinities and more than 128 bias entries (refused)."""
    cm = hip_ready
    run = _gpu_sampler_f32(cm)
    say("sampler_f32 edges")
    assert run(f32([0.0, np.inf, 1.0]), 1.0, 0.0, 0, 3) == (0, 0)
    assert run(f32([-np.inf] * 4), 1.0, 0.0, 0, 3) == (0, 0)
    assert run(f32([-np.inf, 2.0, -np.inf]), 1.0, 0.5, 2, 3) == (0, 1)
    x = f32(np.random.default_rng(2).normal(0, 1, 3000))
    assert run(x, 1.0, 0.0, 0, 1, [(i, 1.0) for i in range(129)])[0] == -2


@pytest.mark.gpu
def test_sampler_f32_large_top_p(hip_ready, orc):
    """More than 16384 entries reaching top-p (min-p keeps a flat row whole):
    20000 ties, a flat high-temperature row of 151936 logits and a coarse
    grid whose ties straddle the cut; the oracle's token every time."""
    cm = hip_ready
    run = _gpu_sampler_f32(cm)
    rng = np.random.default_rng(43)
    cases = [(f32(np.zeros(20000)), (1.0, 0.9, 0)),
             (f32(np.zeros(20000)), (1.0, 0.2, 0)),
             (f32(rng.normal(0, 0.05, 151936)), (4.0, 0.95, 0)),
             (f32(np.round(rng.normal(0, 0.1, 151936) * 20) / 20), (2.0, 0.6, 0)),
             (f32(rng.normal(0, 0.02, 80000)), (1.0, 0.5, 50000))]
    for i, (x, cfg) in enumerate(cases):
        for rep in range(3):
            say("sampler_f32 large top-p", i, cfg, rep)
            seed = int(rng.integers(1, 2**31))
            rc, got = run(x, *cfg, seed)
            assert rc == 0
            assert got < x.size
            assert got == orc.sample_f32(x, *cfg, seed), (i, cfg, rep)
