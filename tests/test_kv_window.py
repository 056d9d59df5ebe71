"""INT8 KV cache with sliding window and attention sinks (engine_cache.cpp).

CPU: the oracle's restatement (oracle/kv_oracle.c) against the reference's
own cases in tests/test_kv_cache.cpp (lengths, totals, sink preservation,
reset, a 600-token first update into a 512 window) and against a
brute-force model of what the cache must hold: the first `sink` rows of the
sequence followed by its most recent `window - sink` rows, each quantized
per token (kernel a7), with the reference's one quirk pinned separately: a
first update longer than the window on window-sized storage does not
rewrite the sinks (engine_cache.cpp:167-197).

GPU: the engine's device cache (cactus_hip_kv_window_shift and the graph
path's update) and the windowed Qwen model in both decode modes against
the oracle: identical tokens, bit-identical caches.
"""
import numpy as np
import pytest

from _data import f16, qwen_small_config, qwen_weights


def say(*a):
    print("[case]", *a, flush=True)


def _const_rows(n, kvh, hd, value):
    return np.full((n, kvh, hd), np.float16(value)).view(np.uint16)


def _quant(orc, rows):
    return orc.quantize_kv(rows)


# ------------------------------------------------------------------ CPU: reference cases
def test_reference_sliding_window_basic(orc):
    """test_kv_cache.cpp:21-130."""
    kv = orc.OracleKV(2, 2048, 8, 64)
    kv.set_window(16, 4)
    assert kv.update([_const_rows(10, 8, 64, l + 1.0) for l in range(2)],
                     [_const_rows(10, 8, 64, l + 2.0) for l in range(2)]) == 0
    assert kv.len() == 10
    assert kv.update([_const_rows(6, 8, 64, l + 10.0) for l in range(2)],
                     [_const_rows(6, 8, 64, l + 20.0) for l in range(2)]) == 0
    assert kv.len() == 16
    assert kv.update([_const_rows(10, 8, 64, 100.0)] * 2, [_const_rows(10, 8, 64, 100.0)] * 2) == 0
    assert kv.len() == 16 and kv.total() == 26
    k, _, ks, _ = kv.layer(0)
    expected = int(np.round(1.0 / ks[0, 0, 0]))
    assert (np.abs(k.reshape(-1)[:8].astype(int) - expected) <= 2).all()


def test_reference_incremental_updates(orc):
    """test_kv_cache.cpp:132-178 (single-token steps, window 8, sink 2)."""
    kv = orc.OracleKV(1, 2048, 4, 32)
    kv.set_window(8, 2)
    for t in range(12):
        assert kv.update([_const_rows(1, 4, 32, t + 1.0)], [_const_rows(1, 4, 32, t + 101.0)]) == 0
        assert kv.len() == min(t + 1, 8)
    assert kv.len() == 8 and kv.total() == 12


def test_reference_reset(orc):
    """test_kv_cache.cpp:180-215."""
    kv = orc.OracleKV(2, 1024, 8, 64)
    kv.set_window(16, 4)
    rows = [_const_rows(10, 8, 64, 1.0)] * 2
    assert kv.update(rows, rows) == 0
    assert (kv.len(), kv.total()) == (10, 10)
    kv.reset()
    assert (kv.len(), kv.total()) == (0, 0)


def test_reference_large_window(orc):
    """test_kv_cache.cpp:217-254: one 600-token update into a 512 window."""
    kv = orc.OracleKV(4, 2048, 8, 64)
    kv.set_window(512, 4)
    assert kv.update([_const_rows(600, 8, 64, l + 1.0) for l in range(4)],
                     [_const_rows(600, 8, 64, l + 101.0) for l in range(4)]) == 0
    assert (kv.len(), kv.total()) == (512, 600)


# ------------------------------------------------------------------ CPU: brute force
def _expected(orc, hist_k, hist_v, window, sink, zero_sinks=None):
    """Cache content after the history: all rows while it fits, else the first
    `sink` rows and the last window - sink rows (or the stale sink slots)."""
    n = len(hist_k)
    if window == 0 or n <= window:
        idx = list(range(n))
    else:
        idx = list(range(sink)) + list(range(n - (window - sink), n))
    k = np.stack([hist_k[i] for i in idx])
    v = np.stack([hist_v[i] for i in idx])
    kc, kscale = _quant(orc, k)
    vc, vscale = _quant(orc, v)
    if zero_sinks is not None:
        kc[:sink], vc[:sink] = zero_sinks[0], zero_sinks[1]
        kscale[:sink], vscale[:sink] = zero_sinks[2], zero_sinks[3]
    return kc, vc, kscale, vscale


@pytest.mark.parametrize("seed", range(6))
def test_window_keeps_sinks_and_recent_rows(orc, seed):
    rng = np.random.default_rng(seed)
    layers, kvh, hd = 2, 2, 128
    window = int(rng.integers(12, 40))
    sink = int(rng.integers(0, 5))
    kv = orc.OracleKV(layers, 64, kvh, hd)
    kv.set_window(window, sink)
    hist = [[[], []] for _ in range(layers)]
    first = int(rng.integers(1, window + 1))        # a first update that fits the window
    sizes = [first] + [int(rng.integers(1, window - sink + 1)) for _ in range(12)]
    for n in sizes:
        ks = [f16(rng.normal(0, 1 + l, (n, kvh, hd))) for l in range(layers)]
        vs = [f16(rng.normal(0, 2 + l, (n, kvh, hd))) for l in range(layers)]
        assert kv.update(ks, vs) == 0
        for l in range(layers):
            hist[l][0].extend(list(ks[l]))
            hist[l][1].extend(list(vs[l]))
        total = len(hist[0][0])
        assert kv.total() == total and kv.len() == min(total, window)
        for l in range(layers):
            want = _expected(orc, hist[l][0], hist[l][1], window, sink)
            for a, b in zip(kv.layer(l), want):
                assert (a == b).all(), (seed, n, l)


def test_first_update_longer_than_window(orc):
    """engine_cache.cpp:167-197: on storage already window-sized (fresh
    set_window_size, or a previous slide) the sinks are not rewritten; after
    a shorter update resized the storage they are."""
    rng = np.random.default_rng(7)
    kvh, hd, W, S = 2, 64, 16, 4
    rows = lambda n: f16(rng.normal(0, 1, (n, kvh, hd)))  # noqa: E731
    kv = orc.OracleKV(1, 64, kvh, hd)
    kv.set_window(W, S)
    k1, v1 = rows(20), rows(20)
    assert kv.update([k1], [v1]) == 0
    stale = (np.zeros((S, kvh, hd), np.int8), np.zeros((S, kvh, hd), np.int8),
             np.ones((S, kvh, 1), np.float32), np.ones((S, kvh, 1), np.float32))
    want = _expected(orc, list(k1), list(v1), W, S, zero_sinks=stale)
    for a, b in zip(kv.layer(0), want):
        assert (a == b).all()
    # reset, long first update again: the previous sequence's slots stay
    kv.reset()
    k2, v2 = rows(30), rows(30)
    assert kv.update([k2], [v2]) == 0
    got = kv.layer(0)
    want2 = _expected(orc, list(k2), list(v2), W, S, zero_sinks=tuple(x[:S] for x in want))
    for a, b in zip(got, want2):
        assert (a == b).all()
    # a short update resizes the storage below the window: the next long
    # first update writes its own sinks
    kv.reset()
    k3, v3 = rows(5), rows(5)
    assert kv.update([k3], [v3]) == 0
    kv.reset()
    k4, v4 = rows(25), rows(25)
    assert kv.update([k4], [v4]) == 0
    for a, b in zip(kv.layer(0), _expected(orc, list(k4), list(v4), W, S)):
        assert (a == b).all()


def test_undefined_sliding_step_is_refused(orc):
    """window - sink - seq wraps in the reference's size_t arithmetic when a
    step is longer than window - sink (engine_cache.cpp:268-270)."""
    kv = orc.OracleKV(1, 64, 2, 64)
    kv.set_window(16, 4)
    assert kv.update([_const_rows(10, 2, 64, 1.0)], [_const_rows(10, 2, 64, 1.0)]) == 0
    assert kv.update([_const_rows(13, 2, 64, 1.0)], [_const_rows(13, 2, 64, 1.0)]) == -1
    assert kv.update([_const_rows(12, 2, 64, 1.0)], [_const_rows(12, 2, 64, 1.0)]) == 0
    assert kv.len() == 16


def test_no_window_grows_without_limit(orc):
    kv = orc.OracleKV(1, 8, 2, 64)
    for _ in range(5):
        assert kv.update([_const_rows(7, 2, 64, 1.0)], [_const_rows(7, 2, 64, 2.0)]) == 0
    assert kv.len() == kv.total() == 35


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
@pytest.mark.parametrize("dst,src,count", [(4, 5, 27), (2, 40, 20), (0, 9, 30), (3, 3, 10), (7, 8, 0)])
def test_kv_window_shift_matches_memmove(hip_ready, dst, src, count):
    """cactus_hip_kv_window_shift against numpy's memmove of every layer, the
    moved tokens' value products against kv_shadow_update of the result, and
    the step state's cache length."""
    import ctypes
    cm = hip_ready
    rng = np.random.default_rng(dst * 100 + src + count)
    layers, cap, kvh, hd = 3, 70, 2, 128
    say("kv_window_shift", dst, src, count)
    keep, recs, host = [], [], []
    nbytes = ctypes.c_size_t()
    cm.call("cactus_hip_kv_shadow_bytes", cap, kvh, hd, ctypes.byref(nbytes))
    for _ in range(layers):
        h = dict(k=rng.integers(-127, 128, (cap, kvh, hd), dtype=np.int8),
                 v=rng.integers(-127, 128, (cap, kvh, hd), dtype=np.int8),
                 ks=np.abs(rng.normal(0, 0.01, (cap, kvh, 1))).astype(np.float32),
                 vs=np.abs(rng.normal(0, 0.01, (cap, kvh, 1))).astype(np.float32))
        d = {n: cm.DeviceBuffer.from_numpy(a) for n, a in h.items()}
        d["sh"] = cm.DeviceBuffer(nbytes.value)
        cm.call("cactus_hip_kv_shadow_update", d["v"].ptr, d["vs"].ptr, d["sh"].ptr, 0, cap, kvh, hd, 128, cap,
                None)
        host.append(h)
        keep.append(d)
        recs += [d["k"].ptr, d["v"].ptr, d["ks"].ptr, d["vs"].ptr, d["sh"].ptr]
    table = cm.DeviceBuffer.from_numpy(np.array(recs, np.uint64))
    tb = ctypes.c_size_t()
    cm.call("cactus_hip_kv_shift_temp_bytes", layers, count, kvh, hd, ctypes.byref(tb))
    temp = cm.DeviceBuffer(max(tb.value, 1))
    state = cm.DeviceBuffer.from_numpy(np.array([9, 99, 5, 0], np.uint32))
    cm.call("cactus_hip_kv_window_shift", table.ptr, layers, kvh, hd, cap, dst, src, count, temp.ptr, tb.value,
            state.ptr, 42, None)
    cm.call("cactus_hip_stream_sync", None)
    assert list(state.to_numpy(np.uint32, (4,))) == [9, 99, 42, 0]
    for h, d in zip(host, keep):
        for n in ("k", "v", "ks", "vs"):
            want = h[n].copy()
            want[dst:dst + count] = h[n][src:src + count]
            assert (d[n].to_numpy(want.dtype, want.shape) == want).all(), n
        # value products of the moved tokens equal a fresh computation
        ref = cm.DeviceBuffer(nbytes.value)
        cm.call("cactus_hip_kv_shadow_update", d["v"].ptr, d["vs"].ptr, ref.ptr, 0, cap, kvh, hd, 128, cap, None)
        # [kv head x 64-dim slice][key / 4][64 dims][4 keys]: only keys below
        # the capacity are ever written
        def keys(buf):
            a = buf.to_numpy(np.float32, (nbytes.value // 4,)).reshape(kvh * 2, -1, 64, 4)
            return a.transpose(0, 2, 1, 3).reshape(kvh * 2, 64, -1)[:, :, :cap]
        assert (keys(d["sh"]).view(np.uint32) == keys(ref).view(np.uint32)).all()
        ref.free()


def _windowed_pair(cfg, window, sink, mode, seed):
    import oracle
    from cactus_amd.engine import Qwen
    rng = np.random.default_rng(seed)
    layers, emb, on = qwen_weights(rng, cfg)
    gpu = Qwen(cfg, layers, emb, on)
    gpu.set_kv_window(window, sink)
    if mode:
        gpu.set_decode_mode(mode)
    orc = oracle.OracleQwen(cfg, layers, emb, on)
    orc.set_window(window, sink)
    return gpu, orc, rng


def _check_same(gpu, orc, cfg, toks, ref, mode):
    assert list(toks) == list(ref)
    assert gpu.cache_len() == orc.cache_len()
    if mode == 0:
        assert (gpu.last_hidden() == orc.last_hidden()).all()
    for layer in range(cfg["num_layers"]):
        for a, b in zip(gpu.read_kv(layer), orc.read_kv(layer)):
            assert (a == b).all(), f"kv cache layer {layer}"


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_windowed_qwen_slides_in_prefill_and_decode(hip_ready, mode):
    """Window 300 with 4 sinks over a 320-token context: the second and third
    prefill chunks slide (256 and 87 new tokens), every decode step slides,
    and positions run past the context size."""
    cfg = qwen_small_config(max_seq=320, vocab=1024)
    gpu, orc, rng = _windowed_pair(cfg, 300, 4, mode, 11)
    prompt = rng.integers(0, cfg["vocab"], 600).astype(np.uint32)
    say("windowed qwen 300/4 prompt 600 mode", mode)
    toks, _ = gpu.generate(prompt, 30)
    ref = orc.generate(prompt, 30, cfg["prefill_chunk"])
    _check_same(gpu, orc, cfg, toks, ref, mode)
    assert gpu.cache_len() == 300 and gpu.total_len() == 599 + 30


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [0, 1])
def test_windowed_qwen_first_chunk_longer_than_window(hip_ready, mode):
    """A 200-token first chunk into a fresh 100-token window leaves the sink
    slots as set_window_size wrote them (engine_cache.cpp:167-197); after a
    reset the next long first chunk keeps the previous sequence's slots."""
    cfg = qwen_small_config(vocab=1024)
    gpu, orc, rng = _windowed_pair(cfg, 100, 4, mode, 12)
    for rnd in range(2):
        prompt = rng.integers(0, cfg["vocab"], 201).astype(np.uint32)
        say("windowed qwen 100/4 prompt 201 mode", mode, "round", rnd)
        toks, _ = gpu.generate(prompt, 9)
        ref = orc.generate(prompt, 9, cfg["prefill_chunk"])
        _check_same(gpu, orc, cfg, toks, ref, mode)
        gpu.reset()
        orc.reset()


@pytest.mark.gpu
def test_window_larger_than_sequence_changes_nothing(hip_ready):
    """A window the sequence never fills gives the unwindowed results."""
    from cactus_amd.engine import Qwen
    cfg = qwen_small_config(vocab=1024)
    rng = np.random.default_rng(13)
    w = qwen_weights(rng, cfg)
    prompt = rng.integers(0, cfg["vocab"], 90).astype(np.uint32)
    say("window 512 over 100 tokens")
    a = Qwen(cfg, *w)
    b = Qwen(cfg, *w)
    b.set_kv_window(512, 4)
    ta, _ = a.generate(prompt, 10)
    tb, _ = b.generate(prompt, 10)
    assert list(ta) == list(tb)
    for layer in range(cfg["num_layers"]):
        for x, y in zip(a.read_kv(layer), b.read_kv(layer)):
            assert (x == y).all()


@pytest.mark.gpu
def test_window_rejects_undefined_steps(hip_ready):
    """A chunk longer than window - sink into a full window is refused (the
    reference's arithmetic wraps); windows larger than the context too."""
    from cactus_amd.engine import Qwen
    from cactus_amd import NativeError
    cfg = qwen_small_config(vocab=1024)
    rng = np.random.default_rng(14)
    m = Qwen(cfg, *qwen_weights(rng, cfg))
    with pytest.raises(NativeError, match="exceeds the cache capacity"):
        m.set_kv_window(cfg["max_seq"] + 1, 4)
    m.set_kv_window(200, 4)
    say("window 200/4, prompt 300")
    m.prefill(rng.integers(0, cfg["vocab"], 150).astype(np.uint32))
    with pytest.raises(NativeError, match="must not exceed window - sink"):
        m.prefill(rng.integers(0, cfg["vocab"], 250).astype(np.uint32))
