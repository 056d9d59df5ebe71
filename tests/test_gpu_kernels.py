"""GPU parity of every kernel-layer entry point against the oracle.

Each test prints the case it runs (flushed) before touching the GPU.  The bar
is bit-equality of every output (quantized codes, scales, fp16 results): the
HIP kernels follow the reference's order of operations exactly.
"""
import ctypes
import math
import sys

import numpy as np
import pytest

from _data import activations, f16, grouped_int4_weights, grouped_int8_weights

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


class Dev:
    """Small helper: numpy <-> device buffers through the C ABI."""

    def __init__(self, cm):
        self.cm = cm
        self.bufs = []

    def put(self, arr):
        b = self.cm.DeviceBuffer.from_numpy(np.ascontiguousarray(arr))
        self.bufs.append(b)
        return b.ptr

    def empty(self, nbytes):
        b = self.cm.DeviceBuffer(nbytes)
        self.bufs.append(b)
        return b

    def get(self, buf, dtype, shape):
        self.cm.call("cactus_hip_stream_sync", None)
        return buf.to_numpy(dtype, shape)

    def get_ptr(self, ptr, dtype, shape):
        """Copy of a buffer made by put (a raw device pointer)."""
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


def assert_bits(got, ref, what):
    got = np.asarray(got)
    ref = np.asarray(ref)
    bad = np.flatnonzero(got.ravel() != ref.ravel())
    assert bad.size == 0, f"{what}: {bad.size}/{ref.size} mismatches, first at {bad[:5]}: " \
                          f"got {got.ravel()[bad[:5]]} ref {ref.ravel()[bad[:5]]}"


# ------------------------------------------------------------------ a1
@pytest.mark.parametrize("M,K", [(1, 640), (1, 1024), (3, 1001), (512, 1024), (2, 3072), (2, 8192), (3, 8200)])
def test_quantize_activations(dev, orc, M, K):
    say("quantize_activations", M, K)
    rng = np.random.default_rng(M * 7 + K)
    x = activations(rng, M, K)
    x[0, :5] = f16([0.0, -0.0, 65504.0, -3.5, 1e-8])
    q = dev.empty(M * K)
    s = dev.empty(M * 4)
    dev.cm.call("cactus_hip_quantize_activations", dev.put(x), q.ptr, s.ptr, M, K, None)
    rq, rs = orc.quantize_activations(x)
    assert_bits(dev.get(s, np.float32, M).view(np.uint32), rs.view(np.uint32), "scales")
    assert_bits(dev.get(q, np.int8, (M, K)), rq, "codes")


def test_max_abs_and_fp16_to_int8(dev, orc):
    say("fp16_max_abs / fp16_to_int8")
    rng = np.random.default_rng(1)
    x = f16(rng.normal(0, 2, 1003))
    out = dev.empty(4)
    xp = dev.put(x)
    dev.cm.call("cactus_hip_fp16_max_abs", xp, 1003, out.ptr, None)
    assert dev.get(out, np.float32, 1)[0] == orc.lib().orc_fp16_max_abs(orc.ptr(x), 1003)
    q = dev.empty(1003)
    dev.cm.call("cactus_hip_fp16_to_int8", xp, q.ptr, 1003, ctypes.c_float(0.031), None)
    ref = np.empty(1003, np.int8)
    orc.lib().orc_fp16_to_int8(orc.ptr(x), orc.ptr(ref), 1003, 0.031)
    assert_bits(dev.get(q, np.int8, 1003), ref, "codes")


# ------------------------------------------------------------------ a2/a3
GEMM_CASES = [
    (1, 640, 2048, 32),     # Gemma-3-270m up-proj GEMV (the headline GEMV)
    (1, 1024, 3072, 32),
    (1, 2048, 1024, 32),
    (2, 1024, 512, 64),
    (3, 512, 384, 128),
    (5, 256, 200, 32),
    (17, 1024, 256, 32),
    (64, 1024, 512, 32),
    (33, 640, 200, 32),     # MFMA path, ragged rows and columns
    (100, 1024, 1024, 64),  # MFMA path, two MFMAs per group
    (40, 512, 96, 128),
    (256, 2048, 1024, 32),  # Qwen3-0.6B o-proj prefill chunk
    (512, 1024, 3072, 32),  # Qwen3-0.6B gate/up prefill GEMM (MFMA, two tiles per wave)
    (1, 10240, 64, 1024),   # row longer than 8 wave slots: block-tiled GEMV
    (2, 16, 300, 16),       # one chunk per row and per group
    (3, 2048, 130, 1024),   # 64-chunk groups, ragged last wave tile
]


@pytest.mark.parametrize("M,K,N,gs", GEMM_CASES)
def test_matmul_int8(dev, orc, M, K, N, gs):
    say("matmul_int8", M, K, N, gs)
    rng = np.random.default_rng(M + K + N + gs)
    x = activations(rng, M, K)
    B, Bs = grouped_int8_weights(rng, N, K, gs)
    rq, rs = orc.quantize_activations(x)
    ref = orc.matmul_int8(rq, rs, B, Bs, gs)
    Bp, Bsp = dev.put(B), dev.put(Bs)
    C = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8", dev.put(rq), dev.put(rs), Bp, Bsp, C.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C, np.uint16, (M, N)), ref, "matmul_int8 (pre-quantized)")
    C2 = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8_f16act", dev.put(x), Bp, Bsp, C2.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C2, np.uint16, (M, N)), ref, "matmul_int8_f16act")


@pytest.mark.parametrize("M,K,N,gs", [(1, 3072, 1024, 32), (256, 3072, 1024, 32), (1, 1024, 3072, 32),
                                      (4, 1024, 640, 64), (2, 512, 96, 128), (70, 1024, 3072, 32),
                                      (48, 2048, 1024, 64), (512, 1024, 3072, 32)])
def test_matmul_int4(dev, orc, M, K, N, gs):
    say("matmul_int4", M, K, N, gs)
    rng = np.random.default_rng(M * 3 + K + N)
    x = activations(rng, M, K)
    codes, packed, Bs = grouped_int4_weights(rng, N, K, gs)
    packed[0, :2] = [0x88, 0x77]     # extremes -8 and 7
    rq, rs = orc.quantize_activations(x)
    ref = orc.matmul_int4(rq, rs, packed, Bs, gs)
    Bp, Bsp = dev.put(packed), dev.put(Bs)
    C = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int4", dev.put(rq), dev.put(rs), Bp, Bsp, C.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C, np.uint16, (M, N)), ref, "matmul_int4")
    C2 = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int4_f16act", dev.put(x), Bp, Bsp, C2.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C2, np.uint16, (M, N)), ref, "matmul_int4_f16act")


def test_int32_accumulator_exact(dev, orc):
    """Scales of 1 and |acc| <= 2048 make C = fp16(acc) exact: the group sums
    themselves are compared."""
    say("int32 accumulators")
    rng = np.random.default_rng(3)
    M, K, N, gs = 4, 16, 300, 16
    A = rng.integers(-8, 9, (M, K), dtype=np.int8)
    B = rng.integers(-8, 9, (N, K), dtype=np.int8)
    As = np.ones(M, np.float32)
    Bs = f16(np.ones((N, 1)))
    C = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8", dev.put(A), dev.put(As), dev.put(B), dev.put(Bs), C.ptr,
                M, K, N, gs, None)
    acc = orc.group_sums_int8(A, B, gs)[:, :, 0]
    got = dev.get(C, np.uint16, (M, N)).view(np.float16).astype(np.int64)
    assert (got == acc).all()


@pytest.mark.parametrize("M,N", [(40, 96), (64, 300)])
def test_int32_accumulator_exact_mfma(dev, orc, M, N):
    """As test_int32_accumulator_exact at prefill sizes (the MFMA path), two
    groups of 32: the fp32 chain adds the two exact group sums."""
    say("int32 accumulators mfma", M, N)
    rng = np.random.default_rng(M + N)
    K, gs = 64, 32
    A = rng.integers(-8, 9, (M, K), dtype=np.int8)
    B = rng.integers(-8, 9, (N, K), dtype=np.int8)
    As = np.ones(M, np.float32)
    Bs = f16(np.ones((N, K // gs)))
    C = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8", dev.put(A), dev.put(As), dev.put(B), dev.put(Bs), C.ptr,
                M, K, N, gs, None)
    acc = orc.group_sums_int8(A, B, gs).sum(axis=2)
    got = dev.get(C, np.uint16, (M, N)).view(np.float16).astype(np.int64)
    assert (got == acc).all()


def test_matmul_int8_batched(dev, orc):
    say("matmul_int8_f16act_batched")
    rng = np.random.default_rng(4)
    M, K, N, gs, R = 1, 640, 2048, 32, 6
    xs = [activations(rng, M, K) for _ in range(R)]
    ws = [grouped_int8_weights(rng, N, K, gs) for _ in range(R)]
    A = np.stack(xs)
    B = np.stack([w[0] for w in ws])
    Bs = np.stack([w[1] for w in ws])
    C = dev.empty(R * M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8_f16act_batched", dev.put(A), dev.put(B), dev.put(Bs), C.ptr,
                M, K, N, gs, R, M * K, N * K, N * (K // gs), M * N, None)
    got = dev.get(C, np.uint16, (R, M, N))
    for r in range(R):
        rq, rs = orc.quantize_activations(xs[r])
        assert_bits(got[r], orc.matmul_int8(rq, rs, ws[r][0], ws[r][1], gs), f"batch {r}")


@pytest.mark.parametrize("M,K,N,gs,R", [(4, 128, 4096, 16, 40), (3, 2048, 1000, 1024, 5), (1, 640, 2048, 32, 1)])
def test_matmul_int8_batched_shapes(dev, orc, M, K, N, gs, R):
    """Batched GEMV shapes that pick the wide wave tiles: 40-row tiles whose
    epilogue loops over 160 outputs (M=4, K=128), 64-chunk groups, and a
    single problem."""
    say("matmul_int8_f16act_batched", M, K, N, gs, R)
    rng = np.random.default_rng(M * K + N + R)
    xs = [activations(rng, M, K) for _ in range(R)]
    ws = [grouped_int8_weights(rng, N, K, gs) for _ in range(R)]
    C = dev.empty(R * M * N * 2)
    dev.cm.call("cactus_hip_matmul_int8_f16act_batched", dev.put(np.stack(xs)),
                dev.put(np.stack([w[0] for w in ws])), dev.put(np.stack([w[1] for w in ws])), C.ptr,
                M, K, N, gs, R, M * K, N * K, N * (K // gs), M * N, None)
    got = dev.get(C, np.uint16, (R, M, N))
    for r in range(R):
        rq, rs = orc.quantize_activations(xs[r])
        assert_bits(got[r], orc.matmul_int8(rq, rs, ws[r][0], ws[r][1], gs), f"batch {r}")


@pytest.mark.parametrize("M,K,N,gs,R", [(1, 3072, 1024, 32, 7), (2, 1024, 3072, 64, 3)])
def test_matmul_int4_batched(dev, orc, M, K, N, gs, R):
    """Strided-batched INT4 GEMV (the config-3 M=1 down-projection shape and
    a gate/up shape), every problem against the oracle."""
    say("matmul_int4_f16act_batched", M, K, N, gs, R)
    rng = np.random.default_rng(M * K + N + R + 4)
    xs = [activations(rng, M, K) for _ in range(R)]
    ws = [grouped_int4_weights(rng, N, K, gs) for _ in range(R)]
    C = dev.empty(R * M * N * 2)
    dev.cm.call("cactus_hip_matmul_int4_f16act_batched", dev.put(np.stack(xs)),
                dev.put(np.stack([w[1] for w in ws])), dev.put(np.stack([w[2] for w in ws])), C.ptr,
                M, K, N, gs, R, M * K, N * K // 2, N * (K // gs), M * N, None)
    got = dev.get(C, np.uint16, (R, M, N))
    for r in range(R):
        rq, rs = orc.quantize_activations(xs[r])
        assert_bits(got[r], orc.matmul_int4(rq, rs, ws[r][1], ws[r][2], gs), f"batch {r}")


def test_unpack_int4(dev, orc):
    say("unpack_int4")
    rng = np.random.default_rng(5)
    codes, packed, _ = grouped_int4_weights(rng, 3, 64, 32)
    out = dev.empty(3 * 64)
    dev.cm.call("cactus_hip_unpack_int4_to_int8", dev.put(packed), out.ptr, 3 * 64, None)
    assert_bits(dev.get(out, np.int8, (3, 64)), codes, "unpack")


# ------------------------------------------------------------------ a4
@pytest.mark.parametrize("M,K,N", [(1, 1024, 4096), (2, 3, 2), (3, 1024, 1000), (5, 520, 77), (1, 24, 9)])
def test_matmul_f16(dev, orc, M, K, N):
    say("matmul_f16", M, K, N)
    rng = np.random.default_rng(M + K + N)
    a = f16(rng.normal(0, 1, (M, K)))
    b = f16(rng.normal(0, 0.02, (N, K)))
    if K == 3:
        a = f16([[1, 2, 3], [4, 5, 6]])
        b = f16([[1, 3, 5], [2, 4, 6]])
    c = dev.empty(M * N * 2)
    dev.cm.call("cactus_hip_matmul_f16", dev.put(a), dev.put(b), c.ptr, M, K, N, None)
    if K == 3:   # tests/test_graph.cpp:75-90 known answer
        assert (dev.get(c, np.uint16, (M, N)).view(np.float16) == [[22, 28], [49, 64]]).all()
    assert_bits(dev.get(c, np.uint16, (M, N)), orc.matmul_f16(a, b), "matmul_f16")


def test_lm_head_argmax_qwen_vocab(dev, orc):
    say("lm_head_argmax K=1024 N=151936")
    rng = np.random.default_rng(6)
    K, N = 1024, 151936
    a = f16(rng.normal(0, 1, (1, K)))
    b = f16(rng.normal(0, 0.02, (N, K)))
    logits = dev.empty(N * 2)
    tok = dev.empty(4)
    bp, ap = dev.put(b), dev.put(a)
    dev.cm.call("cactus_hip_lm_head_argmax_f16", ap, bp, logits.ptr, tok.ptr, K, N, None)
    ref = orc.matmul_f16(a, b)
    assert_bits(dev.get(logits, np.uint16, (1, N)), ref, "logits")
    assert dev.get(tok, np.uint32, 1)[0] == orc.argmax(ref[0])
    # twice more (the argmax scratch resets itself), logits not stored
    for _ in range(2):
        dev.cm.call("cactus_hip_lm_head_argmax_f16", ap, bp, None, tok.ptr, K, N, None)
        assert dev.get(tok, np.uint32, 1)[0] == orc.argmax(ref[0])


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("K,N", [(1024, 151936), (256, 1001), (200, 1000)])
def test_decode_lm_head_state(dev, orc, K, N, tiled):
    """The decode step's LM head: token = argmax(matmul_f16(rms_norm(h),
    embedding)) written to tokens_out[step], step state advanced.  K % 64 == 0
    takes the streamed kernel (ragged N), K = 200 the staged one; `tiled`
    runs the entry over the embedding's step-major tiles (rows past N zero).
    The logits row is written on the second step only (logits_out null on
    the first)."""
    say("decode_lm_head", K, N, "tiled" if tiled else "")
    rng = np.random.default_rng(K + N)
    h = f16(rng.normal(0, 1, (1, K)))
    w = f16(1 + rng.normal(0, 0.05, K))
    emb = f16(rng.normal(0, 0.02, (N, K)))
    eps = 1e-6
    ref_logits = orc.matmul_f16(orc.rms_norm(h, w, eps), emb)[0]
    ref_tok = orc.argmax(ref_logits)
    blocks = (N + 127) // 128
    scr_bytes = 1024 + 8 * blocks   # covers both entries' scratch contracts
    scratch = dev.empty(scr_bytes)
    dev.cm.call("cactus_hip_memset", scratch.ptr, 0, scr_bytes, None)
    state = dev.cm.DeviceBuffer.from_numpy(np.array([7, 100, 100, 2], np.uint32))
    dev.bufs.append(state)
    toks = dev.empty(16)
    hp, wp, ep = dev.put(h), dev.put(w), dev.put(emb)
    logits = dev.empty(2 * N)
    name = "cactus_hip_decode_lm_head"
    if tiled:
        nb = ctypes.c_size_t()
        dev.cm.call("cactus_hip_lm_tiles_bytes", K, N, ctypes.byref(nb))
        assert nb.value == (N + 63) // 64 * 64 * K * 2
        tiles = dev.empty(nb.value)
        dev.cm.call("cactus_hip_lm_tiles_build", ep, K, N, tiles.ptr, None)
        npad = (N + 63) // 64 * 64
        t = dev.get(tiles, np.uint16, nb.value // 2).reshape(K // 8, npad, 8)
        want = np.zeros((npad, K), np.uint16)
        want[:N] = emb
        assert (t.transpose(1, 0, 2).reshape(npad, K) == want).all()
        ep, name = tiles.ptr, "cactus_hip_decode_lm_head_tiled"
    for i in range(2):   # steps 2 and 3; the argmax scratch resets itself
        dev.cm.call(name, hp, wp, ctypes.c_float(eps), ep, K, N, state.ptr, toks.ptr, 4,
                    logits.ptr if i else None, scratch.ptr, scr_bytes, None)
    out = dev.get(toks, np.uint32, 4)
    assert out[2] == ref_tok and out[3] == ref_tok, (out, ref_tok)
    assert (dev.get(logits, np.uint16, N) == ref_logits).all()
    assert list(dev.get(state, np.uint32, 4)) == [ref_tok, 102, 102, 4]


@pytest.mark.parametrize("K,N", [(1024, 151936), (256, 1001)])
def test_decode_lm_head_tiled_embed(dev, orc, K, N):
    """The tiled LM head that also embeds the token it picks: tokens and
    state as the plain entry, h_next = embedding[token]; then two steps
    with h_next = h (the fused step's use), each step's token the oracle's
    argmax over the previous step's embedded row."""
    say("decode_lm_head_tiled_embed", K, N)
    rng = np.random.default_rng(K * 3 + N)
    h = f16(rng.normal(0, 1, (1, K)))
    w = f16(1 + rng.normal(0, 0.05, K))
    emb = f16(rng.normal(0, 0.02, (N, K)))
    eps = 1e-6
    blocks = (N + 639) // 640
    scr_bytes = 1024 + 8 * blocks
    scratch = dev.empty(scr_bytes)
    dev.cm.call("cactus_hip_memset", scratch.ptr, 0, scr_bytes, None)
    state = dev.cm.DeviceBuffer.from_numpy(np.array([0, 50, 50, 0], np.uint32))
    dev.bufs.append(state)
    toks = dev.empty(16)
    hp, wp, ep = dev.put(h), dev.put(w), dev.put(emb)
    nb = ctypes.c_size_t()
    dev.cm.call("cactus_hip_lm_tiles_bytes", K, N, ctypes.byref(nb))
    tiles = dev.empty(nb.value)
    dev.cm.call("cactus_hip_lm_tiles_build", ep, K, N, tiles.ptr, None)
    name = "cactus_hip_decode_lm_head_tiled_embed"
    # into a separate row
    hn = dev.empty(2 * K)
    dev.cm.call(name, hp, wp, ctypes.c_float(eps), tiles.ptr, ep, K, N, state.ptr, toks.ptr, 4, None, hn.ptr,
                scratch.ptr, scr_bytes, None)
    tok = orc.argmax(orc.matmul_f16(orc.rms_norm(h, w, eps), emb)[0])
    assert dev.get(toks, np.uint32, 1)[0] == tok
    assert (dev.get(hn, np.uint16, K) == emb[tok]).all()
    # in place: each step reads the row the one before embedded
    row = emb[tok][None, :]
    dev.cm.call("cactus_hip_memcpy_d2d", hp, hn.ptr, 2 * K, None)
    for step in (1, 2):
        dev.cm.call(name, hp, wp, ctypes.c_float(eps), tiles.ptr, ep, K, N, state.ptr, toks.ptr, 4, None, hp,
                    scratch.ptr, scr_bytes, None)
        tok = orc.argmax(orc.matmul_f16(orc.rms_norm(row, w, eps), emb)[0])
        assert dev.get(toks, np.uint32, step + 1)[step] == tok, step
        row = emb[tok][None, :]
        assert (dev.get_ptr(hp, np.uint16, K) == row[0]).all(), step
    assert list(dev.get(state, np.uint32, 4)) == [tok, 53, 53, 3]


# ------------------------------------------------------------------ a5/a6
def _attn_inputs(rng, B, S, Skv, Hq, Hkv, d):
    q = f16(rng.normal(0, 1, (B, S, Hq, d)))
    k = f16(rng.normal(0, 1, (B, Skv, Hkv, d)))
    v = f16(rng.normal(0, 1, (B, Skv, Hkv, d)))
    return q, k, v


@pytest.mark.parametrize("B,S,Skv,Hq,Hkv,d,pos,window", [
    (1, 1, 4096, 16, 8, 128, 4095, 0),     # KV-cache decode attention (FP16 KV)
    (1, 64, 64, 16, 8, 128, 0, 0),          # prefill chunk, causal
    (2, 5, 37, 4, 2, 64, 32, 0),
    (1, 9, 100, 4, 4, 128, 91, 20),         # sliding window
    (1, 3, 50, 2, 1, 40, 47, 0),            # head_dim not a multiple of 16
    (1, 40, 600, 2, 2, 36, 560, 0),         # 4-byte value chunks, many tiles
    (1, 2, 40, 2, 1, 12, 38, 0),            # head_dim not a multiple of 8
    (2, 130, 130, 8, 1, 64, 0, 0),          # 8 query heads per kv head, prefill
    (1, 5, 70, 4, 2, 256, 65, 0),           # head_dim 256
])
def test_attention_f16(dev, orc, B, S, Skv, Hq, Hkv, d, pos, window):
    say("attention_f16", B, S, Skv, Hq, Hkv, d, pos, window)
    rng = np.random.default_rng(S + Skv + d)
    q, k, v = _attn_inputs(rng, B, S, Skv, Hq, Hkv, d)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_f16(q, k, v, scale, pos_off=pos, window=window)
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_attention_f16", dev.put(q), dev.put(k), dev.put(v), o.ptr, B, S, Skv, Hq,
                Hkv, d, ctypes.c_float(scale), None, pos, window, 1, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "attention_f16")


def test_attention_f16_unaligned_values(dev, orc):
    """Value rows at a 2-byte aligned address take the register-staged form
    of the value chains."""
    say("attention_f16 unaligned values")
    rng = np.random.default_rng(21)
    B, S, Skv, Hq, Hkv, d = 1, 6, 300, 4, 2, 64
    q, k, v = _attn_inputs(rng, B, S, Skv, Hq, Hkv, d)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_f16(q, k, v, scale, pos_off=Skv - S)
    vb = np.zeros(v.size + 1, np.uint16)
    vb[1:] = v.reshape(-1)
    vp = dev.put(vb) + 2
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_attention_f16", dev.put(q), dev.put(k), vp, o.ptr, B, S, Skv, Hq,
                Hkv, d, ctypes.c_float(scale), None, Skv - S, 0, 1, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "attention_f16 unaligned")


def test_attention_f16_mask_noncausal(dev, orc):
    say("attention_f16 mask, non-causal")
    rng = np.random.default_rng(7)
    B, S, Skv, Hq, Hkv, d = 1, 4, 45, 2, 2, 64
    q, k, v = _attn_inputs(rng, B, S, Skv, Hq, Hkv, d)
    mask = f16((rng.random((B, S, Skv)) > 0.3).astype(np.float32))
    ref = orc.attention_f16(q, k, v, 0.0, mask=mask, causal=False)
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_attention_f16", dev.put(q), dev.put(k), dev.put(v), o.ptr, B, S, Skv, Hq,
                Hkv, d, ctypes.c_float(0.0), dev.put(mask), 0, 0, 0, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "attention_f16 masked")


@pytest.mark.parametrize("S,cache,new,Hq,Hkv,d", [
    (1, 4095, 1, 16, 8, 128),      # KV-cache decode attention (INT8 cache)
    (64, 256, 64, 16, 8, 128),     # second prefill chunk
    (3, 33, 3, 4, 2, 64),
    (2, 0, 2, 4, 2, 128),
    (5, 700, 5, 4, 2, 40),         # 4-byte value chunks, new rows past the prefetched one
    (1, 100, 1, 8, 1, 128),        # 8 query heads per kv head
    (40, 1000, 40, 16, 8, 128),    # new rows spanning two blocks, cache not block aligned
    (2, 100, 2, 4, 2, 256),        # head_dim 256
    (128, 1500, 128, 16, 8, 128),  # prefill chunk deep into the context
    (50, 300, 50, 8, 1, 128),      # 8 query heads per kv head, prefill
    (33, 64, 33, 4, 4, 64),        # one query head per kv head, prefill
])
def test_attention_hybrid(dev, orc, S, cache, new, Hq, Hkv, d):
    _attention_hybrid(dev, orc, S, cache, new, Hq, Hkv, d, 1.0)


def test_attention_hybrid_peaked(dev, orc):
    """Queries scaled by 40: scores spread so far that weights underflow to
    zero inside full blocks, which the value chains must skip key by key."""
    _attention_hybrid(dev, orc, 48, 500, 48, 16, 8, 128, 40.0)


def _attention_hybrid(dev, orc, S, cache, new, Hq, Hkv, d, qmul):
    say("attention_hybrid", S, cache, new, Hq, Hkv, d, qmul)
    rng = np.random.default_rng(cache + new + d)
    kf = f16(rng.normal(0, 1, (max(cache, 1), Hkv, d)))
    vf = f16(rng.normal(0, 1, (max(cache, 1), Hkv, d)))
    kc, ks = orc.quantize_kv(kf)
    vc, vs = orc.quantize_kv(vf)
    kc, vc, ks, vs = kc[:cache], vc[:cache], ks[:cache], vs[:cache]
    kn = f16(rng.normal(0, 1, (1, new, Hkv, d)))
    vn = f16(rng.normal(0, 1, (1, new, Hkv, d)))
    q = f16(rng.normal(0, 1, (1, S, Hq, d)) * qmul)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_hybrid(q, kc[None] if cache else None, vc[None] if cache else None,
                               ks[None] if cache else None, vs[None] if cache else None, kn, vn,
                               scale, pos_off=cache)
    o = dev.empty(q.nbytes)
    P = lambda a: dev.put(a) if cache else None
    dev.cm.call("cactus_hip_attention_hybrid_int8_fp16", dev.put(q), P(kc), P(vc), P(ks), P(vs),
                dev.put(kn), dev.put(vn), o.ptr, 1, S, cache, new, Hq, Hkv, d, ctypes.c_float(scale),
                cache, 1, 128, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "attention_hybrid")


def test_attention_hybrid_batch2(dev, orc):
    """Two batch rows: the codes are per batch row, the scale tables are the
    first row's for both (kernel_attention.cpp:353,424 index them without
    the batch)."""
    say("attention_hybrid batch 2")
    rng = np.random.default_rng(99)
    B, S, cache, new, Hq, Hkv, d = 2, 3, 90, 3, 4, 2, 128
    kc = rng.integers(-127, 128, (B, cache, Hkv, d), dtype=np.int8)
    vc = rng.integers(-127, 128, (B, cache, Hkv, d), dtype=np.int8)
    ks = np.abs(rng.normal(0, 0.02, (cache, Hkv, 1))).astype(np.float32)
    vs = np.abs(rng.normal(0, 0.02, (cache, Hkv, 1))).astype(np.float32)
    kn = f16(rng.normal(0, 1, (B, new, Hkv, d)))
    vn = f16(rng.normal(0, 1, (B, new, Hkv, d)))
    q = f16(rng.normal(0, 1, (B, S, Hq, d)))
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_hybrid(q, kc, vc, ks[None], vs[None], kn, vn, scale, pos_off=cache)
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_attention_hybrid_int8_fp16", dev.put(q), dev.put(kc), dev.put(vc), dev.put(ks),
                dev.put(vs), dev.put(kn), dev.put(vn), o.ptr, B, S, cache, new, Hq, Hkv, d, ctypes.c_float(scale),
                cache, 1, 128, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "attention_hybrid batch 2")


def _shadow_ref(vc, vs, cap, d):
    """Product tiles [kvh][slice][key / 4][64 dims][4 keys] (the key capacity
    rounded up to 64) of an INT8 cache (numpy float32 products, the rounding
    the value chain consumes)."""
    n, H = vc.shape[0], vc.shape[1]
    nsl, nt = (d + 63) // 64, (cap + 63) // 64
    ref = np.zeros((H, nsl, nt * 16, 64, 4), np.float32)
    prod = vc.astype(np.float32) * np.repeat(vs, 128, axis=2)[:, :, :d]
    for key in range(n):
        for sl in range(nsl):
            w = min(64, d - sl * 64)
            ref[:, sl, key // 4, :w, key % 4] = prod[key, :, sl * 64:sl * 64 + w]
    return ref


@pytest.mark.parametrize("cache,Hq,Hkv,d,qmul", [(4095, 16, 8, 128, 1.0), (700, 4, 2, 64, 1.0), (63, 8, 1, 128, 1.0),
                                                (1000, 4, 4, 128, 1.0), (640, 8, 4, 128, 40.0)])
@pytest.mark.parametrize("shadow", [True, False])
def test_decode_attention_state(dev, orc, cache, Hq, Hkv, d, qmul, shadow):
    """The decode step's attention: cache length and position from the device
    state, INT8 cache of capacity cache + 37, optionally through the value
    product tiles; equal to the hybrid attention with one new row.  qmul
    scales the query: at 40 the scores spread so far that weights underflow
    to zero, which sends blocks through the zero-skipping path."""
    say("decode_attention", cache, Hq, Hkv, d, qmul, "shadow" if shadow else "int8")
    rng = np.random.default_rng(cache + d)
    cap = cache + 37
    kf = f16(rng.normal(0, 1, (cap, Hkv, d)))
    vf = f16(rng.normal(0, 1, (cap, Hkv, d)))
    kc, ks = orc.quantize_kv(kf)
    vc, vs = orc.quantize_kv(vf)
    kn = f16(rng.normal(0, 1, (1, 1, Hkv, d)))
    vn = f16(rng.normal(0, 1, (1, 1, Hkv, d)))
    q = f16(rng.normal(0, 1, (1, 1, Hq, d)) * qmul)
    scale = 1.0 / math.sqrt(d)
    ref = orc.attention_hybrid(q, kc[None, :cache], vc[None, :cache], ks[None, :cache], vs[None, :cache],
                               kn, vn, scale, pos_off=cache)
    vcp, vsp = dev.put(vc), dev.put(vs)
    shp = None
    if shadow:
        nbytes = ctypes.c_size_t()
        dev.cm.call("cactus_hip_kv_shadow_bytes", cap, Hkv, d, ctypes.byref(nbytes))
        sh = dev.empty(nbytes.value)
        dev.cm.call("cactus_hip_kv_shadow_update", vcp, vsp, sh.ptr, 0, cache, Hkv, d, 128, cap, None)
        got = dev.get(sh, np.float32, (Hkv, (d + 63) // 64, (cap + 63) // 64 * 16, 64, 4))
        want = _shadow_ref(vc[:cache], vs[:cache], cap, d)
        for key in (0, cache // 2, cache - 1):
            t, j = key // 4, key % 4
            assert (got[:, :, t, :, j] == want[:, :, t, :, j]).all(), f"products of key {key}"
        shp = sh.ptr
    state = np.array([0, cache, cache, 0], np.uint32)
    o = dev.empty(q.nbytes)
    dev.cm.call("cactus_hip_decode_attention", dev.put(q), dev.put(kc), vcp, dev.put(ks), vsp, dev.put(kn),
                dev.put(vn), o.ptr, Hq, Hkv, d, ctypes.c_float(scale), dev.put(state), cap, shp, None)
    assert_bits(dev.get(o, np.uint16, q.shape), ref, "decode attention")


@pytest.mark.parametrize("cache,Hq,Hkv,d", [(4095, 16, 8, 128), (700, 4, 4, 64), (127, 4, 2, 128),
                                            (300, 8, 4, 64), (256, 16, 8, 128)])
@pytest.mark.parametrize("shadow", [True, False])
def test_decode_prep_attention_fused(dev, orc, cache, Hq, Hkv, d, shadow):
    """The head preparation fused into the attention's score kernel equals
    cactus_hip_decode_attn_prep followed by cactus_hip_decode_attention:
    the same output bits and the same appended cache row (codes, scales and
    product tiles); the output is also the oracle's hybrid attention on the
    prepared q and key."""
    say("decode_prep_attention", cache, Hq, Hkv, d, "shadow" if shadow else "int8")
    rng = np.random.default_rng(cache * 7 + d)
    cap = cache + 21
    kc, ks = orc.quantize_kv(f16(rng.normal(0, 1, (cap, Hkv, d))))
    vc, vs = orc.quantize_kv(f16(rng.normal(0, 1, (cap, Hkv, d))))
    q_raw = f16(rng.normal(0, 1, (Hq, d)))
    k_raw = f16(rng.normal(0, 1, (Hkv, d)))
    v_raw = f16(rng.normal(0, 1, (Hkv, d)))
    qn = f16(rng.normal(1, 0.2, d))
    kn = f16(rng.normal(1, 0.2, d))
    eps, theta, scale = 1e-6, 1e6, 1.0 / math.sqrt(d)
    state = dev.put(np.array([0, cache, cache, 0], np.uint32))

    def caches():
        bufs = [dev.put(kc), dev.put(vc), dev.put(ks), dev.put(vs)]
        sh = None
        if shadow:
            nbytes = ctypes.c_size_t()
            dev.cm.call("cactus_hip_kv_shadow_bytes", cap, Hkv, d, ctypes.byref(nbytes))
            sh = dev.empty(nbytes.value)
            dev.cm.call("cactus_hip_kv_shadow_update", bufs[1], bufs[3], sh.ptr, 0, cache, Hkv, d, 128, cap, None)
        return bufs, sh

    args = lambda: (dev.put(q_raw), dev.put(k_raw), dev.put(v_raw), dev.put(qn), dev.put(kn))
    # separate kernels
    (kcA, vcA, ksA, vsA), shA = caches()
    qa, ka, va, qna, kna = args()
    q_out, k_out, oA = dev.empty(q_raw.nbytes), dev.empty(k_raw.nbytes), dev.empty(q_raw.nbytes)
    dev.cm.call("cactus_hip_decode_attn_prep", qa, ka, va, qna, kna, ctypes.c_float(eps), Hq, Hkv, d,
                ctypes.c_float(theta), state, q_out.ptr, k_out.ptr, kcA, vcA, ksA, vsA, cap,
                shA.ptr if shadow else None, None)
    dev.cm.call("cactus_hip_decode_attention", q_out.ptr, kcA, vcA, ksA, vsA, k_out.ptr, va, oA.ptr, Hq, Hkv, d,
                ctypes.c_float(scale), state, cap, shA.ptr if shadow else None, None)
    # fused
    (kcB, vcB, ksB, vsB), shB = caches()
    qb, kb, vb, qnb, knb = args()
    oB = dev.empty(q_raw.nbytes)
    dev.cm.call("cactus_hip_decode_prep_attention", qb, kb, vb, qnb, knb, ctypes.c_float(eps), Hq, Hkv, d,
                ctypes.c_float(theta), state, kcB, vcB, ksB, vsB, cap, shB.ptr if shadow else None,
                ctypes.c_float(scale), oB.ptr, None)
    got_a = dev.get(oA, np.uint16, (Hq, d))
    got_b = dev.get(oB, np.uint16, (Hq, d))
    assert_bits(got_b, got_a, "fused output")
    for name, x, y, dt, shp in (("k codes", kcA, kcB, np.int8, (cap, Hkv, d)), ("v codes", vcA, vcB, np.int8, (cap, Hkv, d)),
                                ("k scales", ksA, ksB, np.float32, (cap, Hkv, 1)),
                                ("v scales", vsA, vsB, np.float32, (cap, Hkv, 1))):
        a_, b_ = dev.get_ptr(x, dt, shp), dev.get_ptr(y, dt, shp)
        assert (a_[cache] == b_[cache]).all(), name + " of the appended row"
        assert (a_[:cache] == b_[:cache]).all(), name + " before the appended row"
    if shadow:
        # written entries only: keys 0..cache (padding and later keys are
        # never written, so two fresh buffers differ there)
        ts = (Hkv, (d + 63) // 64, (cap + 63) // 64 * 16, 64, 4)
        keys = np.arange(cache + 1)
        ta = dev.get(shA, np.float32, ts)[:, :, keys // 4, :, keys % 4]
        tb = dev.get(shB, np.float32, ts)[:, :, keys // 4, :, keys % 4]
        assert (ta.view(np.uint32) == tb.view(np.uint32)).all(), "product tiles"
    qp = dev.get(q_out, np.uint16, (Hq, d)).reshape(1, 1, Hq, d)
    kp = dev.get(k_out, np.uint16, (Hkv, d)).reshape(1, 1, Hkv, d)
    ref = orc.attention_hybrid(qp, kc[None, :cache], vc[None, :cache], ks[None, :cache], vs[None, :cache], kp,
                               v_raw.reshape(1, 1, Hkv, d), scale, pos_off=cache)
    assert_bits(got_b.reshape(1, 1, Hq, d), ref, "fused output vs oracle")


# ------------------------------------------------------------------ a7
@pytest.mark.parametrize("S,H,d,gs", [(256, 8, 128, 128), (3, 2, 100, 128), (5, 4, 256, 128), (2, 2, 64, 32)])
def test_quantize_kv(dev, orc, S, H, d, gs):
    say("quantize_kv", S, H, d, gs)
    rng = np.random.default_rng(S + d)
    x = f16(rng.normal(0, 1, (S, H, d)))
    ng = (d + gs - 1) // gs
    q = dev.empty(S * H * d)
    sc = dev.empty(S * H * ng * 4)
    dev.cm.call("cactus_hip_quantize_kv_fp16_to_int8", dev.put(x), q.ptr, sc.ptr, S, H, d, gs, None)
    rq, rs = orc.quantize_kv(x, gs)
    assert_bits(dev.get(sc, np.float32, (S, H, ng)).view(np.uint32), rs.view(np.uint32), "kv scales")
    assert_bits(dev.get(q, np.int8, (S, H, d)), rq, "kv codes")


@pytest.mark.parametrize("Hkv,d,count,at", [(8, 128, 256, 0), (2, 128, 37, 50), (2, 72, 9, 60), (1, 256, 3, 130)])
def test_kv_append_layers(dev, orc, Hkv, d, count, at):
    """The all-layer cache append equals, layer by layer, the quantization
    of the new K and V rows (oracle: codes and scales at slots [at, at +
    count), nothing else written) and the value products of
    cactus_hip_kv_shadow_update over the same cache."""
    say("kv_append_layers", Hkv, d, count, at)
    nl, cap = 3, 300
    rng = np.random.default_rng(Hkv * d + count + at)
    ng = (d + 127) // 128
    shb = ctypes.c_size_t()
    dev.cm.call("cactus_hip_kv_shadow_bytes", cap, Hkv, d, ctypes.byref(shb))
    recs, cache, srcs, want = [], [], [], []
    for l in range(nl):
        kf = f16(rng.normal(0, 1 + l, (count, Hkv, d)))
        vf = f16(rng.normal(0, 2, (count, Hkv, d)))
        init_c = rng.integers(-128, 128, (2, cap, Hkv, d), dtype=np.int8)
        init_s = rng.random((2, cap, Hkv, ng), dtype=np.float32)
        bufs = [dev.put(init_c[0]), dev.put(init_c[1]), dev.put(init_s[0]), dev.put(init_s[1]),
                dev.put(np.zeros(shb.value // 4, np.float32))]
        recs.append(bufs)
        srcs.append((dev.put(kf), dev.put(vf)))
        kc, ks = orc.quantize_kv(kf)
        vc, vs = orc.quantize_kv(vf)
        wc, ws = init_c.copy(), init_s.copy()
        wc[0, at:at + count], wc[1, at:at + count] = kc, vc
        ws[0, at:at + count], ws[1, at:at + count] = ks, vs
        want.append((wc, ws))
    table = dev.put(np.array(recs, np.uint64))
    karr = (ctypes.c_void_p * nl)(*[k for k, _ in srcs])
    varr = (ctypes.c_void_p * nl)(*[v for _, v in srcs])
    dev.cm.call("cactus_hip_kv_append_layers", table, karr, varr, nl, count, at, Hkv, d, 128, cap, None)
    for l in range(nl):
        kb, vb, ksb, vsb, shp = recs[l]
        wc, ws = want[l]
        assert_bits(dev.get_ptr(kb, np.int8, (cap, Hkv, d)), wc[0], f"layer {l} key codes")
        assert_bits(dev.get_ptr(vb, np.int8, (cap, Hkv, d)), wc[1], f"layer {l} value codes")
        assert_bits(dev.get_ptr(ksb, np.float32, (cap, Hkv, ng)).view(np.uint32), ws[0].view(np.uint32),
                    f"layer {l} key scales")
        assert_bits(dev.get_ptr(vsb, np.float32, (cap, Hkv, ng)).view(np.uint32), ws[1].view(np.uint32),
                    f"layer {l} value scales")
        ref_sh = dev.empty(shb.value)
        dev.cm.call("cactus_hip_memset", ref_sh.ptr, 0, shb.value, None)
        dev.cm.call("cactus_hip_kv_shadow_update", vb, vsb, ref_sh.ptr, at, count, Hkv, d, 128, cap, None)
        assert_bits(dev.get_ptr(shp, np.uint32, shb.value // 4), dev.get(ref_sh, np.uint32, shb.value // 4),
                    f"layer {l} value products")


# ------------------------------------------------------------------ a8-a14
@pytest.mark.parametrize("rows,dims,eps", [(1, 1024, 1e-6), (256, 1024, 1e-6), (4096, 128, 1e-6),
                                           (3, 1000, 1e-5), (2, 1004, 1e-5), (1, 8, 1e-5)])
def test_rms_norm(dev, orc, rows, dims, eps):
    say("rms_norm", rows, dims)
    rng = np.random.default_rng(rows + dims)
    x = f16(rng.normal(0, 1, (rows, dims)))
    w = f16(1 + rng.normal(0, 0.02, dims))
    y = dev.empty(x.nbytes)
    dev.cm.call("cactus_hip_rms_norm_f16", dev.put(x), dev.put(w), y.ptr, rows, dims,
                ctypes.c_float(eps), None)
    assert_bits(dev.get(y, np.uint16, x.shape), orc.rms_norm(x, w, eps), "rms_norm")


@pytest.mark.parametrize("B,S,H,d,start,theta", [(1, 256, 16, 128, 0, 1e6), (1, 1, 8, 128, 4095, 1e6),
                                                 (2, 3, 2, 36, 7, 1e4), (1, 64, 8, 128, 3900, 1e6)])
def test_rope(dev, orc, B, S, H, d, start, theta):
    say("rope", B, S, H, d, start, theta)
    rng = np.random.default_rng(S + start)
    x = f16(rng.normal(0, 1, (B, S, H, d)))
    y = dev.empty(x.nbytes)
    dev.cm.call("cactus_hip_rope_f16", dev.put(x), y.ptr, B, S, H, d, start, ctypes.c_float(theta), None)
    assert_bits(dev.get(y, np.uint16, x.shape), orc.rope(x, start, theta), "rope")


@pytest.mark.parametrize("rows,V", [(2, 3), (4, 96), (3, 1000), (1, 151936)])
def test_softmax(dev, orc, rows, V):
    say("softmax", rows, V)
    rng = np.random.default_rng(V)
    x = f16(rng.normal(0, 3, (rows, V)))
    y = dev.empty(x.nbytes)
    dev.cm.call("cactus_hip_softmax_f16", dev.put(x), y.ptr, 1, rows, V, None)
    assert_bits(dev.get(y, np.uint16, x.shape), orc.softmax(x), "softmax")


@pytest.mark.parametrize("n", [3072, 786432, 1003])
def test_silu_add_multiply(dev, orc, n):
    say("silu/add/multiply", n)
    rng = np.random.default_rng(n)
    a = f16(rng.normal(0, 3, n))
    b = f16(rng.normal(0, 3, n))
    ap, bp = dev.put(a), dev.put(b)
    y = dev.empty(a.nbytes)
    dev.cm.call("cactus_hip_silu_f16", ap, y.ptr, n, None)
    assert_bits(dev.get(y, np.uint16, n), orc.silu(a), "silu")
    dev.cm.call("cactus_hip_add_f16", ap, bp, y.ptr, n, None)
    assert_bits(dev.get(y, np.uint16, n), orc.add(a, b), "add")
    dev.cm.call("cactus_hip_multiply_f16", ap, bp, y.ptr, n, None)
    assert_bits(dev.get(y, np.uint16, n), orc.multiply(a, b), "multiply")


def test_embedding(dev, orc):
    say("embedding")
    rng = np.random.default_rng(8)
    V, Hd = 1000, 1024
    table = f16(rng.normal(0, 0.02, (V, Hd)))
    ids = np.array([5, 999, 0, 5, 123], np.float32)
    out = dev.empty(5 * Hd * 2)
    err = dev.empty(4)
    dev.cm.call("cactus_hip_memset", err.ptr, 0, 4, None)
    tp = dev.put(table)
    dev.cm.call("cactus_hip_embedding_f16", tp, dev.put(ids), out.ptr, 5, Hd, V, err.ptr, None)
    assert_bits(dev.get(out, np.uint16, (5, Hd)), table[ids.astype(int)], "embedding")
    assert dev.get(err, np.int32, 1)[0] == 0
    dev.cm.call("cactus_hip_embedding_f16", tp, dev.put(np.array([1000], np.float32)), out.ptr, 1, Hd,
                V, err.ptr, None)
    assert dev.get(err, np.int32, 1)[0] == 1


def test_sample_greedy(dev, orc):
    say("sample greedy")
    rng = np.random.default_rng(9)
    V = 151936
    logits = f16(rng.normal(0, 1, V))
    logits[[77, 150000]] = f16([9.0, 9.0])       # planted tie: first index wins
    out = dev.empty(4)
    lp = dev.put(logits)
    dev.cm.call("cactus_hip_sample_f16", lp, out.ptr, V, ctypes.c_float(0.0), ctypes.c_float(0.0), 0, 0,
                None)
    assert dev.get(out, np.uint32, 1)[0] == orc.argmax(logits) == 77
    # the full sampler (tests/test_sampler.py covers it in depth), with a
    # top-k and with top-p over the whole vocabulary (top_k 0)
    for top_k in (20, 0):
        dev.cm.call("cactus_hip_sample_history_reset", None)
        dev.cm.call("cactus_hip_sample_f16", lp, out.ptr, V, ctypes.c_float(0.7), ctypes.c_float(0.9), top_k, 1,
                    None)
        assert dev.get(out, np.uint32, 1)[0] == orc.OracleSampler().sample(logits, 0.7, 0.9, top_k, 1)


@pytest.mark.parametrize("K,gs,Nq,Nkv,F", [(1024, 32, 2048, 1024, 3072), (640, 32, 1024, 256, 2048),
                                            (1040, 16, 160, 96, 200), (256, 128, 128, 40, 96)])
def test_decode_step_matmuls(dev, orc, K, gs, Nq, Nkv, F):
    """The decode step's matmul kernels against the oracle's node chains, bit
    for bit: RMSNorm + q/k/v (INT8), RMSNorm + gate/up (INT4) + SiLU * up,
    and the INT8 / INT4 projections with the residual add.  Rows of a
    multiple of 128 values take the chain-major RMS path, others (K 1040)
    the row-major one."""
    say("decode step matmuls", K, gs, Nq, Nkv, F)
    rng = np.random.default_rng(K + gs + F)
    eps = 1e-6
    h = f16(rng.normal(0, 1.5, (1, K)))
    nw = f16(1 + rng.normal(0, 0.05, K))
    xq, xs = orc.quantize_activations(orc.rms_norm(h, nw, eps))
    hp, nwp = dev.put(h), dev.put(nw)
    ws = [grouped_int8_weights(rng, n, K, gs) for n in (Nq, Nkv, Nkv)]
    outs = [dev.empty(n * 2) for n in (Nq, Nkv, Nkv)]
    args = []
    for (B, Bs), o in zip(ws, outs):
        args += [dev.put(B), dev.put(Bs), o.ptr, B.shape[0]]
    dev.cm.call("cactus_hip_decode_qkv", hp, nwp, ctypes.c_float(eps), K, gs, *args, None)
    for (B, Bs), o, what in zip(ws, outs, "qkv"):
        assert_bits(dev.get(o, np.uint16, (1, B.shape[0])), orc.matmul_int8(xq, xs, B, Bs, gs), f"decode {what}")
    # gate/up (INT4, group 32) with SiLU * up; INT4 needs K % 32 == 0
    if K % 32 == 0:
        _, Wg, Sg = grouped_int4_weights(rng, F, K, 32)
        _, Wu, Su = grouped_int4_weights(rng, F, K, 32)
        m = dev.empty(F * 2)
        dev.cm.call("cactus_hip_decode_mlp_up", hp, nwp, ctypes.c_float(eps), K, 32, dev.put(Wg), dev.put(Sg),
                    dev.put(Wu), dev.put(Su), F, m.ptr, None)
        want = orc.multiply(orc.silu(orc.matmul_int4(xq, xs, Wg, Sg, 32)), orc.matmul_int4(xq, xs, Wu, Su, 32))
        assert_bits(dev.get(m, np.uint16, (1, F)), want, "decode gate/up")
    # projections with the residual add: INT8 (K -> Nq) and INT4 (F -> K)
    a = f16(rng.normal(0, 1, (1, Nq)))
    Wo, So = grouped_int8_weights(rng, K, Nq, gs)
    hr = dev.put(h)
    dev.cm.call("cactus_hip_decode_matmul_residual", dev.put(a), Nq, gs, dev.put(Wo), dev.put(So), K, 0, hr, None)
    aq, as_ = orc.quantize_activations(a)
    want_o = orc.add(h, orc.matmul_int8(aq, as_, Wo, So, gs))
    assert_bits(dev.get_ptr(hr, np.uint16, (1, K)), want_o, "decode o-proj + residual")
    if F % 32 == 0:
        mm = f16(rng.normal(0, 1, (1, F)))
        _, Wd, Sd = grouped_int4_weights(rng, K, F, 32)
        hd = dev.put(h)
        dev.cm.call("cactus_hip_decode_matmul_residual", dev.put(mm), F, 32, dev.put(Wd), dev.put(Sd), K, 1, hd, None)
        mq, ms = orc.quantize_activations(mm)
        assert_bits(dev.get_ptr(hd, np.uint16, (1, K)), orc.add(h, orc.matmul_int4(mq, ms, Wd, Sd, 32)),
                    "decode down + residual")


@pytest.mark.parametrize("M,K", [(256, 1024), (33, 1001), (1, 3072), (512, 2048), (40, 16), (2, 8192),
                                 (3, 8200)])
def test_rms_norm_quantize_fused(dev, orc, M, K):
    """The fused RMSNorm + row quantization equals cactus_hip_rms_norm_f16
    followed by cactus_hip_quantize_activations, and the oracle's pair."""
    say("rms_norm_quantize", M, K)
    rng = np.random.default_rng(M + K)
    x = f16(rng.normal(0, 1.5, (M, K)))
    w = f16(1 + rng.normal(0, 0.05, K))
    xp, wp = dev.put(x), dev.put(w)
    q, s = dev.empty(M * K), dev.empty(M * 4)
    dev.cm.call("cactus_hip_rms_norm_quantize_f16", xp, wp, q.ptr, s.ptr, M, K, ctypes.c_float(1e-6), None)
    rq, rs = orc.quantize_activations(orc.rms_norm(x, w, 1e-6))
    assert_bits(dev.get(s, np.float32, M).view(np.uint32), rs.view(np.uint32), "scales")
    assert_bits(dev.get(q, np.int8, (M, K)), rq, "codes")


@pytest.mark.parametrize("M,K", [(256, 3072), (33, 1001), (64, 12), (1, 3072)])
def test_silu_mul_quantize_fused(dev, orc, M, K):
    """silu(gate) * up with the row quantization in one launch equals the
    oracle's silu, multiply and quantize_activations (ragged M*K puts the
    silu expf tail in the last row)."""
    say("silu_mul_quantize", M, K)
    rng = np.random.default_rng(M * 3 + K)
    gate = f16(rng.normal(0, 2, (M, K)))
    up = f16(rng.normal(0, 1, (M, K)))
    q, s = dev.empty(M * K), dev.empty(M * 4)
    dev.cm.call("cactus_hip_silu_mul_quantize_f16", dev.put(gate), dev.put(up), q.ptr, s.ptr, M, K, None)
    prod = orc.multiply(orc.silu(gate.reshape(-1)), up.reshape(-1)).reshape(M, K)
    rq, rs = orc.quantize_activations(prod)
    assert_bits(dev.get(s, np.float32, M).view(np.uint32), rs.view(np.uint32), "scales")
    assert_bits(dev.get(q, np.int8, (M, K)), rq, "codes")


@pytest.mark.parametrize("S,H,d,pos", [(256, 16, 128, 3840), (1, 8, 128, 4095), (7, 4, 64, 0), (5, 2, 12, 9),
                                       (3, 2, 256, 17), (6, 3, 200, 40)])
def test_rms_norm_rope_fused(dev, orc, S, H, d, pos):
    """The head RMSNorm then RoPE in one launch equals the oracle's pair."""
    say("rms_norm_rope", S, H, d, pos)
    rng = np.random.default_rng(S + H + d + pos)
    x = f16(rng.normal(0, 1.5, (1, S, H, d)))
    w = f16(1 + rng.normal(0, 0.05, d))
    y = dev.empty(x.nbytes)
    dev.cm.call("cactus_hip_rms_norm_rope_f16", dev.put(x), dev.put(w), y.ptr, 1, S, H, d, pos,
                ctypes.c_float(1e6), ctypes.c_float(1e-6), None)
    ref = orc.rope(orc.rms_norm(x.reshape(S * H, d), w, 1e-6).reshape(1, S, H, d), pos, 1e6)
    assert_bits(dev.get(y, np.uint16, x.shape), ref, "rms_norm_rope")


@pytest.mark.parametrize("S,Hq,Hkv,d,pos", [(256, 16, 8, 128, 3840), (1, 16, 8, 128, 77), (5, 3, 1, 200, 2),
                                            (4, 2, 0, 64, 0), (4, 0, 2, 64, 5)])
def test_rms_norm_rope_qk(dev, orc, S, Hq, Hkv, d, pos):
    """The q and k head RMSNorm + RoPE in one launch: each output equals the
    oracle's pair on that tensor (either head count may be zero)."""
    say("rms_norm_rope_qk", S, Hq, Hkv, d, pos)
    rng = np.random.default_rng(S + Hq + Hkv + d + pos)
    xs = [f16(rng.normal(0, 1.5, (1, S, H, d))) for H in (Hq, Hkv)]
    ws = [f16(1 + rng.normal(0, 0.05, d)) for _ in range(2)]
    ys = [dev.empty(max(x.nbytes, 2)) for x in xs]
    ptr = lambda x: dev.put(x) if x.size else None
    dev.cm.call("cactus_hip_rms_norm_rope_qk_f16", ptr(xs[0]), dev.put(ws[0]), ys[0].ptr, Hq, ptr(xs[1]),
                dev.put(ws[1]), ys[1].ptr, Hkv, 1, S, d, pos, ctypes.c_float(1e6), ctypes.c_float(1e-6), None)
    for x, w, y, what in zip(xs, ws, ys, ("q", "k")):
        if x.size == 0:
            continue
        H = x.shape[2]
        ref = orc.rope(orc.rms_norm(x.reshape(S * H, d), w, 1e-6).reshape(1, S, H, d), pos, 1e6)
        assert_bits(dev.get(y, np.uint16, x.shape), ref, f"rms_norm_rope_qk ({what})")


@pytest.mark.parametrize("M,K,N,gs,int4,shift", [(256, 1024, 1024, 32, False, 0), (256, 3072, 1024, 32, True, 0),
                                                 (256, 1024, 1024, 32, False, 1), (40, 1024, 640, 64, True, 0),
                                                 (5, 1024, 1024, 32, False, 0), (3, 3072, 1024, 32, True, 0)])
def test_matmul_add_fused(dev, orc, M, K, N, gs, int4, shift):
    """The grouped matmul with the residual add fused equals the matmul
    followed by an fp16 add, for pre-quantized and FP16 activations: the
    LDS MFMA path (and with a residual 2 bytes off 16-byte alignment:
    shift 1), the register-streamed path (M 40, 2-byte-aligned scales) and
    the small-M GEMV path."""
    say("matmul_add", M, K, N, gs, int4, shift)
    rng = np.random.default_rng(M + K + N + int4)
    x = activations(rng, M, K)
    if int4:
        _, B, Bs = grouped_int4_weights(rng, N, K, gs)
    else:
        B, Bs = grouped_int8_weights(rng, N, K, gs)
    rq, rs = orc.quantize_activations(x)
    mm = orc.matmul_int4(rq, rs, B, Bs, gs) if int4 else orc.matmul_int8(rq, rs, B, Bs, gs)
    res = f16(rng.normal(0, 4, (M, N)))
    want = (mm.view(np.float16) + res.view(np.float16)).astype(np.float16).view(np.uint16)
    Bp = dev.put(B)
    if M == 40:   # scales at a 2-byte offset: the LDS path declines
        Bsp = dev.put(np.concatenate([np.zeros(1, np.uint16), Bs.ravel()])) + 2
    else:
        Bsp = dev.put(Bs)
    Rp = dev.put(np.concatenate([np.zeros(shift, np.uint16), res.ravel()])) + 2 * shift
    kind = "int4" if int4 else "int8"
    C = dev.empty(M * N * 2)
    dev.cm.call(f"cactus_hip_matmul_{kind}_add", dev.put(rq), dev.put(rs), Bp, Bsp, Rp, C.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C, np.uint16, (M, N)), want, f"matmul_{kind}_add")
    C2 = dev.empty(M * N * 2)
    dev.cm.call(f"cactus_hip_matmul_{kind}_f16act_add", dev.put(x), Bp, Bsp, Rp, C2.ptr, M, K, N, gs, None)
    assert_bits(dev.get(C2, np.uint16, (M, N)), want, f"matmul_{kind}_f16act_add")


@pytest.mark.parametrize("M,K,Ns,gs,int4", [(256, 1024, (2048, 1024, 1024), 32, False),   # Qwen3-0.6B q/k/v chunk
                                            (256, 1024, (3072, 3072), 32, True),          # its gate/up
                                            (100, 640, (200, 96, 136), 32, False),        # ragged tiles
                                            (33, 1024, (520, 1000), 64, True),
                                            (40, 512, (96, 64, 32), 128, False),
                                            (512, 1024, (3072, 3072), 32, False),
                                            (5, 1024, (64, 128, 96), 32, False),          # small M: one GEMV each
                                            (64, 1024, (256,), 32, True)])
def test_matmul_grouped_multi(dev, orc, M, K, Ns, gs, int4):
    """Several grouped matmuls over one pre-quantized activation in one call
    (the merged q/k/v and gate/up launches): every output bit-identical to
    the oracle's matmul of its own weights."""
    say("matmul_grouped_multi", M, K, Ns, gs, int4)
    rng = np.random.default_rng(M + K + sum(Ns) + int4)
    x = activations(rng, M, K)
    rq, rs = orc.quantize_activations(x)
    cnt = len(Ns)
    Bp, Bsp, Cs, refs = [], [], [], []
    for N in Ns:
        if int4:
            _, B, Bs = grouped_int4_weights(rng, N, K, gs)
            refs.append(orc.matmul_int4(rq, rs, B, Bs, gs))
        else:
            B, Bs = grouped_int8_weights(rng, N, K, gs)
            refs.append(orc.matmul_int8(rq, rs, B, Bs, gs))
        Bp.append(dev.put(B))
        Bsp.append(dev.put(Bs))
        Cs.append(dev.empty(M * N * 2))
    arr = lambda vals, t: (t * cnt)(*vals)
    dev.cm.call("cactus_hip_matmul_grouped_multi", dev.put(rq), dev.put(rs), cnt, arr(Bp, ctypes.c_void_p),
                arr(Bsp, ctypes.c_void_p), arr([c.ptr for c in Cs], ctypes.c_void_p), arr(Ns, ctypes.c_size_t),
                M, K, gs, int(int4), None)
    for i, N in enumerate(Ns):
        assert_bits(dev.get(Cs[i], np.uint16, (M, N)), refs[i], f"matmul_grouped_multi problem {i}")
