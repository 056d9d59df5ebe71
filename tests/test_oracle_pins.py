"""Pins of the CPU restatement (oracle/) -- runs without a GPU.

Every oracle function is checked against something that does not share its
code: the reference's own known-answer tests (tests/test_graph.cpp,
tests/test_kernel.cpp), closed forms evaluated independently in float64 /
numpy, special cases the mathematics fixes, and exact integer brute force.
"""
import ctypes
import math

import numpy as np
import pytest

from _data import f16, grouped_int8_weights, grouped_int4_weights, pack_int4

F16 = np.float16


def h(x):
    return np.float64(np.asarray(x, np.uint16).view(np.float16))


def to16(x64) -> int:
    """float64 -> fp16 bits with numpy's own (independent) conversion."""
    return int(np.array([x64], np.float64).astype(np.float16).view(np.uint16)[0])


# ----------------------------------------------------------------- fp16 helpers
def test_h2f_all_patterns(orc):
    L = orc.lib()
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    got = np.array([L.orc_h2f(int(p)) for p in pats[::7]], np.float32)
    r = ref[::7]
    same = (got == r) | (np.isnan(got) & np.isnan(r))
    assert same.all()


def test_f2h_matches_numpy_rne(orc):
    L = orc.lib()
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.normal(0, 1, 4000), rng.normal(0, 3e4, 2000), rng.normal(0, 1e-5, 2000),
        rng.normal(0, 1e-7, 1000),
        np.array([65504.0, 65519.99, 65520.0, 70000.0, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 0.0, -0.0, np.inf, -np.inf])]).astype(np.float32)
    ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.orc_f2h(float(x)) for x in xs], np.uint16)
    assert (got == ref).all()


def test_fp16_arith_single_rounding(orc):
    """hadd/hmul/hfma equal numpy's float64->float16 rounding of the exact value."""
    L = orc.lib()
    rng = np.random.default_rng(1)
    a = f16(rng.normal(0, 4, 3000))
    b = f16(rng.normal(0, 4, 3000))
    c = f16(rng.normal(0, 4, 3000))
    for i in range(3000):
        x, y, z = int(a[i]), int(b[i]), int(c[i])
        assert L.orc_hadd(x, y) == to16(h(x) + h(y))
        assert L.orc_hmul(x, y) == to16(h(x) * h(y))
        assert L.orc_hfma(x, y, z) == to16(h(x) * h(y) + h(z))   # exact in float64


# ----------------------------------------------------------------- exp helpers
def test_expf_against_double_exp(orc):
    """orc_expf equals the float rounding of the double-precision exp."""
    L = orc.lib()
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.uniform(-104, 88.7, 20000), rng.uniform(-1, 1, 5000),
                         [0.0, -0.0, 1.0, -1.0, 88.72283, -87.0, -103.9]]).astype(np.float32)
    mism = 0
    for x in xs:
        got = np.float32(L.orc_expf(float(x)))
        ref = np.float32(math.exp(float(x)))
        if got != ref:
            mism += 1
            assert abs(int(got.view(np.int32)) - int(ref.view(np.int32))) <= 1
    assert mism <= 2
    assert L.orc_expf(0.0) == 1.0
    assert math.isinf(L.orc_expf(89.0))
    assert L.orc_expf(-120.0) == 0.0


def test_fast_exp_closed_form(orc):
    """fast_exp(x) = 2^floor(z) * P(frac(z)*ln2), z = x*log2(e), P the degree-4
    Taylor polynomial of 2^u (kernel_utils.h:108-141) -- i.e. up to ~19% below
    e^x, exact 1 at 0."""
    L = orc.lib()
    assert L.orc_fast_exp(0.0) == 1.0
    c = [1.0, 0.6931471805599453, 0.2402265069591007, 0.05550410866482158, 0.009618129842071803]
    for x in np.linspace(-80, 80, 4001):
        z = np.float32(x) * np.float32(1.4426950408889634)
        fl = math.floor(z)
        u = (float(z) - fl) * 0.6931471805599453
        p = sum(ci * u ** i for i, ci in enumerate(c))
        ref = p * 2.0 ** fl
        got = L.orc_fast_exp(float(x))
        assert abs(got - ref) <= 4e-6 * ref
    # the documented deviation from e^x: fast_exp(0.5) ~ 2^0.5, 14% below e^0.5
    assert abs(L.orc_fast_exp(0.5) / math.sqrt(2) - 1) < 1e-4
    assert 0.85 < L.orc_fast_exp(0.5) / math.exp(0.5) < 0.86


def test_poly_weight_closed_form(orc):
    """Second-order 2^x weight (kernel_attention.cpp:174-195): 2^trunc(t) *
    (1 + 0.6931472 f + 0.2402265 f^2), t = (s-m)*1.442695, f = t - trunc(t)."""
    L = orc.lib()
    assert L.orc_poly_exp_weight(1.5, 1.5) == 1.0
    assert L.orc_poly_exp_weight(-math.inf, 0.0) == 0.0
    worst = 0.0
    for d in np.linspace(-20, 0, 2001):
        t = float(np.float32(np.float32(d) * np.float32(1.442695)))
        ti = math.trunc(t)
        f = t - ti
        ref = (1 + 0.6931472 * f + 0.2402265 * f * f) * 2.0 ** ti
        got = L.orc_poly_exp_weight(float(d), 0.0)
        assert abs(got - ref) <= 3e-6 * ref
        worst = max(worst, got / math.exp(d) - 1)
    assert 0.08 < worst < 0.10   # "up to ~9.4% high" near f -> -1


# ----------------------------------------------------------------- a1 quantization
def test_quantize_special_cases(orc):
    # all-zero row: scale floored at 1e-10, codes 0
    x = f16(np.zeros((1, 64)))
    q, s = orc.quantize_activations(x)
    assert s[0] == np.float32(1e-10) and (q == 0).all()
    # the max element maps to +-127
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (4, 64)).astype(np.float16)
    x[1, 5] = -7.5
    q, s = orc.quantize_activations(x.view(np.uint16))
    assert q[1, 5] == -127
    for m in range(4):
        i = np.argmax(np.abs(x[m].astype(np.float32)))
        assert abs(int(q[m, i])) == 127
        assert s[m] == np.float32(np.abs(x[m].astype(np.float32)).max()) / np.float32(127)


def test_quantize_rounding_ties(orc):
    """Body (first K//8*8) rounds ties to even (vcvtnq), the tail away from 0."""
    L = orc.lib()
    # scale 1 -> inv 1; values k+0.5 are exact in fp16
    x = f16([0.5, 1.5, 2.5, -0.5, -2.5, 3.5, 4.0, 5.0, 0.5, 2.5, -2.5])
    q = np.empty(11, np.int8)
    L.orc_fp16_to_int8(orc.ptr(x), orc.ptr(q), 11, 1.0)
    assert list(q[:8]) == [0, 2, 2, 0, -2, 4, 4, 5]
    assert list(q[8:]) == [1, 3, -3]


def test_quantize_bounded_error(orc):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (8, 1000)).astype(np.float16)
    q, s = orc.quantize_activations(x.view(np.uint16))
    err = np.abs(q.astype(np.float64) - x.astype(np.float64) / s[:, None].astype(np.float64))
    assert err.max() <= 0.5 + 1e-5


# ----------------------------------------------------------------- a2/a3 matmul
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_group_sums_brute_force(orc, gs):
    rng = np.random.default_rng(5)
    M, K, N = 3, 256, 5
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (N, K), dtype=np.int8)
    acc = orc.group_sums_int8(A, B, gs)
    ref = np.einsum("mgk,ngk->mng", A.reshape(M, -1, gs).astype(np.int64),
                    B.reshape(N, -1, gs).astype(np.int64))
    assert (acc == ref).all()
    # B all ones -> group row sums of A; A one-hot -> column picks of B
    ones = np.ones((N, K), np.int8)
    assert (orc.group_sums_int8(A, ones, gs) == A.reshape(M, -1, gs).sum(-1)[:, None, :]).all()


def test_matmul_int8_reference_known_answer(orc):
    """tests/test_kernel.cpp:214-303 (grouped INT8 vs its definitional C_ref,
    M=2 K=128 N=4 g=64, abs tolerance 0.1), over several seeds."""
    for seed in range(10):
        rng = np.random.default_rng(100 + seed)
        M, K, N, gs = 2, 128, 4, 64
        A = ((rng.random((M, K)) - 0.5) * 0.5).astype(np.float16)
        B = (rng.integers(0, 128, (N, K)) - 64).astype(np.int8)
        Bs = np.empty((N, K // gs), np.float16)
        for n in range(N):
            for g in range(K // gs):
                s = np.abs(B[n, g * gs:(g + 1) * gs].astype(np.float32)).max() / np.float32(127)
                Bs[n, g] = max(s, np.float32(1e-6))
        q, As = orc.quantize_activations(A.view(np.uint16))
        C = orc.bits2f(orc.matmul_int8(q, As, B, Bs.view(np.uint16), gs))
        Cref = np.zeros((M, N))
        for m in range(M):
            a_s = max(np.abs(A[m].astype(np.float32)).max() / 127.0, 1e-10)
            aq = np.clip(np.round(A[m].astype(np.float64) / a_s), -128, 127)
            for n in range(N):
                for g in range(K // gs):
                    gsum = (aq[g * gs:(g + 1) * gs] * B[n, g * gs:(g + 1) * gs]).sum()
                    Cref[m, n] += gsum * a_s * float(Bs[n, g])
        assert np.abs(C - Cref).max() < 0.1


def test_matmul_epilogue_is_fused_chain(orc):
    """C = fp16(fma(acc1, s1, fl(acc0*s0)) * As): checked with exact float64
    arithmetic rounded once per step (G=2), over random cases."""
    rng = np.random.default_rng(6)
    K, gs = 64, 32
    for _ in range(300):
        A = rng.integers(-127, 128, (1, K), dtype=np.int8)
        B = rng.integers(-127, 128, (1, K), dtype=np.int8)
        Bs = f16(np.abs(rng.normal(0, 0.02, (1, 2))))
        As = np.array([rng.uniform(0.001, 0.05)], np.float32)
        acc = orc.group_sums_int8(A, B, gs)[0, 0]
        s0, s1 = h(Bs[0, 0]), h(Bs[0, 1])
        r0 = np.float32(float(acc[0]) * s0)               # fma with r=0: one rounding
        r1 = np.float32(float(acc[1]) * s1 + float(r0))   # exact in float64, one rounding
        ref = to16(float(np.float32(float(r1) * float(As[0]))))
        got = orc.matmul_int8(A, As, B, Bs, gs)[0, 0]
        assert got == ref


def test_int4_packing_and_equivalence(orc):
    """Nibble order of tests/test_kernel.cpp:323-330 and equality of the INT4
    kernel with the INT8 kernel on the unpacked codes (product-path identity)."""
    rng = np.random.default_rng(7)
    N, K, gs = 6, 128, 32
    codes = rng.integers(-8, 8, (N, K), dtype=np.int8)
    codes[0, :4] = [-8, 7, -1, 0]
    packed = pack_int4(codes)
    assert packed[0, 0] == 0x78 and packed[0, 1] == 0x0F
    un = np.empty(N * K, np.int8)
    orc.lib().orc_unpack_int4_to_int8(orc.ptr(packed), orc.ptr(un), N * K)
    assert (un.reshape(N, K) == codes).all()
    A = rng.integers(-127, 128, (3, K), dtype=np.int8)
    As = rng.uniform(0.001, 0.05, 3).astype(np.float32)
    Bs = f16(np.abs(rng.normal(0, 0.02, (N, K // gs))))
    assert (orc.matmul_int4(A, As, packed, Bs, gs) == orc.matmul_int8(A, As, codes, Bs, gs)).all()


# ----------------------------------------------------------------- a4 fp16 matmul
def test_matmul_f16_reference_known_answer(orc):
    """tests/test_graph.cpp:75-90: [[1,2,3],[4,5,6]] @ [[1,2],[3,4],[5,6]]."""
    a = f16([[1, 2, 3], [4, 5, 6]])
    bT = f16([[1, 3, 5], [2, 4, 6]])
    assert (orc.bits2f(orc.matmul_f16(a, bT)) == [[22, 28], [49, 64]]).all()


def test_matmul_f16_lane_tree(orc):
    """K=8: each lane holds one rounded product; the result is
    ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) with fp16 rounding at every add
    (kernel_gemm.cpp:8-15), evaluated here with numpy's fp16 conversion."""
    rng = np.random.default_rng(8)
    for _ in range(200):
        a = f16(rng.normal(0, 8, (1, 8)))
        b = f16(rng.normal(0, 8, (1, 8)))
        l = [h(to16(h(a[0, j]) * h(b[0, j]))) for j in range(8)]
        add = lambda x, y: h(to16(x + y))
        ref = to16(add(add(add(l[0], l[4]), add(l[2], l[6])), add(add(l[1], l[5]), add(l[3], l[7]))))
        assert orc.matmul_f16(a, b)[0, 0] == ref


def test_matmul_f16_fp16_accumulation(orc):
    """Accumulation in fp16: a long sum of 1.0 + many tiny terms stays 1.0 in
    every lane (fp32 accumulation would not)."""
    K = 1024
    a = f16(np.full((1, K), 1.0))
    b = np.full((1, K), 2.0 ** -12, np.float32)
    b[0, :8] = 1.0
    out = h(orc.matmul_f16(a, f16(b))[0, 0])
    assert out == 8.0


# ----------------------------------------------------------------- a5/a6 attention
def _blocked_poly_attention(q, k, v, scale):
    """Closed form of cactus_attention_f16 for one query row, float64:
    out = sum_b e^{m_b} sum_j P(s_j-m_b) v_j / sum_b e^{m_b} sum_j P(s_j-m_b),
    P = poly weight for the first floor(n/4)*4 keys of a block, exp otherwise."""
    L = len(k)
    s = (k @ q) * scale
    num = np.zeros(v.shape[1])
    den = 0.0
    for b0 in range(0, L, 32):
        sb = s[b0:b0 + 32]
        mb = sb.max()
        n = len(sb)
        w = np.empty(n)
        for j in range(n):
            if j < (n // 4) * 4:
                t = (sb[j] - mb) * 1.442695
                ti = math.trunc(t)
                f = t - ti
                w[j] = (1 + 0.6931472 * f + 0.2402265 * f * f) * 2.0 ** ti
            else:
                w[j] = math.exp(sb[j] - mb)
        num += math.exp(mb) * (w[:, None] * v[b0:b0 + 32]).sum(0)
        den += math.exp(mb) * w.sum()
    return num / den


def test_attention_f16_closed_form(orc):
    rng = np.random.default_rng(9)
    B, S, Hq, Hkv, d, L = 1, 1, 4, 2, 64, 77
    q = f16(rng.normal(0, 1, (B, S, Hq, d)))
    k = f16(rng.normal(0, 1, (B, L, Hkv, d)))
    v = f16(rng.normal(0, 1, (B, L, Hkv, d)))
    scale = 1.0 / math.sqrt(d)
    o = orc.bits2f(orc.attention_f16(q, k, v, scale, pos_off=L - 1))
    for hq in range(Hq):
        kv = hq // (Hq // Hkv)
        ref = _blocked_poly_attention(h(q[0, 0, hq]), h(k[0, :, kv]), h(v[0, :, kv]), scale)
        assert np.allclose(o[0, 0, hq], ref, rtol=2e-3, atol=2e-3)


def test_attention_special_cases(orc):
    d = 8
    # equal scores -> exact mean of V (integer values)
    q = f16(np.zeros((1, 1, 1, d)))
    k = f16(np.ones((1, 4, 1, d)))
    v = f16(np.arange(4 * d).reshape(1, 4, 1, d))
    o = orc.bits2f(orc.attention_f16(q, k, v, 1.0, pos_off=3))
    assert (o[0, 0, 0] == np.arange(4 * d).reshape(4, d).mean(0)).all()
    # causal S = Skv = 2: row 0 attends only to key 0 -> V0 exactly
    q = f16(np.random.default_rng(1).normal(0, 1, (1, 2, 1, d)))
    k = f16(np.random.default_rng(2).normal(0, 1, (1, 2, 1, d)))
    v = f16(np.random.default_rng(3).normal(0, 1, (1, 2, 1, d)))
    o = orc.attention_f16(q, k, v, 0.5)
    assert (o[0, 0, 0] == v[0, 0, 0]).all()
    # inputs of tests/test_graph.cpp:220-240 (no numeric assertion there): with
    # head_dim 4 the 8-wide vector prefix is empty, so the reference writes
    # zeros (kernel_attention.cpp:229-252)
    q = f16([[[[1, 0, 0, 0]], [[0, 1, 0, 0]]]])
    k = f16([[[[1, 0, 0, 0]], [[0, 1, 0, 0]]]])
    v = f16([[[[1, 2, 3, 4]], [[5, 6, 7, 8]]]])
    o = orc.bits2f(orc.attention_f16(q, k, v, 0.5))
    assert (o == 0).all()


def test_attention_hybrid_closed_form(orc):
    """INT8-cache attention is a plain softmax over dequantized keys/values
    (k = code*scale) and the fp16 new tokens (kernel_attention.cpp:257-482)."""
    rng = np.random.default_rng(10)
    Hq, Hkv, d, cache, new = 4, 2, 128, 70, 3
    kf = f16(rng.normal(0, 1, (cache, Hkv, d)))
    vf = f16(rng.normal(0, 1, (cache, Hkv, d)))
    kc, ks = orc.quantize_kv(kf)
    vc, vs = orc.quantize_kv(vf)
    kn = f16(rng.normal(0, 1, (1, new, Hkv, d)))
    vn = f16(rng.normal(0, 1, (1, new, Hkv, d)))
    q = f16(rng.normal(0, 1, (1, new, Hq, d)))
    scale = 1 / math.sqrt(d)
    o = orc.bits2f(orc.attention_hybrid(q, kc[None], vc[None], ks[None], vs[None], kn, vn, scale,
                                        pos_off=cache))
    kd = np.concatenate([(kc.astype(np.float32) * ks).astype(np.float64), h(kn[0])])
    vd = np.concatenate([(vc.astype(np.float32) * vs).astype(np.float64), h(vn[0])])
    for s in range(new):
        for hq in range(Hq):
            kv = hq // 2
            n = cache + s + 1
            sc = kd[:n, kv] @ h(q[0, s, hq]) * scale
            w = np.exp(sc - sc.max())
            ref = (w[:, None] * vd[:n, kv]).sum(0) / w.sum()
            assert np.allclose(o[0, s, hq], ref, rtol=2e-3, atol=2e-3)


# ----------------------------------------------------------------- a7 kv quant
def test_quantize_kv_closed_form(orc):
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, (5, 3, 128)).astype(np.float16)
    q, s = orc.quantize_kv(x.view(np.uint16))
    m = np.abs(x.astype(np.float32)).max(-1)
    assert (s[..., 0] == np.maximum(m / np.float32(127), np.float32(1e-10))).all()
    err = np.abs(q - x.astype(np.float64) / s.astype(np.float64))
    assert err.max() <= 0.5 + 1e-4
    assert (np.abs(q).max(-1) == 127).all()


# ----------------------------------------------------------------- a8-a12
def test_rms_norm_reference_known_answer(orc):
    """tests/test_graph.cpp:176-204 (1..8, eps 1e-5, tolerance 0.01)."""
    x = f16([[1, 2, 3, 4, 5, 6, 7, 8]])
    w = f16([1] * 8)
    y = orc.bits2f(orc.rms_norm(x, w, 1e-5))
    inv = 1 / math.sqrt(sum(i * i for i in range(1, 9)) / 8 + 1e-5)
    assert np.allclose(y[0], [i * inv for i in range(1, 9)], atol=0.01)


def test_rms_norm_two_fp16_multiplies(orc):
    rng = np.random.default_rng(12)
    for dims in (128, 1024):
        x = f16(rng.normal(0, 1, (4, dims)))
        w = f16(1 + rng.normal(0, 0.02, dims))
        y = orc.rms_norm(x, w, 1e-6)
        for r in range(4):
            ss = float((h(x[r]) ** 2).sum())
            inv16 = h(to16(1 / math.sqrt(ss / dims + 1e-6)))
            ref = [to16(h(to16(h(x[r, i]) * inv16)) * h(w[i])) for i in range(dims)]
            # ss is order-dependent in its last bits: allow 1 ulp of fp16
            assert np.abs(y[r].astype(np.int32) - np.array(ref, np.int32)).max() <= 1


def test_softmax_reference_known_answer(orc):
    """tests/test_graph.cpp:206-218 and test_kernel.cpp:137-158 (rows sum to 1)."""
    y = orc.bits2f(orc.softmax(f16([[1, 2, 3], [4, 5, 6]])))
    assert np.allclose(y, [[0.09003, 0.24473, 0.66524]] * 2, atol=0.01)
    y = orc.bits2f(orc.softmax(f16([[1, 2, 3], [2, 3, 4], [3, 4, 5], [4, 5, 6]])))
    assert np.allclose(y.sum(1), 1, atol=1e-2)


def test_softmax_fast_exp_closed_form(orc):
    rng = np.random.default_rng(13)
    x = f16(rng.normal(0, 2, (2, 96)))
    y = orc.bits2f(orc.softmax(x))
    L = orc.lib()
    for r in range(2):
        xf = h(x[r]).astype(np.float32)
        e = np.array([L.orc_fast_exp(float(np.float32(v - xf.max()))) for v in xf])
        assert np.allclose(y[r], e / e.sum(), rtol=2e-3, atol=1e-4)


def test_rope_identity_at_zero_and_rotation(orc):
    rng = np.random.default_rng(14)
    x = f16(rng.normal(0, 1, (1, 3, 2, 128)))
    y = orc.rope(x, 0, 1e6)
    assert (y[0, 0] == x[0, 0]).all()        # pos 0: cos 1, sin 0
    assert (y[0, 1] != x[0, 1]).any()        # test_kernel.cpp:161-184
    # closed form: rotate (x_i, x_{i+64}) by pos * theta^(-2i/d)
    for s in (1, 2):
        for hh in range(2):
            xs = h(x[0, s, hh])
            i = np.arange(64)
            ang = s * (1e6 ** (-(2.0 * i) / 128))
            r1 = xs[:64] * np.cos(ang) - xs[64:] * np.sin(ang)
            r2 = xs[64:] * np.cos(ang) + xs[:64] * np.sin(ang)
            got = orc.bits2f(y[0, s, hh])
            assert np.allclose(got, np.concatenate([r1, r2]), atol=4e-3, rtol=4e-3)


def test_silu_closed_form(orc):
    rng = np.random.default_rng(15)
    x = f16(rng.normal(0, 3, 1003))           # 1000 body + 3 expf tail
    y = orc.silu(x)
    L = orc.lib()
    for i in range(1003):
        xv = float(h(x[i]))
        e = L.orc_fast_exp(-xv) if i < 1000 else math.exp(-xv)
        ref = to16(xv / (1 + e))
        assert abs(int(y[i]) - ref) <= 1


def test_add_multiply_fp16(orc):
    rng = np.random.default_rng(16)
    a = f16(rng.normal(0, 10, 500))
    b = f16(rng.normal(0, 10, 500))
    assert (orc.add(a, b) == [to16(h(x) + h(y)) for x, y in zip(a, b)]).all()
    assert (orc.multiply(a, b) == [to16(h(x) * h(y)) for x, y in zip(a, b)]).all()


def test_argmax_first_index_wins(orc):
    logits = f16([0.5, 3.0, -1.0, 3.0, 2.9])
    assert orc.argmax(logits) == 1
    assert orc.argmax(f16([-np.inf, -5.0])) == 1


def test_embedding_rows_and_bounds(orc):
    table = f16(np.arange(20).reshape(5, 4))
    ids = np.array([3, 0, 4], np.float32)
    out = np.empty((3, 4), np.uint16)
    L = orc.lib()
    assert L.orc_embedding_f16(orc.ptr(table), orc.ptr(ids), orc.ptr(out), 3, 4, 5) == 0
    assert (out == table[[3, 0, 4]]).all()
    bad = np.array([5], np.float32)
    assert L.orc_embedding_f16(orc.ptr(table), orc.ptr(bad), orc.ptr(out), 1, 4, 5) != 0
