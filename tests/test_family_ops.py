"""Ops of the other model families (GELU, GELU-erf, LayerNorm, conv1d).

CPU: the oracle (oracle/family_oracle.c) against what the mathematics
fixes: fast_tanh is a tanh approximation within 0.03 on [-4.5, 4.5] and
saturates beyond; GELU and GELU-erf lie within an fp16 ulp (plus the
approximation) of their float64 definitions and are exact at 0 and +-8;
LayerNorm of a constant row is the bias exactly and of random rows the
float64 definition within fp16 rounding; both convolutions equal numpy's
direct sums on integer data, where every order of summation is exact.

GPU: the HIP entry points against the oracle, bit for bit, on random fp16
data at model-like shapes.
"""
import ctypes
import math

import numpy as np
import pytest

from _data import f16


def say(*a):
    print("[case]", *a, flush=True)


def h2f(u):
    return np.asarray(u, np.uint16).view(np.float16).astype(np.float64)


# ------------------------------------------------------------------ CPU
def test_fast_tanh_is_a_tanh(orc):
    xs = np.linspace(-4.5, 4.5, 2001)
    err = max(abs(orc.fast_tanh(float(x)) - math.tanh(x)) for x in xs)
    assert err < 0.03
    assert orc.fast_tanh(4.6) == 1.0 and orc.fast_tanh(-4.6) == -1.0 and orc.fast_tanh(0.0) == 0.0
    assert all(orc.fast_tanh(float(x)) == -orc.fast_tanh(float(-x)) for x in xs[:50])


@pytest.mark.parametrize("n", [64, 69])
def test_gelu_against_definition(orc, n):
    x = f16(np.linspace(-6, 6, n))
    g = h2f(orc.gelu(x))
    xd = h2f(x)
    exact = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(g - exact) <= 0.02 * np.maximum(1, np.abs(xd)))
    tail = slice((n // 8) * 8, n)   # libm tanh there: one fp16 rounding away
    assert np.all(np.abs(g[tail] - exact[tail]) <= np.abs(exact[tail]) * 2 ** -10 + 2 ** -24)
    special = f16([0.0, 8.0, -8.0, 0.0, 8.0, -8.0, 0.0, 8.0, 0.0])
    out = orc.gelu(special)
    assert list(out) == list(f16([0.0, 8.0, -0.0, 0.0, 8.0, -0.0, 0.0, 8.0, 0.0]))


def test_gelu_erf_against_definition(orc):
    x = f16(np.linspace(-6, 6, 501))
    g = h2f(orc.gelu_erf(x))
    xd = h2f(x)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xd])
    # 1 + erff cancels in float for negative x (the reference's formula):
    # one float ulp of erf costs |x| * 2^-24 absolute, then the fp16 rounding
    assert np.all(np.abs(g - exact) <= np.abs(exact) * 2 ** -10 + np.abs(xd) * 2 ** -23 + 2 ** -24)
    assert list(orc.gelu_erf(f16([0.0, 9.0]))) == list(f16([0.0, 9.0]))


def test_layer_norm_against_definition(orc):
    rng = np.random.default_rng(4)
    F = 384
    w = f16(1 + rng.normal(0, 0.1, F))
    b = f16(rng.normal(0, 0.1, F))
    const = f16(np.full((2, F), 3.25))
    assert (orc.layer_norm(const, w, b, 1e-5) == np.stack([b, b])).all()
    x = f16(rng.normal(0.5, 2, (5, F)))
    y = h2f(orc.layer_norm(x, w, b, 1e-5))
    xd = h2f(x)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    exact = (xd - mu) / np.sqrt(var + 1e-5) * h2f(w) + h2f(b)
    assert np.all(np.abs(y - exact) <= np.abs(exact) * 2 ** -10 + 2e-3)


@pytest.mark.parametrize("K,dil", [(3, 1), (4, 2), (8, 1), (11, 3), (16, 1)])
def test_conv1d_causal_depthwise_integers(orc, K, dil):
    rng = np.random.default_rng(K * 10 + dil)
    N, L, C = 2, 37, 5
    x = rng.integers(-4, 5, (N, L, C)).astype(np.float64)
    w = rng.integers(-3, 4, (C, K)).astype(np.float64)
    y = h2f(orc.conv1d_causal_depthwise(f16(x), f16(w), dil))
    want = np.zeros((N, L, C))
    for t in range(L):
        for k in range(K):
            if t - k * dil >= 0:
                want[:, t, :] += w[:, K - 1 - k] * x[:, t - k * dil, :]
    assert (y == want).all()


@pytest.mark.parametrize("L,stride", [(31, 1), (32, 2), (7, 3)])
def test_conv1d_k3_integers(orc, L, stride):
    rng = np.random.default_rng(L + stride)
    N, Cin, Cout = 2, 19, 6
    x = rng.integers(-4, 5, (N, Cin, L)).astype(np.float64)
    w = rng.integers(-3, 4, (Cout, Cin, 3)).astype(np.float64)
    y = h2f(orc.conv1d_k3(f16(x), f16(w), stride))
    xp = np.pad(x, ((0, 0), (0, 0), (1, 1)))
    out_len = (L - 1) // stride + 1
    want = np.zeros((N, Cout, out_len))
    for o in range(out_len):
        t = o * stride
        want[:, :, o] = np.einsum("nij,oij->no", xp[:, :, t:t + 3], w)
    assert (y == want).all()


# ------------------------------------------------------------------ GPU
def _dev(cm, a):
    return cm.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def _get(cm, buf, like):
    cm.call("cactus_hip_stream_sync", None)
    return buf.to_numpy(like.dtype, like.shape)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 7, 4096, 300001])
def test_gelu_matches_oracle(hip_ready, orc, n):
    cm = hip_ready
    x = f16(np.random.default_rng(n).normal(0, 3, n))
    say("gelu", n)
    for name, fn in (("cactus_hip_gelu_f16", orc.gelu), ("cactus_hip_gelu_erf_f16", orc.gelu_erf)):
        want = fn(x)
        d, o = _dev(cm, x), cm.DeviceBuffer(x.nbytes)
        cm.call(name, d.ptr, o.ptr, n, None)
        assert (_get(cm, o, want) == want).all(), name


@pytest.mark.gpu
@pytest.mark.parametrize("rows,F", [(1, 1280), (37, 384), (1500, 1280), (3, 7)])
def test_layer_norm_matches_oracle(hip_ready, orc, rows, F):
    cm = hip_ready
    rng = np.random.default_rng(rows + F)
    x = f16(rng.normal(0.3, 2, (rows, F)))
    w = f16(1 + rng.normal(0, 0.1, F))
    b = f16(rng.normal(0, 0.1, F))
    say("layer_norm", rows, F)
    want = orc.layer_norm(x, w, b, 1e-5)
    o = cm.DeviceBuffer(x.nbytes)
    dx, dw, db = _dev(cm, x), _dev(cm, w), _dev(cm, b)   # alive until the kernel has run
    cm.call("cactus_hip_layer_norm_f16", dx.ptr, dw.ptr, db.ptr, o.ptr, rows, F, ctypes.c_float(1e-5), None)
    assert (_get(cm, o, want) == want).all()


@pytest.mark.gpu
@pytest.mark.parametrize("N,L,C,K,dil", [(1, 256, 1024, 3, 1), (2, 100, 64, 8, 1), (1, 50, 33, 11, 2),
                                         (1, 17, 16, 16, 3)])
def test_conv1d_causal_depthwise_matches_oracle(hip_ready, orc, N, L, C, K, dil):
    cm = hip_ready
    rng = np.random.default_rng(L + C + K)
    x = f16(rng.normal(0, 1, (N, L, C)))
    w = f16(rng.normal(0, 0.5, (C, K)))
    say("conv1d depthwise", N, L, C, K, dil)
    want = orc.conv1d_causal_depthwise(x, w, dil)
    o = cm.DeviceBuffer(x.nbytes)
    dx, dw = _dev(cm, x), _dev(cm, w)
    cm.call("cactus_hip_conv1d_causal_depthwise_f16", dx.ptr, dw.ptr, o.ptr, N, L, C, K, dil, None)
    assert (_get(cm, o, want) == want).all()


@pytest.mark.gpu
@pytest.mark.parametrize("N,Cin,Cout,L,stride", [(1, 80, 384, 300, 1), (1, 384, 384, 300, 2), (2, 19, 7, 31, 3)])
def test_conv1d_k3_matches_oracle(hip_ready, orc, N, Cin, Cout, L, stride):
    cm = hip_ready
    rng = np.random.default_rng(Cin + Cout + L)
    x = f16(rng.normal(0, 1, (N, Cin, L)))
    w = f16(rng.normal(0, 0.1, (Cout, Cin, 3)))
    say("conv1d k3", N, Cin, Cout, L, stride)
    want = orc.conv1d_k3(x, w, stride)
    o = cm.DeviceBuffer(want.nbytes)
    dx, dw = _dev(cm, x), _dev(cm, w)
    cm.call("cactus_hip_conv1d_f16_k3", dx.ptr, dw.ptr, o.ptr, N, L, Cin, Cout, stride, None)
    assert (_get(cm, o, want) == want).all()
