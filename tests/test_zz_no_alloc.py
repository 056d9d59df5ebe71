"""cactus_hip_matmul_int8_f16act_noalloc (static device scratch, no
allocation) against cactus_hip_matmul_int8_f16act, bit for bit, through the
C ABI: two calls in a row on the MFMA path (the second smaller, so stale
codes of the first would show), a GEMV-sized call, and a shape above the
static buffer refused before any launch."""
import numpy as np
import pytest

from _data import activations, grouped_int8_weights

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def _both(cm, rng, M, K, N, gs):
    x = activations(rng, M, K)
    B, Bs = grouped_int8_weights(rng, N, K, gs)
    dx, dB, dBs = (cm.DeviceBuffer.from_numpy(a) for a in (x, B, Bs))
    c_ref, c_na = cm.DeviceBuffer(M * N * 2), cm.DeviceBuffer(M * N * 2)
    cm.call("cactus_hip_matmul_int8_f16act", dx.ptr, dB.ptr, dBs.ptr, c_ref.ptr, M, K, N, gs, None)
    cm.call("cactus_hip_matmul_int8_f16act_noalloc", dx.ptr, dB.ptr, dBs.ptr, c_na.ptr, M, K, N, gs, None)
    cm.call("cactus_hip_stream_sync", None)
    return c_ref.to_numpy(np.uint16, (M, N)), c_na.to_numpy(np.uint16, (M, N))


def test_noalloc_matches_allocating_entry(hip_ready):
    cm = hip_ready
    rng = np.random.default_rng(77)
    for M, K, N, gs in [(512, 1024, 3072, 32), (64, 640, 256, 64), (1, 640, 2048, 32)]:
        say("matmul_int8_f16act_noalloc", M, K, N, gs)
        ref, got = _both(cm, rng, M, K, N, gs)
        assert (ref == got).all(), (M, K, N, gs, int((ref != got).sum()))


def test_noalloc_refuses_shapes_above_its_buffer(hip_ready):
    cm = hip_ready
    M, K, N, gs = 4096, 1024, 64, 32
    say("matmul_int8_f16act_noalloc refusal", M, K)
    dx = cm.DeviceBuffer(M * K * 2)
    dB, dBs, dC = cm.DeviceBuffer(N * K), cm.DeviceBuffer(N * (K // gs) * 2), cm.DeviceBuffer(M * N * 2)
    lib = cm.hip()
    rc = lib.cactus_hip_matmul_int8_f16act_noalloc(dx.ptr, dB.ptr, dBs.ptr, dC.ptr, M, K, N, gs, None)
    assert rc != 0
    assert b"4 MiB" in lib.cactus_hip_last_error()
