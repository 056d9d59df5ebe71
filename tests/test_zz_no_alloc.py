"""cactus_hip_matmul_int8_f16act_noalloc (static device scratch, no
allocation) against cactus_hip_matmul_int8_f16act, bit for bit, through the
C ABI: two calls in a row on the MFMA path (the second smaller, so stale
codes of the first would show), a GEMV-sized call, free device memory
unchanged across its calls on a fresh stream (with the allocating entry as
the control that the measurement sees an allocation), and a shape above the
static buffer refused before any launch."""
import ctypes

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


def _free_bytes(cm):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    cm.call("cactus_hip_device_memory", ctypes.byref(free), ctypes.byref(total))
    return free.value


def test_noalloc_allocates_no_device_memory(hip_ready):
    """Free device memory is unchanged across no-alloc calls on a stream
    that never ran the allocating entry; the same measurement sees the
    allocating entry's scratch grow on another fresh stream (the control)."""
    cm = hip_ready
    rng = np.random.default_rng(78)
    M, K, N, gs = 512, 1024, 3072, 32
    x = activations(rng, M, K)
    B, Bs = grouped_int8_weights(rng, N, K, gs)
    dx, dB, dBs = (cm.DeviceBuffer.from_numpy(a) for a in (x, B, Bs))
    dC = cm.DeviceBuffer(M * N * 2)
    # control inputs: M = 4096, K = 4096 needs 16 MiB of activation codes
    Mc, Kc, Nc = 4096, 4096, 64
    cx = cm.DeviceBuffer.from_numpy(activations(rng, Mc, Kc))
    cB, cBs = (cm.DeviceBuffer.from_numpy(a) for a in grouped_int8_weights(rng, Nc, Kc, gs))
    cC = cm.DeviceBuffer(Mc * Nc * 2)
    # the library's kernels loaded and the static buffer looked up (default stream)
    cm.call("cactus_hip_matmul_int8_f16act_noalloc", dx.ptr, dB.ptr, dBs.ptr, dC.ptr, M, K, N, gs, None)
    cm.call("cactus_hip_stream_sync", None)
    s1 = cm.Stream()
    cm.call("cactus_hip_memset", dC.ptr, 0, 256, s1.handle)      # the stream's queue in use
    s1.sync()
    free0 = _free_bytes(cm)
    say("noalloc free memory", free0)
    for m in (M, 64):
        cm.call("cactus_hip_matmul_int8_f16act_noalloc", dx.ptr, dB.ptr, dBs.ptr, dC.ptr, m, K, N, gs, s1.handle)
    s1.sync()
    free1 = _free_bytes(cm)
    assert free1 == free0, (free0, free1)
    # control: the allocating entry's per-stream scratch on a fresh stream
    s2 = cm.Stream()
    cm.call("cactus_hip_memset", cC.ptr, 0, 256, s2.handle)
    s2.sync()
    free2 = _free_bytes(cm)
    cm.call("cactus_hip_matmul_int8_f16act", cx.ptr, cB.ptr, cBs.ptr, cC.ptr, Mc, Kc, Nc, gs, s2.handle)
    s2.sync()
    free3 = _free_bytes(cm)
    say("allocating entry free memory", free2, "->", free3)
    assert free2 - free3 >= Mc * Kc, (free2, free3)


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
