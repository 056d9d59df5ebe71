#!/usr/bin/env python3
"""Benchmark of the quantized kernel layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline: INT8 grouped GEMV throughput (GB/s and fraction of the 8 TB/s HBM
peak) on the Gemma-3-270m MLP up-projection shape M=1, K=640, N=2048, group
32, with FP16 activations quantized in-kernel.  One step is one launch of the
strided-batched GEMV over R distinct weight sets (R x 1.4 MB > 1 GiB, so the
256 MB Infinity Cache cannot hold them): every launch streams its weights
from HBM.  Inputs are resident in HBM before the timed region starts.

The same JSON line carries the CPU baseline: the CPU restatement of the
reference kernel (oracle/, x86 build) timed on this host on a bounded sample
of the same workload, with the reference's M=1 thread policy
(min(pool, 4) threads, kernel_utils.h:446-453); the host's core count and
CPU model; and the other workloads the kernel layer is quoted on:

  int4_gemv           INT4 GEMV M=1 K=3072 N=1024 g32, 604 rotated weight sets
  prefill_gemm        INT8 M=512 K=1024 N=3072 and INT4 K=3072 N=1024 M=256/1
  decode_attention    one decode query over 4096 positions, INT8 cache and
                      FP16 K/V, exact and tolerance (split-K) modes, rotated
                      over >= 1 GiB of caches
  qwen3_0p6b_decode   Qwen3-0.6B-shape 4096-token prefill + 128 greedy steps,
                      exact attention (tokens compared with the oracle's
                      frozen run) and tolerance attention
  qwen3_0p6b_decode_cpu_baseline   the oracle model's decode on the host
  qwen3_0p6b_prefill_cpu_baseline  the oracle model's prefill of 512 prompt
                                   tokens on the host

Every other leg carries its own `cpu_baseline` beside its GPU figure, timed
with the reference's thread policy: the INT8 M=512 matmul (whole pool), INT4
M=1 (one thread: N < 5000) and M=256 (whole pool), and decode attention over
both cache forms (one thread: 16 work items, below the ATTENTION threshold).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0

# Gemma-3-270m MLP up-projection GEMV
M, K, N, GS = 1, 640, 2048, 32
SET_BYTES = N * K + 2 * N * (K // GS) + 2 * K + 2 * N   # 1,398,016 algorithmic bytes


def gemv_sets(R: int, seed: int = 1):
    """Device buffers for R distinct GEMV problems (weights at distinct addresses)."""
    import cactus_amd as cm
    from _data import f16
    rng = np.random.default_rng(seed)
    # 64 MiB of random codes, tiled over the R weight sets at distinct addresses
    pool = rng.integers(-127, 128, size=(48, N, K), dtype=np.int8)
    B = cm.DeviceBuffer(R * N * K)
    chunk = pool.reshape(-1)
    per = pool.shape[0]
    for r0 in range(0, R, per):
        n = min(per, R - r0)
        cm.call("cactus_hip_memcpy_h2d", B.ptr + r0 * N * K, chunk.ctypes.data, n * N * K, None)
    Bs = cm.DeviceBuffer.from_numpy(
        f16(np.abs(rng.normal(0, 0.02, size=(R, N, K // GS))) / 127.0))
    A = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, size=(R, M, K))))
    C = cm.DeviceBuffer(R * M * N * 2)
    return A, B, Bs, C


def bench_gemv(steps: int, warmup: int, R: int = 768, sets=None):
    import cactus_amd as cm
    A, B, Bs, C = sets if sets is not None else gemv_sets(R)
    stream = cm.Stream()

    def launch():
        cm.call("cactus_hip_matmul_int8_f16act_batched", A.ptr, B.ptr, Bs.ptr, C.ptr, M, K, N, GS, R,
                M * K, N * K, N * (K // GS), M * N, stream.handle)

    for _ in range(warmup):
        launch()
    stream.sync()
    e0, e1 = cm.Event(), cm.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        launch()
    e1.record(stream)
    stream.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    per_launch_s = ms / 1e3 / steps
    gbs = R * SET_BYTES / per_launch_s / 1e9
    return {"gbs": gbs, "ms_per_step": ms / steps, "wall_s": wall, "R": R}


INT8_MFMA_PEAK_TOPS = 5000.0   # MI355X dense INT8 MFMA

# Qwen3-0.6B down-projection GEMV, packed INT4 (config 3 at M=1)
K4, N4 = 3072, 1024
SET_BYTES_INT4 = N4 * K4 // 2 + 2 * N4 * (K4 // GS) + 2 * K4 + 2 * N4   # 1,777,664 algorithmic bytes


INT4_STEPS, INT4_WARMUP = 50, 100   # the INT4 GEMV leg's own launch counts


def gemv_int4_sets(R: int = 604):
    """Device buffers for R distinct INT4 GEMV problems."""
    import cactus_amd as cm
    from _data import f16
    rng = np.random.default_rng(3)
    per = N4 * K4 // 2
    pool = rng.integers(0, 256, size=(32, per), dtype=np.uint8)
    B = cm.DeviceBuffer(R * per)
    for r0 in range(0, R, pool.shape[0]):
        n = min(pool.shape[0], R - r0)
        cm.call("cactus_hip_memcpy_h2d", B.ptr + r0 * per, pool.ctypes.data, n * per, None)
    Bs = cm.DeviceBuffer.from_numpy(f16(np.abs(rng.normal(0, 0.02, size=(R, N4, K4 // GS))) / 7.0))
    A = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, size=(R, 1, K4))))
    C = cm.DeviceBuffer(R * N4 * 2)
    return A, B, Bs, C


def bench_gemv_int4(steps: int, warmup: int, R: int = 604, sets=None):
    """INT4 grouped GEMV M=1 K=3072 N=1024 g32 through the streaming GEMV:
    one launch of the strided-batched entry over R distinct weight sets
    (R x 1.78 MB > 1 GiB, so every launch streams from HBM)."""
    import cactus_amd as cm
    A, B, Bs, C = sets if sets is not None else gemv_int4_sets(R)
    per = N4 * K4 // 2
    stream = cm.Stream()

    def launch():
        cm.call("cactus_hip_matmul_int4_f16act_batched", A.ptr, B.ptr, Bs.ptr, C.ptr, 1, K4, N4, GS, R,
                K4, per, N4 * (K4 // GS), N4, stream.handle)

    for _ in range(warmup):
        launch()
    stream.sync()
    e0, e1 = cm.Event(), cm.Event()
    e0.record(stream)
    for _ in range(steps):
        launch()
    e1.record(stream)
    stream.sync()
    us = e0.elapsed_ms(e1) * 1e3 / steps
    gbs = R * SET_BYTES_INT4 / (us * 1e-6) / 1e9
    return {"workload": f"INT4 grouped GEMV M=1 K=3072 N=1024 group 32, FP16 activations quantized in-kernel; "
                        f"one launch over {R} distinct weight sets",
            "steps": steps, "warmup": warmup,
            "bytes_per_set": SET_BYTES_INT4, "sets_per_launch": R, "us_per_launch": round(us, 2),
            "gbs": round(gbs, 1), "hbm_fraction": round(gbs / HBM_PEAK_GBS, 4)}


# KV-cache decode attention (config 4): 16 query / 8 KV heads, head_dim 128,
# 4096 positions, one query row
ATT_HQ, ATT_HKV, ATT_D, ATT_CTX = 16, 8, 128, 4096
ATT_BYTES_F16 = 2 * ATT_CTX * ATT_HKV * ATT_D * 2 + 4 * ATT_HQ * ATT_D                 # 16,785,408
ATT_BYTES_INT8 = 2 * ATT_CTX * ATT_HKV * ATT_D + 2 * ATT_CTX * ATT_HKV * 4 + 4 * ATT_HQ * ATT_D  # 8,658,944


def _graph_time(fn, launches, rounds=4):
    """us per call of `launches` calls captured into one HIP graph."""
    import cactus_amd as cm
    st = fn.stream
    for i in range(min(launches, 4)):
        fn(i)
    st.sync()
    cm.call("cactus_hip_graph_capture_begin", st.handle)
    for i in range(launches):
        fn(i)
    ge = ctypes.c_void_p()
    cm.call("cactus_hip_graph_capture_end", st.handle, ctypes.byref(ge))
    cm.call("cactus_hip_graph_launch", ge, st.handle)
    st.sync()
    e0, e1 = cm.Event(), cm.Event()
    e0.record(st)
    for _ in range(rounds):
        cm.call("cactus_hip_graph_launch", ge, st.handle)
    e1.record(st)
    st.sync()
    cm.call("cactus_hip_graph_destroy", ge)
    return e0.elapsed_ms(e1) * 1e3 / (launches * rounds)


def bench_attention():
    """Config 4 in both attention modes and both cache forms: each call one
    decode query over 4096 positions; R distinct caches rotated (>= 1 GiB) so
    every call streams its cache from HBM; timed as a HIP graph of R calls.
    Also a single-set form (the same cache every call: L2/MALL-resident) and
    a single-shot latency (one call between two events)."""
    import cactus_amd as cm
    from _data import f16
    rng = np.random.default_rng(5)
    Hq, Hkv, d, ctx = ATT_HQ, ATT_HKV, ATT_D, ATT_CTX
    scale = ctypes.c_float(d ** -0.5)
    st = cm.Stream()
    out = {}
    # INT8 cache (cache 4095 + one FP16 new row): the hybrid entry points
    R8 = 124
    cache = ctx - 1
    row = cache * Hkv * d
    codes = rng.integers(-127, 128, (row,), dtype=np.int8)
    kc, vc = cm.DeviceBuffer(R8 * row), cm.DeviceBuffer(R8 * row)
    for r in range(R8):
        cm.call("cactus_hip_memcpy_h2d", kc.ptr + r * row, codes.ctypes.data, row, None)
        cm.call("cactus_hip_memcpy_h2d", vc.ptr + r * row, codes.ctypes.data, row, None)
    sc = np.abs(rng.normal(0, 0.02, (R8, cache, Hkv, 1))).astype(np.float32)
    sbytes = sc[0].nbytes
    ks, vs = cm.DeviceBuffer.from_numpy(sc), cm.DeviceBuffer.from_numpy(sc)
    kn = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, (R8, 1, Hkv, d))))
    vn = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, (R8, 1, Hkv, d))))
    q = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, (R8, 1, Hq, d))))
    o = cm.DeviceBuffer(R8 * Hq * d * 2)
    for mode, name in (("exact", "cactus_hip_attention_hybrid_int8_fp16"),
                       ("tolerance", "cactus_hip_attention_hybrid_int8_fp16_fast")):
        def call(i, rot=True, name=name):
            r = i % R8 if rot else 0
            cm.call(name, q.ptr + r * Hq * d * 2, kc.ptr + r * row, vc.ptr + r * row, ks.ptr + r * sbytes,
                    vs.ptr + r * sbytes, kn.ptr + r * Hkv * d * 2, vn.ptr + r * Hkv * d * 2, o.ptr + r * Hq * d * 2,
                    1, 1, cache, 1, Hq, Hkv, d, scale, cache, 1, 128, st.handle)
        call.stream = st
        us = _graph_time(call, R8)
        res = lambda i, call=call: call(i, rot=False)
        res.stream = st
        us_res = _graph_time(res, 50)
        e0, e1 = cm.Event(), cm.Event()
        st.sync()
        e0.record(st)
        call(0)
        e1.record(st)
        st.sync()
        one = e0.elapsed_ms(e1) * 1e3
        out[f"int8_cache_{mode}"] = {
            "us_per_call": round(us, 2), "gbs": round(ATT_BYTES_INT8 / us / 1e3, 1),
            "hbm_fraction": round(ATT_BYTES_INT8 / us / 1e3 / HBM_PEAK_GBS, 4),
            "us_per_call_l2_mall_resident": round(us_res, 2), "us_single_shot": round(one, 2)}
    del kc, vc, ks, vs
    # FP16 K/V (4096 positions): the FP16 entry points
    R16 = 64
    row16 = ctx * Hkv * d
    kv = f16(rng.normal(0, 1, (row16,)))
    k16, v16 = cm.DeviceBuffer(R16 * row16 * 2), cm.DeviceBuffer(R16 * row16 * 2)
    for r in range(R16):
        cm.call("cactus_hip_memcpy_h2d", k16.ptr + r * row16 * 2, kv.ctypes.data, row16 * 2, None)
        cm.call("cactus_hip_memcpy_h2d", v16.ptr + r * row16 * 2, kv.ctypes.data, row16 * 2, None)
    for mode, name in (("exact", "cactus_hip_attention_f16"), ("tolerance", "cactus_hip_attention_f16_fast")):
        def call(i, rot=True, name=name):
            r = i % R16 if rot else 0
            cm.call(name, q.ptr + (r % R8) * Hq * d * 2, k16.ptr + r * row16 * 2, v16.ptr + r * row16 * 2,
                    o.ptr, 1, 1, ctx, Hq, Hkv, d, scale, None, ctx - 1, 0, 1, st.handle)
        call.stream = st
        us = _graph_time(call, R16)
        res = lambda i, call=call: call(i, rot=False)
        res.stream = st
        us_res = _graph_time(res, 50)
        out[f"fp16_{mode}"] = {
            "us_per_call": round(us, 2), "gbs": round(ATT_BYTES_F16 / us / 1e3, 1),
            "hbm_fraction": round(ATT_BYTES_F16 / us / 1e3 / HBM_PEAK_GBS, 4),
            "us_per_call_l2_mall_resident": round(us_res, 2)}
    out["workload"] = (f"decode attention, one query, {Hq} query / {Hkv} KV heads, head_dim {d}, {ctx} positions; "
                       f"INT8 cache ({ATT_BYTES_INT8} B/call, {R8} caches rotated) and FP16 K/V "
                       f"({ATT_BYTES_F16} B/call, {R16} rotated); exact = the reference's operation order, "
                       f"tolerance = split-K (within 1e-3 + 1e-2|ref|)")
    return out


def exact_ceiling_us(M: int, K: int, N: int, gs: int) -> float:
    """Lower bound on a grouped matmul that keeps the reference's exact
    epilogue (kernel_gemm.cpp:311-324): per output and group one int32 ->
    fp32 convert and one fp32 FMA (the fp16 scale enters a mixed-precision
    FMA unconverted), i.e. 2 M N K/gs VALU lane operations; a wave64 VALU
    instruction occupies a SIMD for 4 cycles, so on MI355X's 1024 SIMDs at
    2.4 GHz they take 2 M N (K/gs) / 64 * 4 / 1024 / 2.4e9 s.  The integer
    group sums (2 M N K ops on MFMA at the 5.0 POP/s dense INT8 peak) and the
    operand traffic (A, B and C once at 8 TB/s) run beside it on other units;
    the bound is the largest of the three."""
    valu = 2.0 * M * N * (K // gs) / 64 * 4 / 1024 / 2.4e9
    mfma = 2.0 * M * N * K / (INT8_MFMA_PEAK_TOPS * 1e12)
    hbm = (M * K * 2 + N * K + 2 * N * (K // gs) + 2 * M * N) / (HBM_PEAK_GBS * 1e9)
    return max(valu, mfma, hbm) * 1e6


def bench_gemm(M: int, K: int, N: int, gs: int, int4: bool, f16act: bool, reps: int = 50, rounds: int = 5,
               eager: bool = False):
    """One grouped matmul (the reference's compute_matmul_node: FP16
    activations quantized per row, then the INT8/INT4 grouped matmul; or the
    matmul alone on pre-quantized activations), timed as a HIP graph of
    `reps` launches replayed `rounds` times, so host call overhead stays
    out of the per-call time."""
    ceiling = exact_ceiling_us(M, K, N, gs)
    import cactus_amd as cm
    from _data import f16
    rng = np.random.default_rng(M + K + N)
    A16 = cm.DeviceBuffer.from_numpy(f16(rng.normal(0, 1, (M, K))))
    A8 = cm.DeviceBuffer.from_numpy(rng.integers(-127, 128, (M, K), dtype=np.int8))
    As = cm.DeviceBuffer.from_numpy(np.abs(rng.normal(0, 0.01, M)).astype(np.float32))
    if int4:
        B = cm.DeviceBuffer.from_numpy(rng.integers(0, 256, (N, K // 2), dtype=np.uint8))
    else:
        B = cm.DeviceBuffer.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8))
    Bs = cm.DeviceBuffer.from_numpy(f16(np.abs(rng.normal(0, 0.02, (N, K // gs))) / 127.0))
    C = cm.DeviceBuffer(M * N * 2)
    st = cm.Stream()
    name = "cactus_hip_matmul_int4" if int4 else "cactus_hip_matmul_int8"
    if f16act:
        def fn():
            cm.call(name + "_f16act", A16.ptr, B.ptr, Bs.ptr, C.ptr, M, K, N, gs, st.handle)
    else:
        def fn():
            cm.call(name, A8.ptr, As.ptr, B.ptr, Bs.ptr, C.ptr, M, K, N, gs, st.handle)
    for _ in range(3):
        fn()   # first call sizes the activation scratch outside the capture
    st.sync()
    if eager:
        # direct launches (kernel tracers); the per-call time then includes
        # host call overhead
        e0, e1 = cm.Event(), cm.Event()
        e0.record(st)
        for _ in range(reps * rounds):
            fn()
        e1.record(st)
        st.sync()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * rounds)
        tops = 2.0 * M * K * N / (us * 1e-6) / 1e12
        return {"us_per_call": round(us, 2), "tops": round(tops, 1),
                "frac_int8_mfma_peak": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                "exact_ceiling_us": round(ceiling, 3), "frac_of_exact_ceiling": round(ceiling / us, 4),
                "timing": "direct launches"}
    def graph_us(branches):
        """us per call of a graph holding len(branches) chains of `reps`
        calls, chain i on stream branches[i][0] (forked from and joined
        back to `st`), replayed `rounds` times"""
        fork, joins = cm.Event(), [cm.Event() for _ in branches]
        cm.call("cactus_hip_graph_capture_begin", st.handle)
        fork.record(st)
        for bs, _ in branches:
            if bs is not st:
                cm.call("cactus_hip_stream_wait_event", bs.handle, fork.handle)
        for _, bfn in branches:
            for _ in range(reps):
                bfn()
        for (bs, _), j in zip(branches, joins):
            if bs is not st:
                j.record(bs)
                cm.call("cactus_hip_stream_wait_event", st.handle, j.handle)
        ge = ctypes.c_void_p()
        cm.call("cactus_hip_graph_capture_end", st.handle, ctypes.byref(ge))
        cm.call("cactus_hip_graph_launch", ge, st.handle)
        st.sync()
        e0, e1 = cm.Event(), cm.Event()
        e0.record(st)
        for _ in range(rounds):
            cm.call("cactus_hip_graph_launch", ge, st.handle)
        e1.record(st)
        st.sync()
        cm.call("cactus_hip_graph_destroy", ge)
        return e0.elapsed_ms(e1) * 1e3 / (reps * rounds * len(branches))

    def rate(us):
        tops = 2.0 * M * K * N / (us * 1e-6) / 1e12
        return {"us_per_call": round(us, 2), "tops": round(tops, 1),
                "frac_int8_mfma_peak": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                "exact_ceiling_us": round(ceiling, 3), "frac_of_exact_ceiling": round(ceiling / us, 4)}

    out = rate(graph_us([(st, fn)]))
    # three independent calls in flight, one per stream (each with its own
    # output and activation scratch), the way the overlapped prefill runs its
    # chunks' matmuls: aggregate rate with the launch latency overlapped
    extra = []
    for _ in range(2):
        s2, C2 = cm.Stream(), cm.DeviceBuffer(M * N * 2)
        if f16act:
            def f2(s2=s2, C2=C2):
                cm.call(name + "_f16act", A16.ptr, B.ptr, Bs.ptr, C2.ptr, M, K, N, gs, s2.handle)
        else:
            def f2(s2=s2, C2=C2):
                cm.call(name, A8.ptr, As.ptr, B.ptr, Bs.ptr, C2.ptr, M, K, N, gs, s2.handle)
        for _ in range(3):
            f2()   # sizes this stream's activation scratch outside the capture
        s2.sync()
        extra.append((s2, f2, C2))
    out["three_streams"] = rate(graph_us([(st, fn)] + [(e[0], e[1]) for e in extra]))
    return out


def bench_prefill_gemms(eager: bool = False):
    """Prefill matmul shapes: Qwen3-0.6B MLP gate/up (INT8, M=512) and
    down-proj (INT4, M=256 prefill and M=1 decode)."""
    out = {"int8_m512_k1024_n3072_g32": {
        "workload": "INT8 grouped matmul M=512 K=1024 N=3072 group 32, FP16 activations quantized per row",
        **bench_gemm(512, 1024, 3072, 32, False, True, eager=eager),
        "matmul_only": bench_gemm(512, 1024, 3072, 32, False, False, eager=eager)}}
    out["int4_k3072_n1024_g32"] = {
        "workload": "INT4 grouped matmul K=3072 N=1024 group 32, FP16 activations quantized per row",
        "m256": bench_gemm(256, 3072, 1024, 32, True, True, eager=eager),
        "m1": bench_gemm(1, 3072, 1024, 32, True, True, eager=eager)}
    return out


def measured_traffic():
    """HBM bytes per GEMV launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated),
    as recorded by the rocprofv3 counter runs summarised in
    profiles/gemv_int8_traffic.md (line 'traffic_bytes_per_launch: N')."""
    f = ROOT / "profiles" / "gemv_int8_traffic.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def cpu_baseline(seconds: float = 10.0, nsets: int = 768):
    """Reference-restated CPU GEMV (oracle build) on this host, streaming
    `nsets` distinct weight sets (about 1 GiB, as the GPU line) so that the
    host's caches do not hold them: one GEMV per set in turn."""
    import oracle
    from _data import activations, grouped_int8_weights
    L = oracle.lib()
    threads = min(4, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(11)
    x = activations(rng, M, K)
    B0, Bs0 = grouped_int8_weights(rng, N, K, GS)
    # distinct codes per set (any byte is a valid INT8 code); the scales keep
    # the seeded distribution, one copy per set
    Bw = np.frombuffer(rng.bytes(nsets * N * K), np.int8).reshape(nsets, N, K)
    Bsw = np.ascontiguousarray(np.broadcast_to(Bs0, (nsets,) + Bs0.shape))
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    C = np.empty((M, N), np.uint16)
    P = oracle.ptr
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        i = n % nsets
        L.orc_quantize_activations(P(x), P(q), P(s), M, K)
        L.orc_matmul_int8_mt(P(q), P(s), P(Bw[i]), P(Bsw[i]), P(C), M, K, N, GS, threads)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n * SET_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} GEMVs M=1 K=640 N=2048 g=32 over {nsets} distinct weight sets "
                      f"({nsets * SET_BYTES / 2**30:.2f} GiB, streamed in turn) in {dt:.1f} s, "
                      f"x86 build of the CPU restatement, {threads} threads (the reference's M=1 pool)"}


def cpu_gemm_baseline(seconds: float = 10.0, M: int = 512, K: int = 1024, N: int = 3072, gs: int = 32):
    """The prefill matmul of config 2 on this host's cores: per-row
    activation quantization, then the grouped INT8 matmul of the CPU
    restatement with the reference's M > 1 thread policy (the whole pool,
    kernel_utils.h:439-456), timed until `seconds` pass (at least once)."""
    import oracle
    from _data import f16
    L = oracle.lib()
    threads = min(16, os.cpu_count() or 1)
    rng = np.random.default_rng(M + K + N)
    x = f16(rng.normal(0, 1, (M, K)))
    B = rng.integers(-127, 128, (N, K), dtype=np.int8)
    Bs = f16(np.abs(rng.normal(0, 0.02, (N, K // gs))) / 127.0)
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    C = np.empty((M, N), np.uint16)
    P = oracle.ptr
    n = 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        L.orc_quantize_activations(P(x), P(q), P(s), M, K)
        L.orc_matmul_int8_mt(P(q), P(s), P(B), P(Bs), P(C), M, K, N, gs, threads)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(2.0 * M * K * N * n / dt / 1e12, 4), "unit": "TOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{n} calls of the INT8 M={M} K={K} N={N} g{gs} matmul with FP16 activations "
                      f"quantized per row, {dt:.1f} s, x86 build of the CPU restatement, {threads} threads"}


def cpu_int4_gemv_baseline(seconds: float = 5.0, nsets: int = 604):
    """Config 3 at M=1 (INT4 K=3072 N=1024 g32) on one host core: the
    reference runs the M=1 INT4 path through parallel_for over N columns
    with the ELEMENT_WISE threshold (kernel_gemm.cpp:354-358,
    kernel_utils.h:419-431), which keeps N=1024 on a single thread.  The
    activation row is quantized per call, and `nsets` distinct packed weight
    sets (about 1 GiB, as the GPU leg) are streamed in turn."""
    import oracle
    from _data import f16
    L = oracle.lib()
    L.orc_set_threads(1)
    rng = np.random.default_rng(31)
    per = N4 * K4 // 2
    Bw = np.frombuffer(rng.bytes(nsets * per), np.uint8).reshape(nsets, per)
    Bs = f16(np.abs(rng.normal(0, 0.02, size=(N4, K4 // GS))) / 7.0)
    x = f16(rng.normal(0, 1, size=(1, K4)))
    q = np.empty((1, K4), np.int8)
    s = np.empty(1, np.float32)
    C = np.empty((1, N4), np.uint16)
    P = oracle.ptr
    n = 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        L.orc_quantize_activations(P(x), P(q), P(s), 1, K4)
        L.orc_matmul_int4(P(q), P(s), P(Bw[n % nsets]), P(Bs), P(C), 1, K4, N4, GS)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n * SET_BYTES_INT4 / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "us_per_call": round(dt / n * 1e6, 1),
            "sample": f"{n} INT4 GEMVs M=1 K={K4} N={N4} g{GS} (activation row quantized per call) over "
                      f"{nsets} distinct packed weight sets streamed in turn, {dt:.1f} s, x86 build of the "
                      f"CPU restatement, 1 thread (the reference's M=1 policy at N < 5000)"}


def cpu_int4_m256_baseline(seconds: float = 5.0, M: int = 256):
    """Config 3 at M=256 on the host's pool (the reference tiles M > 1 over
    every pool thread, kernel_gemm.cpp:380 with kernel_utils.h:439-456):
    per-row activation quantization, then the INT4 grouped matmul."""
    import oracle
    from _data import f16
    L = oracle.lib()
    threads = min(16, os.cpu_count() or 1)
    L.orc_set_threads(threads)
    rng = np.random.default_rng(32)
    Bp = rng.integers(0, 256, (N4, K4 // 2), dtype=np.uint8)
    Bs = f16(np.abs(rng.normal(0, 0.02, size=(N4, K4 // GS))) / 7.0)
    x = f16(rng.normal(0, 1, size=(M, K4)))
    q = np.empty((M, K4), np.int8)
    s = np.empty(M, np.float32)
    C = np.empty((M, N4), np.uint16)
    P = oracle.ptr
    n = 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        L.orc_quantize_activations(P(x), P(q), P(s), M, K4)
        L.orc_matmul_int4(P(q), P(s), P(Bp), P(Bs), P(C), M, K4, N4, GS)
        n += 1
    dt = time.perf_counter() - t0
    L.orc_set_threads(1)
    return {"value": round(2.0 * M * K4 * N4 * n / dt / 1e12, 5), "unit": "TOP/s", "cores": threads,
            "kind": "port", "us_per_call": round(dt / n * 1e6, 1),
            "sample": f"{n} calls of the INT4 M={M} K={K4} N={N4} g{GS} matmul with FP16 activations "
                      f"quantized per row, {dt:.1f} s, x86 build of the CPU restatement, {threads} threads"}


def cpu_attention_baselines(seconds: float = 5.0):
    """Config 4 on one host core, both cache forms: one decode query (16
    query / 8 KV heads, head_dim 128) over 4095 INT8 cached positions plus
    one FP16 new row, and over 4096 FP16 positions.  The reference splits
    the batch * heads * rows = 16 work items with the ATTENTION threshold
    (kernel_attention.cpp:45 and :299, kernel_utils.h:419-431), so decode
    attention runs on one thread.  Distinct caches are rotated so that the
    host's caches do not hold them."""
    import oracle
    from _data import f16
    L = oracle.lib()
    L.orc_set_threads(1)
    rng = np.random.default_rng(33)
    Hq, Hkv, d, ctx = ATT_HQ, ATT_HKV, ATT_D, ATT_CTX
    P = oracle.ptr
    scale = d ** -0.5
    out = {}
    q = f16(rng.normal(0, 1, (1, Hq, d)))
    o = np.empty((1, Hq, d), np.uint16)
    # INT8 cache: 4095 cached positions + 1 new row
    R8, cache = 32, ctx - 1
    kc = rng.integers(-127, 128, (R8, cache, Hkv, d), dtype=np.int8)
    vc = rng.integers(-127, 128, (R8, cache, Hkv, d), dtype=np.int8)
    ks = np.abs(rng.normal(0, 0.02, (R8, cache, Hkv, 1))).astype(np.float32)
    vs = np.abs(rng.normal(0, 0.02, (R8, cache, Hkv, 1))).astype(np.float32)
    kn = f16(rng.normal(0, 1, (1, Hkv, d)))
    vn = f16(rng.normal(0, 1, (1, Hkv, d)))
    n = 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds / 2:
        r = n % R8
        L.orc_attention_hybrid_int8_fp16(P(q), P(kc[r]), P(vc[r]), P(ks[r]), P(vs[r]), P(kn), P(vn), P(o),
                                         1, 1, cache, 1, Hq, Hkv, d, scale, cache, 1, 128)
        n += 1
    dt = time.perf_counter() - t0
    us = dt / n * 1e6
    out["int8_cache"] = {"us_per_call": round(us, 1), "gbs": round(ATT_BYTES_INT8 / us / 1e3, 3), "cores": 1,
                         "kind": "port",
                         "sample": f"{n} calls over {R8} distinct INT8 caches rotated, {dt:.1f} s, 1 thread"}
    del kc, vc, ks, vs
    # FP16 K/V: 4096 positions
    R16 = 16
    k16 = f16(rng.normal(0, 1, (R16, ctx, Hkv, d)))
    v16 = f16(rng.normal(0, 1, (R16, ctx, Hkv, d)))
    n = 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds / 2:
        r = n % R16
        L.orc_attention_f16(P(q), P(k16[r]), P(v16[r]), P(o), 1, 1, ctx, Hq, Hkv, d, scale, None, ctx - 1, 0, 1)
        n += 1
    dt = time.perf_counter() - t0
    us = dt / n * 1e6
    out["fp16"] = {"us_per_call": round(us, 1), "gbs": round(ATT_BYTES_F16 / us / 1e3, 3), "cores": 1,
                   "kind": "port", "sample": f"{n} calls over {R16} distinct FP16 caches rotated, {dt:.1f} s, 1 thread"}
    out["unit"] = "us/call"
    return out


def cpu_prefill_baseline(tokens: int = 512):
    """The oracle's Qwen3-0.6B-shape model prefilling the first `tokens`
    tokens of the bench prompt on this host's cores (256-token chunks, 16 threads
    at most): a bounded sample of the GPU line's 4096-token prefill, whose
    per-token cost only grows with the context."""
    import oracle
    from cactus_amd.engine import qwen3_0p6b, random_weights
    threads = min(16, os.cpu_count() or 1)
    oracle.lib().orc_set_threads(threads)
    cfg = qwen3_0p6b(max_seq=tokens + 64)
    layers, emb, on = random_weights(cfg, 6)
    orc = oracle.OracleQwen(cfg, layers, emb, on)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 4096).astype(np.uint32)
    t0 = time.perf_counter()
    orc.prefill(prompt[:tokens], cfg["prefill_chunk"])
    dt = time.perf_counter() - t0
    orc.close()
    oracle.lib().orc_set_threads(1)
    return {"value": round(tokens / dt, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"prefill of the first {tokens} prompt tokens by the 28-layer Qwen3-0.6B-shape "
                      f"oracle model, {dt:.1f} s, {threads} threads"}


def host_info():
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": cpu}


def _decode_run(m, cfg, prompt, new_tokens, attention_mode):
    m.reset()
    m.set_attention_mode(attention_mode)
    # one untimed prefill of the prompt first: the timed one then measures
    # steady state, not the first launch of each kernel or the one-time
    # allocation of per-stream scratch
    m.prefill(prompt[:-1])
    m.reset()
    toks, t = m.generate(prompt, new_tokens)
    decode_steps = t.decode_tokens + 1
    decode_s = (t.decode_ms + t.first_decode_ms) / 1e3
    ctx = len(prompt) - 1 + new_tokens / 2
    # bytes per decoded token: every weight once (INT8 attention, INT4 MLP,
    # fp16 scales/norms), the tied FP16 LM head, and the INT8 KV cache at the
    # mean context
    H, F, hd = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    nq, nkv, gs = cfg["heads"] * hd, cfg["kv_heads"] * hd, cfg["group_size"]
    per_layer = (nq * H + 2 * nkv * H + H * nq) * (1 + 2 / gs) + 3 * F * H * (0.5 + 2 / gs) + 4 * H + 4 * hd
    kv = cfg["num_layers"] * 2 * cfg["kv_heads"] * (hd + 4) * ctx
    bytes_tok = cfg["num_layers"] * per_layer + cfg["vocab"] * H * 2 + kv
    return toks, {
        "decode_tok_s": round(decode_steps / decode_s, 2),
        "prefill_tok_s": round(t.prefill_tokens / (t.prefill_ms / 1e3), 1),
        "decode_ms_per_token": round(decode_s * 1e3 / decode_steps, 3),
        "decode_hbm_fraction": round(bytes_tok * decode_steps / decode_s / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_token": int(bytes_tok),
        "distinct_tokens": len(set(int(x) for x in toks)),
    }


def bench_decode(prompt_len: int = 4096, new_tokens: int = 128, mode: int = 1):
    """Qwen3-0.6B-architecture forward, random-init weights (INT4 MLP, INT8
    attention projections, FP16 embeddings/norms): prefill of a 4096-token
    random prompt through the reference's FFI flow, then greedy decode -- in
    the exact attention mode (bit-identical to the reference's arithmetic;
    its tokens are compared with the oracle's frozen run of this same
    workload) and in the tolerance mode (split-K decode attention)."""
    from cactus_amd.engine import Qwen, qwen3_0p6b
    cfg = qwen3_0p6b(max_seq=prompt_len + new_tokens + 64)
    t0 = time.perf_counter()
    m = Qwen(cfg, seed=6)
    if mode:
        m.set_decode_mode(mode)
    init_s = time.perf_counter() - t0
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], prompt_len).astype(np.uint32)
    toks_exact, exact = _decode_run(m, cfg, prompt, new_tokens, 0)
    toks_tol, tol = _decode_run(m, cfg, prompt, new_tokens, 1)
    m.set_attention_mode(0)
    m.close()
    fx = ROOT / "tests" / "golden" / "qwen3_0p6b_generate.npz"
    if fx.exists() and prompt_len == 4096 and new_tokens == 128:
        ref = np.load(fx)["tokens"]
        exact["tokens_equal_oracle"] = bool((toks_exact == ref).all())
        same = toks_tol == ref
        tol["tokens_equal_oracle_prefix"] = int(np.argmin(same)) if not same.all() else len(ref)
    return {**exact, "decode_mode": mode, "attention": "exact", "prompt_tokens": prompt_len,
            "new_tokens": new_tokens, "first_tokens": [int(x) for x in toks_exact[:8]], "init_s": round(init_s, 1),
            "tolerance_attention": tol}


def cpu_decode_baseline(seconds: float = 10.0, prompt_len: int = 32):
    """The oracle's Qwen3-0.6B-shape model on this host's cores: a short
    prefill (not timed), then greedy decode steps timed until `seconds` pass
    (at least one).  The oracle runs its row and head loops on up to 16
    threads; its decode at this short context is dominated by the 151936 x
    1024 FP16 LM head, emulated in exact fp16 arithmetic."""
    import oracle
    from cactus_amd.engine import qwen3_0p6b, random_weights
    threads = min(16, os.cpu_count() or 1)
    oracle.lib().orc_set_threads(threads)
    cfg = qwen3_0p6b(max_seq=prompt_len + 64)
    layers, emb, on = random_weights(cfg, 6)
    orc = oracle.OracleQwen(cfg, layers, emb, on)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], prompt_len).astype(np.uint32)
    orc.prefill(prompt[:-1], cfg["prefill_chunk"])
    tok, n = int(prompt[-1]), 0
    t0 = time.perf_counter()
    while n == 0 or time.perf_counter() - t0 < seconds:
        tok = orc.decode(tok)
        n += 1
    dt = time.perf_counter() - t0
    orc.close()
    oracle.lib().orc_set_threads(1)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} greedy decode steps of the 28-layer Qwen3-0.6B-shape oracle model after a "
                      f"{prompt_len - 1}-token prefill, {dt:.1f} s, {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200)   # ~33 ms of GEMV launches: steady clocks
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--decode-mode", type=int, default=1,
                    help="1: fused decode step replayed as one HIP graph (default); 0: node-by-node graph")
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--decode-only", action="store_true")
    ap.add_argument("--attention-only", action="store_true")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the prefill matmul leg (configs 2 and 3), e.g. under rocprofv3 --pmc with --eager")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the INT8 (config 1) and INT4 (config 3, M=1) streaming GEMV legs, e.g. under rocprofv3 --pmc")
    ap.add_argument("--new-tokens", type=int, default=128)
    ap.add_argument("--eager", action="store_true",
                    help="no HIP graphs: matmuls launched directly and the decode step enqueued per token "
                         "(for kernel tracers; timings then include host launch overhead)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device-to-device copy (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)

    if args.eager:
        os.environ["CACTUS_DECODE_EAGER"] = "1"
    import cactus_amd as cm
    cm.call("cactus_hip_init", 0)
    if args.copy_calibration:
        n = 1 << 30
        src, dst = cm.DeviceBuffer(n), cm.DeviceBuffer(n)
        cm.call("cactus_hip_memcpy_d2d", dst.ptr, src.ptr, n, None)
        cm.call("cactus_hip_stream_sync", None)
        del src, dst
    if args.decode_only:
        print(json.dumps(bench_decode(new_tokens=args.new_tokens, mode=args.decode_mode)), flush=True)
        return
    if args.attention_only:
        print(json.dumps(bench_attention()), flush=True)
        return
    if args.gemm_only:
        print(json.dumps(bench_prefill_gemms(eager=args.eager)), flush=True)
        return
    if args.gemv_only:
        g4 = bench_gemv_int4(INT4_STEPS, INT4_WARMUP)
        g = bench_gemv(args.steps, args.warmup)
        print(json.dumps({"int8_gemv_gbs": round(g["gbs"], 1), "int4_gemv": g4}), flush=True)
        return
    # The streaming GEMVs run last.  When a GPU goes from idle (or from the
    # latency-bound decode) to streaming HBM at full rate, its launches slow
    # down by up to ~25% after the first ~10 and take ~100 launches (~20 ms)
    # to settle back (per-launch series: INT4 188 -> 236 -> 186 us, INT8
    # 157 -> 180 -> 158 us), so a timed region of a few milliseconds right
    # after idle measures the transient.  The INT4 leg (fixed counts: 100
    # warmup + 50 timed launches, ~30 ms) runs first and the INT8 headline
    # follows it with --warmup/--steps as given.  Both weight sets are
    # uploaded before the other legs, so no host copy separates them.
    sets8 = gemv_sets(768)
    sets4 = gemv_int4_sets(604)
    gemms = bench_prefill_gemms(eager=args.eager)
    att = bench_attention()
    dec = None if args.skip_decode else bench_decode(new_tokens=args.new_tokens, mode=args.decode_mode)
    g4 = bench_gemv_int4(INT4_STEPS, INT4_WARMUP, sets=sets4)
    g = bench_gemv(args.steps, args.warmup, sets=sets8)
    del sets8, sets4
    cpu = cpu_baseline(args.cpu_seconds)
    cpu_dec = None if args.skip_decode else cpu_decode_baseline(args.cpu_seconds)
    cpu_gemm = cpu_gemm_baseline(args.cpu_seconds)
    cpu_pf = None if args.skip_decode else cpu_prefill_baseline()
    # each CPU baseline beside the GPU figure it is quoted with
    g4["cpu_baseline"] = cpu_int4_gemv_baseline(args.cpu_seconds / 2)
    gemms["int8_m512_k1024_n3072_g32"]["cpu_baseline"] = cpu_gemm
    gemms["int4_k3072_n1024_g32"]["m256"]["cpu_baseline"] = cpu_int4_m256_baseline(args.cpu_seconds / 2)
    gemms["int4_k3072_n1024_g32"]["m1"]["cpu_baseline"] = g4["cpu_baseline"]
    cpu_att = cpu_attention_baselines(args.cpu_seconds)
    for mode in ("exact", "tolerance"):
        att[f"int8_cache_{mode}"]["cpu_baseline"] = cpu_att["int8_cache"]
        att[f"fp16_{mode}"]["cpu_baseline"] = cpu_att["fp16"]
    out = {
        "metric": "INT8 GEMV GB/s (% HBM peak) + Qwen3-0.6B-shape decode tok/s, 1 MI355X",
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded INT8 codes, |N(0,0.02)|/127 fp16 group scales, N(0,1) fp16 activations)",
        "config": {
            "workload": f"int8 grouped GEMV M=1 K=640 N=2048 group=32, fp16 activations quantized "
                        f"in-kernel; one step = one launch over {g['R']} distinct weight sets",
            "sets_per_launch": g["R"],
            "bytes_per_set": SET_BYTES,
        },
        "hbm_fraction": round(g["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(g["gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
        "cpu_baseline": cpu,
        "host": host_info(),
        "int4_gemv": g4,
        "prefill_gemm": gemms,
        "decode_attention": att,
        "qwen3_0p6b_decode": dec,
        "qwen3_0p6b_decode_cpu_baseline": cpu_dec,
        "qwen3_0p6b_prefill_cpu_baseline": cpu_pf,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
