"""Seeded synthetic inputs shared by the parity tests, the smoke test and the
bench (shapes and distributions of the workloads the kernels are quoted on)."""
from __future__ import annotations

import numpy as np


def f16(x) -> np.ndarray:
    """float array -> fp16 bit patterns (uint16)."""
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).astype(np.float16)).view(np.uint16)


def grouped_int8_weights(rng, N, K, gs):
    """INT8 codes U{-127..127}, fp16 group scales |N(0,0.02)|/127."""
    B = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    Bs = f16(np.abs(rng.normal(0, 0.02, size=(N, K // gs))) / 127.0)
    return B, Bs


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """[N][K] int codes in [-8,7] -> [N][K/2] bytes, low nibble = even k
    (the packing of tests/test_kernel.cpp:323-330 and tensor_io.py:225-229)."""
    lo = codes[:, 0::2].astype(np.uint8) & 0x0F
    hi = codes[:, 1::2].astype(np.uint8) & 0x0F
    return np.ascontiguousarray(lo | (hi << 4))


def grouped_int4_weights(rng, N, K, gs):
    """INT4 codes U{-7..7}, fp16 group scales |N(0,0.02)|/7."""
    codes = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    Bs = f16(np.abs(rng.normal(0, 0.02, size=(N, K // gs))) / 7.0)
    return codes, pack_int4(codes), Bs


def activations(rng, M, K):
    return f16(rng.normal(0, 1, size=(M, K)))
