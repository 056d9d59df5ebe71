"""C-ABI checks that need no GPU: the libraries load, export every symbol the
headers in include/ declare, and reject bad shapes before launching."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared(header):
    from cactus_amd._native import parse_header
    return parse_header(ROOT / "include" / header)


def test_hip_library_exports_every_declared_symbol():
    import cactus_amd
    lib = cactus_amd.hip()
    decls = _declared("cactus_hip.h")
    assert len(decls) >= 35
    for name in decls:
        assert hasattr(lib, name), name
    # nothing exported under the ABI prefix that the header does not declare
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "cactus_amd/lib/libcactus_hip.so")],
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r"\b(cactus_hip_\w+)\b", out))
    assert exported == set(decls), exported ^ set(decls)


def test_rejects_bad_shapes_without_launching():
    import cactus_amd
    lib = cactus_amd.hip()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # group size must be a power of two dividing K
    assert lib.cactus_hip_matmul_int8(p, p, p, p, p, 1, 96, 8, 48, None) == -1
    assert lib.cactus_hip_matmul_int8(p, p, p, p, p, 1, 100, 8, 32, None) == -1
    assert lib.cactus_hip_matmul_int4(p, p, p, p, p, 1, 64, 8, 16, None) == -1
    assert b"group_size" in lib.cactus_hip_last_error()
    # zero-sized problems are a silent no-op, as in kernel_gemm.cpp:137
    assert lib.cactus_hip_matmul_int8(None, None, None, None, None, 0, 64, 8, 32, None) == 0
    # GQA head counts
    assert lib.cactus_hip_attention_f16(p, p, p, p, 1, 1, 4, 3, 2, 128, ctypes.c_float(0), None, 0, 0,
                                        1, None) == -1
    # a negative temperature is refused before anything is launched
    assert lib.cactus_hip_sample_f16(p, p, 10, ctypes.c_float(-0.7), ctypes.c_float(0.9), 0, 0,
                                     None) == -1
    assert b"temperature" in lib.cactus_hip_last_error()
    # the merged matmul takes one to three weight sets
    arr = (ctypes.c_void_p * 4)(16, 16, 16, 16)
    ns = (ctypes.c_size_t * 4)(64, 64, 64, 64)
    for cnt in (0, 4):
        assert lib.cactus_hip_matmul_grouped_multi(p, p, cnt, arr, arr, arr, ns, 32, 64, 32, 0, None) == -1
        assert b"count" in lib.cactus_hip_last_error()
    ns[1] = 8
    assert lib.cactus_hip_matmul_grouped_multi(p, p, 2, arr, arr, arr, ns, 32, 96, 48, 0, None) == -1
    assert b"group_size" in lib.cactus_hip_last_error()
