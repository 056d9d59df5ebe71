"""Build recipe for the native libraries of cactus_amd.

    python -m cactus_amd.build          # or cactus_amd.build.build_all()

Produces, in-tree:
    cactus_amd/lib/libcactus_hip.so     HIP kernels + C ABI (include/cactus_hip.h)
    cactus_amd/lib/libcactus_engine.so  C++ graph/engine layer over that ABI
                                        (include/cactus_engine.h)

Every HIP source is compiled for gfx950 only, with contraction off (fused
multiply-adds appear only where the sources write them) and the packed-FP32
target feature disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
ENGINE_SRC = CSRC / "engine"
LIBDIR = PKG / "lib"
OBJDIR = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-ffp-contract=off"]
# per-source additions: MFMA accumulators in ordinary VGPRs, so the VALU
# work on them (the matmul's fp32 group epilogue, the attention's per-tile
# rescale) needs no v_accvgpr_read / v_accvgpr_write copies
HIP_FILE_FLAGS = {
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the prefill attention scales its output accumulators every key tile
    "attention_fast.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # the decode value chains: the next block's scalar weight loads must stay
    # ahead of this block's FMAs (machine sinking moves them behind)
    "chain_stream.hip": ["-mllvm", "-disable-machine-sink"],
}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        sys.stderr.write(proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    # keep the host-pass notice about the packed-fp32 feature out of the log
    for line in proc.stderr.splitlines():
        if "packed-fp32-ops" in line and "not a recognized feature" in line:
            continue
        if line.strip():
            sys.stderr.write(line + "\n")


def _compile_hip(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    _run([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(src.name, []), "-I", str(ROOT / "include"), "-c", str(src),
          "-o", str(obj)])
    return obj


def build_hip(jobs: int | None = None) -> Path:
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    out = LIBDIR / "libcactus_hip.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_engine() -> Path | None:
    srcs = sorted(ENGINE_SRC.glob("*.cpp")) if ENGINE_SRC.exists() else []
    if not srcs:
        return None
    out = LIBDIR / "libcactus_engine.so"
    tmp = out.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    _run([cxx, *CXX_FLAGS, "-shared", "-I", str(ROOT / "include"), *map(str, srcs),
          "-L", str(LIBDIR), "-lcactus_hip", "-Wl,-rpath,$ORIGIN", "-pthread", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_oracle() -> Path:
    """Compile the CPU restatement used by the tests (oracle/Makefile)."""
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "_build" / "libcactus_oracle.so"


def build_all() -> None:
    build_hip()
    build_engine()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built:", *sorted(p.name for p in LIBDIR.glob("*.so")))
