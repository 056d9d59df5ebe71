"""ctypes loader for the native libraries.

The argument types of every entry point are read from the C headers in
include/, so the Python side cannot drift from the ABI.  Loading fails loudly
when a library has not been built: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
LIBDIR = PKG / "lib"

_DECL = re.compile(r"^\s*([A-Za-z_][\w\s\*]*?)\b(cactus_\w+)\s*\(([^)]*)\)\s*;", re.M)


def _ctype(tok: str):
    t = "".join(tok.replace("const", " ").split())
    if t == "char*":
        return ctypes.c_char_p
    if t.endswith("**"):
        return ctypes.POINTER(ctypes.c_void_p)
    if t.endswith("*"):
        return ctypes.c_void_p
    return {
        "int": ctypes.c_int,
        "float": ctypes.c_float,
        "double": ctypes.c_double,
        "size_t": ctypes.c_size_t,
        "uint32_t": ctypes.c_uint32,
        "int32_t": ctypes.c_int32,
        "uint64_t": ctypes.c_uint64,
        "void": None,
    }[t]


def parse_header(path: Path) -> dict[str, tuple]:
    """Map entry-point name -> (restype, [argtypes]) for every declaration."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)
    text = text.replace('extern "C" {', "").replace("}", "")
    text = re.sub(r"\s+", " ", text).replace(";", ";\n")
    out = {}
    for m in _DECL.finditer(text):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        argtypes = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name
                mm = re.match(r"(.*?)([A-Za-z_]\w*)$", a)
                typ = mm.group(1).strip() if mm else a
                argtypes.append(_ctype(typ))
        out[name] = (_ctype(ret), argtypes)
    return out


class NativeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def _load(libname: str, header: str, preload: list[ctypes.CDLL] | None = None):
    path = LIBDIR / libname
    if not path.exists():
        raise ImportError(
            f"{path} is not built; run `python -m cactus_amd.build` (or "
            f"__graft_entry__.build()). There is no CPU fallback.")
    lib = ctypes.CDLL(str(path), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    decls = parse_header(INCLUDE / header)
    for name, (res, args) in decls.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib._decls = decls
    return lib


_hip = None
_engine = None


def hip():
    """The kernel library (include/cactus_hip.h)."""
    global _hip
    if _hip is None:
        _hip = _load("libcactus_hip.so", "cactus_hip.h")
    return _hip


def engine():
    """The graph/engine library (include/cactus_engine.h)."""
    global _engine
    if _engine is None:
        hip()
        _engine = _load("libcactus_engine.so", "cactus_engine.h")
    return _engine


def check(rc: int, lib=None) -> None:
    if rc != 0:
        lib = lib or hip()
        msg = lib.cactus_hip_last_error() if hasattr(lib, "cactus_hip_last_error") else b""
        raise NativeError(rc, (msg or b"").decode(errors="replace"))
