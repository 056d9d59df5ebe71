"""CACT tensor files and Qwen model folders (the reference's weight format).

Format (cactus/graph/graph_io.cpp:145-222 writer, :497-566 reader;
python/src/tensor_io.py:163-321 converter): an 80-byte little-endian header

    magic "CACT" | version u32 | flags u32 | alignment u32 | ndim u32 |
    dims[4] u64 | precision u32 | data bytes u64 | scales bytes u64 |
    group size u32 | group count u32

then fp16 group scales ``[rows][groups]`` at ``align(80, alignment)`` and the
data at ``align(end of scales, alignment)``.  Precision codes: 0 INT8, 1 FP16,
2 FP32, 3 INT4 (two codes per byte, low nibble = even column).

This module writes and reads files on the host in pure Python (so it checks
the C++ reader and writer of libcactus_engine.so independently), quantizes
weights the way the reference converter does, and writes a Qwen3 model
folder that ``Qwen.from_folder`` / ``cactus_qwen_create_from_folder`` load.
"""
from __future__ import annotations

import ctypes
import struct
from pathlib import Path

import numpy as np

MAGIC = 0x54434143
VERSION = 1
ALIGNMENT = 32
FLAG_HAS_SCALES = 1 << 0
HEADER = 80
INT8, FP16, FP32, INT4 = 0, 1, 2, 3
_ELEM = {INT8: 1, FP16: 2, FP32: 4}


class CactInfo(ctypes.Structure):
    """cactus_cact_info of include/cactus_engine.h."""
    _fields_ = [("version", ctypes.c_uint32), ("flags", ctypes.c_uint32), ("alignment", ctypes.c_uint32),
                ("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 4), ("precision", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("num_groups", ctypes.c_uint32),
                ("data_bytes", ctypes.c_uint64), ("scales_bytes", ctypes.c_uint64),
                ("scales_offset", ctypes.c_uint64), ("data_offset", ctypes.c_uint64)]


class GraphNodeDesc(ctypes.Structure):
    """cactus_graph_node_desc of include/cactus_engine.h."""
    _fields_ = [("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 4), ("precision", ctypes.c_uint32),
                ("data_bytes", ctypes.c_uint64), ("group_size", ctypes.c_uint32), ("num_groups", ctypes.c_uint32)]


def _align(off: int, a: int) -> int:
    return -(-off // a) * a


def save(path, data: np.ndarray, shape, precision: int, scales: np.ndarray | None = None,
         group_size: int = 0, alignment: int = ALIGNMENT) -> None:
    """Write one tensor.  ``data`` holds the stored bytes (INT4 already packed);
    ``scales`` fp16 ``[rows][groups]`` or None."""
    shape = [int(d) for d in shape]
    if len(shape) > 4:
        raise ValueError("CACT files hold at most 4 dimensions")
    raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    sc = None if scales is None else np.ascontiguousarray(scales, dtype=np.float16).view(np.uint8).reshape(-1)
    ngroups = 0 if sc is None else (shape[1] if len(shape) > 1 else shape[0]) // group_size
    head = struct.pack("<IIIII", MAGIC, VERSION, FLAG_HAS_SCALES if sc is not None else 0, alignment, len(shape))
    head += struct.pack("<4Q", *(shape + [0] * (4 - len(shape))))
    head += struct.pack("<IQQII", precision, raw.size, 0 if sc is None else sc.size,
                        group_size if sc is not None else 0, ngroups)
    assert len(head) == HEADER
    a = max(alignment, 1)
    with open(path, "wb") as f:
        f.write(head)
        off = _align(HEADER, a)
        f.write(b"\0" * (off - HEADER))
        if sc is not None:
            f.write(sc.tobytes())
            end = off + sc.size
            f.write(b"\0" * (_align(end, a) - end))
        f.write(raw.tobytes())


def load(path) -> tuple[dict, np.ndarray, np.ndarray | None]:
    """Read one tensor on the host: (header fields, data, scales or None).
    INT8 -> int8, FP16 -> float16, FP32 -> float32 in the file's shape; INT4
    -> the packed uint8 bytes ``[rows][cols/2]``."""
    buf = Path(path).read_bytes()
    if len(buf) < HEADER:
        raise ValueError("File too small: insufficient data for header")
    magic, version, flags, alignment, ndim = struct.unpack_from("<IIIII", buf, 0)
    if magic != MAGIC:
        raise ValueError("Invalid tensor file: missing CACT magic number")
    dims = struct.unpack_from("<4Q", buf, 20)
    precision, nbytes, sbytes, gs, ng = struct.unpack_from("<IQQII", buf, 52)
    a = alignment or 1
    shape = [int(d) for i, d in enumerate(dims) if i < ndim and d > 0]
    off = _align(HEADER, a)
    scales = None
    if sbytes:
        scales = np.frombuffer(buf, np.float16, sbytes // 2, off).reshape(shape[0] if shape else 1, -1)
        off = _align(off + sbytes, a)
    if off + nbytes > len(buf):
        raise ValueError("File corrupted: data extends beyond file size")
    raw = np.frombuffer(buf, np.uint8, nbytes, off)
    if precision == INT4:
        data = raw.reshape(shape[0], -1) if len(shape) == 2 else raw.copy()
    else:
        data = raw.view({INT8: np.int8, FP16: np.float16, FP32: np.float32}[precision]).reshape(shape)
    info = dict(version=version, flags=flags, alignment=alignment, ndim=ndim, shape=shape, precision=precision,
                data_bytes=nbytes, scales_bytes=sbytes, group_size=gs, num_groups=ng)
    return info, data.copy(), None if scales is None else scales.copy()


def read_info(path) -> CactInfo:
    """The engine library's header parser (MappedFile::parse_header)."""
    from ._native import NativeError, engine
    lib = engine()
    info = CactInfo()
    if lib.cactus_cact_read_info(str(path).encode(), ctypes.byref(info)) != 0:
        raise NativeError(-1, lib.cactus_engine_last_error().decode(errors="replace"))
    return info


# ---------------------------------------------------------------- quantization
def quantize_grouped(w: np.ndarray, group_size: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """The converter's group quantization (tensor_io.py:82-112 INT8, :199-221
    INT4): per row and group, ``s = max(|w|)/qmax`` in float32 (floor 1e-10),
    ``code = clip(round_half_even(w/s))`` to [-128, 127] or [-8, 7]; scales
    are stored as fp16.  K is padded with zeros to a whole group.  Returns
    (codes int8 ``[N][K]``, scales fp16 ``[N][K/g]``)."""
    w = np.asarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("grouped quantization takes a 2D weight")
    N, K = w.shape
    if K % group_size:
        w = np.pad(w, ((0, 0), (0, group_size - K % group_size)))
        K = w.shape[1]
    qmax, lo, hi = (127.0, -128, 127) if bits == 8 else (7.0, -8, 7)
    g = w.reshape(N, K // group_size, group_size)
    s = np.maximum((np.abs(g).max(axis=2) / np.float32(qmax)).astype(np.float32), np.float32(1e-10))
    codes = np.clip(np.round(g / s[:, :, None]), lo, hi).astype(np.int8).reshape(N, K)
    return codes, s.astype(np.float16)


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte, low nibble = even column (tensor_io.py:216-222)."""
    c = np.asarray(codes, dtype=np.int8)
    if c.shape[-1] % 2:
        raise ValueError("INT4 packing needs an even number of columns")
    lo = c[..., 0::2].astype(np.uint8) & 0x0F
    hi = c[..., 1::2].astype(np.uint8) & 0x0F
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    lo = (p & 0x0F).astype(np.int16)
    hi = (p >> 4).astype(np.int16)
    lo = np.where(lo > 7, lo - 16, lo)
    hi = np.where(hi > 7, hi - 16, hi)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def save_tensor_with_header(tensor, path, precision: str = "FP16", group_size: int = 128) -> None:
    """The converter's tensor writer (tensor_io.py:40-321) without its
    statistics: 2D INT8 / INT4 tensors are group-quantized (norm and bias
    files stay FP16, :71-74); everything else is written as FP16."""
    data = np.asarray(tensor, dtype=np.float32)
    name = Path(path).name
    if precision in ("INT8", "INT4") and any(x in name for x in ("norm", "bias", "vision")):
        precision = "FP16"
    if precision in ("INT8", "INT4") and data.ndim == 2:
        codes, scales = quantize_grouped(data, group_size, 8 if precision == "INT8" else 4)
        if precision == "INT8":
            save(path, codes, codes.shape, INT8, scales, group_size)
        else:
            save(path, pack_int4(codes), codes.shape, INT4, scales, group_size)
        return
    h = data.astype(np.float16)
    save(path, h, h.shape, FP16)


# ---------------------------------------------------------------- model folders
def write_config(folder, cfg: dict, tie_word_embeddings: bool = True, extra: dict | None = None) -> None:
    """config.txt in the reference's key=value form (engine_model.cpp:403-520)."""
    keys = dict(vocab_size=cfg["vocab"], num_layers=cfg["num_layers"], hidden_dim=cfg["hidden"],
                ffn_intermediate_dim=cfg["ffn"], attention_heads=cfg["heads"],
                attention_kv_heads=cfg["kv_heads"], attention_head_dim=cfg["head_dim"],
                layer_norm_eps=repr(float(cfg["eps"])), rope_theta=repr(float(cfg["rope_theta"])),
                tie_word_embeddings="true" if tie_word_embeddings else "false", model_type="qwen")
    keys.update(extra or {})
    Path(folder).mkdir(parents=True, exist_ok=True)
    with open(Path(folder) / "config.txt", "w") as f:
        for k, v in keys.items():
            f.write(f"{k}={v}\n")


def write_qwen_folder(folder, cfg: dict, layers: list[dict], embedding: np.ndarray,
                      output_norm: np.ndarray) -> None:
    """A Qwen3 model folder from already-quantized host weights in the
    engine's layout (``Qwen.read_weights``): grouped INT8 attention
    projections, packed INT4 MLP, fp16 (uint16 bits) norms and embeddings;
    file names of model_qwen.cpp:17-42."""
    folder = Path(folder)
    write_config(folder, cfg)
    gs = cfg["group_size"]
    f16 = lambda a: np.asarray(a, np.uint16).view(np.float16)  # noqa: E731
    save(folder / "token_embeddings.weights", f16(embedding), np.shape(embedding), FP16)
    save(folder / "output_norm.weights", f16(output_norm), np.shape(output_norm), FP16)
    for i, L in enumerate(layers):
        p = lambda n: folder / f"layer_{i}_{n}.weights"  # noqa: E731
        for key, name in (("input_norm", "input_norm"), ("post_norm", "post_attn_norm"),
                          ("q_norm", "attn_q_norm"), ("k_norm", "attn_k_norm")):
            save(p(name), f16(L[key]), np.shape(L[key]), FP16)
        for key, name in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output")):
            w = L[key + "_w"]
            save(p(name), w, w.shape, INT8, f16(L[key + "_s"]), gs)
        for key, name in (("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
            w = L[key + "_w"]
            save(p(name), w, (w.shape[0], w.shape[1] * 2), INT4, f16(L[key + "_s"]), gs)
