"""CACT tensor files and model folders (cactus/graph/graph_io.cpp,
python/src/tensor_io.py, Model::init / Config::from_json).

The reference ships no tensor files, so the format is pinned three ways:
headers assembled here field by field at the offsets graph_io.cpp reads
them from (:497-566), two independent writers (the engine's C++
``cactus_cact_save`` and the pure-Python ``cactus_amd.cact.save``) that must
agree byte for byte, and device round trips that must return every byte.
The converter's quantization is pinned by hand-computed codes.

CPU tests use only host entry points of libcactus_engine.so; GPU tests
upload through the engine and compare.  The reference's own tests of this
path are tests/test_graph.cpp:477-520 (save_node + load_into_graph) and
:733-770 (mmap_embeddings); test_graph_load_save_roundtrip and
test_graph_mmap_embeddings mirror them.
"""
import ctypes
import re
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from _data import f16, qwen_small_config, qwen_weights

ROOT = Path(__file__).resolve().parent.parent


def say(*a):
    print("[case]", *a, flush=True)


def _lib():
    from cactus_amd._native import engine
    return engine()


def _err(lib):
    return lib.cactus_engine_last_error().decode()


def _header(precision, dims, data_bytes, scales_bytes=0, gs=0, ng=0, alignment=32, ndim=None, magic=0x54434143,
            version=1, flags=None):
    """80 header bytes, each field at the offset graph_io.cpp:505-551 reads it."""
    h = bytearray(80)
    ndim = len(dims) if ndim is None else ndim
    flags = (1 if scales_bytes else 0) if flags is None else flags
    struct.pack_into("<I", h, 0, magic)
    struct.pack_into("<I", h, 4, version)
    struct.pack_into("<I", h, 8, flags)
    struct.pack_into("<I", h, 12, alignment)
    struct.pack_into("<I", h, 16, ndim)
    for i, d in enumerate(list(dims) + [0] * (4 - len(dims))):
        struct.pack_into("<Q", h, 20 + 8 * i, d)
    struct.pack_into("<I", h, 52, precision)
    struct.pack_into("<Q", h, 56, data_bytes)
    struct.pack_into("<Q", h, 64, scales_bytes)
    struct.pack_into("<I", h, 72, gs)
    struct.pack_into("<I", h, 76, ng)
    return bytes(h)


def _info(path):
    from cactus_amd.cact import read_info
    i = read_info(path)
    return dict(version=i.version, flags=i.flags, alignment=i.alignment, ndim=i.ndim, shape=list(i.shape),
                precision=i.precision, group_size=i.group_size, num_groups=i.num_groups, data_bytes=i.data_bytes,
                scales_bytes=i.scales_bytes, scales_offset=i.scales_offset, data_offset=i.data_offset)


# ------------------------------------------------------------------ CPU
def test_engine_library_exports_every_declared_symbol():
    from cactus_amd._native import parse_header
    lib = _lib()
    decls = parse_header(ROOT / "include" / "cactus_engine.h")
    for name in decls:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "cactus_amd/lib/libcactus_engine.so")],
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r"\b(cactus_(?:qwen|cact|graph|engine)_\w+)\b", out))
    assert exported == set(decls), exported ^ set(decls)


def test_header_fields_at_reference_offsets(tmp_path):
    """INT8 [3][64], g=32: scales at align(80, 32) = 96 (12 bytes), data at
    align(108, 32) = 128; both readers report the same fields."""
    from cactus_amd import cact
    codes = np.arange(3 * 64, dtype=np.int64).astype(np.int8).reshape(3, 64)
    sc = np.arange(6, dtype=np.float16).reshape(3, 2)
    img = _header(0, [3, 64], 192, 12, 32, 2) + bytes(16) + sc.tobytes() + bytes(20) + codes.tobytes()
    assert len(img) == 128 + 192
    p = tmp_path / "w.weights"
    p.write_bytes(img)
    i = _info(p)
    assert i["shape"][:2] == [3, 64] and i["ndim"] == 2 and i["precision"] == 0
    assert (i["scales_offset"], i["scales_bytes"], i["data_offset"], i["data_bytes"]) == (96, 12, 128, 192)
    assert (i["group_size"], i["num_groups"], i["flags"], i["alignment"], i["version"]) == (32, 2, 1, 32, 1)
    info, data, scales = cact.load(p)
    assert info["shape"] == [3, 64] and (data == codes).all() and (scales == sc).all()


@pytest.mark.parametrize("alignment,data_offset", [(0, 80), (1, 80), (64, 128), (4096, 4096)])
def test_header_alignment(tmp_path, alignment, data_offset):
    """alignment 0 reads as 1 (graph_io.cpp:522-523); FP16 data without
    scales starts at align(80, alignment)."""
    from cactus_amd import cact
    x = np.arange(10, dtype=np.float16)
    img = _header(1, [10], 20, alignment=alignment)
    img += bytes(data_offset - 80) + x.tobytes()
    p = tmp_path / "x.weights"
    p.write_bytes(img)
    i = _info(p)
    assert i["alignment"] == max(alignment, 1) and i["data_offset"] == data_offset and i["scales_offset"] == 0
    _, data, scales = cact.load(p)
    assert scales is None and (data == x).all()


def test_header_shape_keeps_nonzero_dims_below_ndim(tmp_path):
    """graph_io.cpp:531-538: dims past ndim are ignored, zero dims dropped."""
    p = tmp_path / "s.weights"
    p.write_bytes(_header(1, [4, 0, 6, 9], 48, ndim=3) + bytes(16) + bytes(48))
    i = _info(p)
    assert i["ndim"] == 3 and i["shape"] == [4, 0, 6, 9]   # raw dims as stored
    from cactus_amd import cact
    info, _, _ = cact.load(p)
    assert info["shape"] == [4, 6]


@pytest.mark.parametrize("case", ["int8", "int4", "fp16", "fp32", "fp16_4d"])
def test_writers_agree_byte_for_byte(tmp_path, case):
    """cactus_cact_save (C++, GraphFile::save_node's layout) and cact.save
    (Python, tensor_io.py's layout) write identical files."""
    from cactus_amd import cact
    lib = _lib()
    rng = np.random.default_rng(11)
    scales, gs = None, 0
    if case == "int8":
        shape, prec, gs = (5, 96), cact.INT8, 32
        data = rng.integers(-127, 128, shape, dtype=np.int8)
        scales = f16(rng.random((5, 3))).view(np.float16)
    elif case == "int4":
        shape, prec, gs = (4, 128), cact.INT4, 64
        data = cact.pack_int4(rng.integers(-7, 8, shape, dtype=np.int8))
        scales = f16(rng.random((4, 2))).view(np.float16)
    elif case == "fp16":
        shape, prec = (7, 3), cact.FP16
        data = rng.random(shape).astype(np.float16)
    elif case == "fp32":
        shape, prec = (13,), cact.FP32
        data = rng.random(shape).astype(np.float32)
    else:
        shape, prec = (2, 3, 4, 5), cact.FP16
        data = rng.random(shape).astype(np.float16)
    a, b = tmp_path / "py.weights", tmp_path / "cpp.weights"
    cact.save(a, data, shape, prec, scales, gs)
    dims = (ctypes.c_uint64 * 4)(*shape)
    raw = np.ascontiguousarray(data)
    sc = None if scales is None else np.ascontiguousarray(scales)
    ng = 0 if sc is None else sc.shape[1]
    rc = lib.cactus_cact_save(str(b).encode(), dims, len(shape), prec, raw.ctypes.data, raw.nbytes,
                              None if sc is None else sc.ctypes.data, gs, ng)
    assert rc == 0, _err(lib)
    assert a.read_bytes() == b.read_bytes()
    info, back, bsc = cact.load(b)
    assert info["precision"] == prec
    assert (np.ascontiguousarray(back).view(np.uint8).reshape(-1) == raw.view(np.uint8).reshape(-1)).all()
    if sc is not None:
        assert (bsc == sc).all()


def test_reader_errors(tmp_path):
    """The reference's messages for a short file, a wrong magic and data past
    the end (graph_io.cpp:497-501, 510-511, 561-563), plus scales past the
    end and unknown precisions."""
    from cactus_amd.cact import CactInfo
    lib = _lib()
    info = CactInfo()

    def expect(img, msg):
        p = tmp_path / "bad.weights"
        p.write_bytes(img)
        assert lib.cactus_cact_read_info(str(p).encode(), ctypes.byref(info)) == -1
        assert msg in _err(lib), _err(lib)

    expect(b"CACT" + bytes(40), "insufficient data for header")
    expect(_header(1, [4], 8, magic=0x54434144) + bytes(24), "missing CACT magic number")
    expect(_header(1, [4], 8) + bytes(16) + bytes(7), "data extends beyond file size")
    expect(_header(0, [2, 64], 128, 1 << 40, 32, 2) + bytes(200), "scales extend beyond file size")
    expect(_header(7, [4], 8) + bytes(24), "unknown precision")
    assert lib.cactus_cact_read_info(str(tmp_path / "missing.weights").encode(), ctypes.byref(info)) == -1
    assert "Cannot open file" in _err(lib)


def test_converter_quantization_known_answers():
    """tensor_io.py:82-112 / :199-221 on hand-computed groups:
    s = max|w|/127 (INT8) or /7 (INT4), code = round(w/s), K padded."""
    from cactus_amd import cact
    w = np.zeros((2, 40), np.float32)
    w[0, :4] = [1.0, -0.75, 0.3, 0.1]          # /(1/127): 127, -95.25, 38.1, 12.7
    w[0, 32:35] = [0.03, -0.04, 0.01]          # second group, s = 0.04/127: 95.25, -127, 31.75
    codes, s = cact.quantize_grouped(w, 32, 8)
    assert codes.shape == (2, 64) and s.shape == (2, 2)
    assert list(codes[0, :4]) == [127, -95, 38, 13] and not codes[0, 4:32].any()
    assert list(codes[0, 32:35]) == [95, -127, 32]
    assert s[0, 0] == np.float16(1.0 / 127) and s[0, 1] == np.float16(np.float32(0.04) / np.float32(127))
    assert not codes[1].any() and (s[1] == np.float16(1e-10)).all()   # all-zero rows: floor 1e-10
    w4 = np.array([[0.7, -0.3, 0.14, 0.0]], np.float32)   # s = 0.1: 7, -3, 1.4, 0
    c4, s4 = cact.quantize_grouped(w4, 4, 4)
    assert list(c4[0]) == [7, -3, 1, 0] and s4[0, 0] == np.float16(0.1)


def test_int4_packing_known_answer():
    """low nibble = even column (tensor_io.py:216-222): codes [1, -2] -> 0xE1."""
    from cactus_amd import cact
    assert cact.pack_int4(np.array([[1, -2, -8, 7]], np.int8)).tolist() == [[0xE1, 0x78]]
    rng = np.random.default_rng(5)
    c = rng.integers(-8, 8, (3, 64), dtype=np.int8)
    assert (cact.unpack_int4(cact.pack_int4(c)) == c).all()


def _qwen_file_stub(folder, gs=64, hidden=256, nq=512):
    from cactus_amd import cact
    q = np.zeros((nq, hidden), np.int8)
    cact.save(Path(folder) / "layer_0_attn_q.weights", q, q.shape, cact.INT8,
              np.zeros((nq, hidden // gs), np.float16), gs)


def test_read_config_defaults_and_keys(tmp_path):
    """Config::from_json: key=value with spaces and comments, unknown keys
    ignored, missing keys keep engine.h:42-58 defaults; group size from the
    q projection file."""
    from cactus_amd.engine import QwenConfig
    lib = _lib()
    (tmp_path / "config.txt").write_text(
        "# converted\nnum_layers = 3\nhidden_dim=256\n\nattention_heads=4\nmodel_type=qwen\n"
        "rope_theta=10000.0\nlayer_norm_eps=1e-05\nsome_other_key=7\nprecision=INT8\n")
    _qwen_file_stub(tmp_path)
    c = QwenConfig()
    assert lib.cactus_qwen_read_config(str(tmp_path).encode(), ctypes.byref(c)) == 0, _err(lib)
    assert (c.num_layers, c.hidden, c.heads, c.group_size) == (3, 256, 4, 64)
    assert (c.ffn, c.kv_heads, c.head_dim, c.vocab, c.prefill_chunk) == (3072, 8, 128, 151936, 256)
    assert c.rope_theta == np.float32(10000.0) and c.eps == np.float32(1e-5)


@pytest.mark.parametrize("line,msg", [("model_type=gemma", "not built"), ("tie_word_embeddings=false", "untied"),
                                      ("num_experts=8", "mixture-of-experts"), ("hidden_dim=abc", "bad value")])
def test_read_config_rejects(tmp_path, line, msg):
    from cactus_amd.engine import QwenConfig
    lib = _lib()
    (tmp_path / "config.txt").write_text(line + "\n")
    _qwen_file_stub(tmp_path)
    assert lib.cactus_qwen_read_config(str(tmp_path).encode(), ctypes.byref(QwenConfig())) == -1
    assert msg in _err(lib), _err(lib)


def _write_small_folder(folder, cfg, seed):
    from cactus_amd.cact import write_qwen_folder
    rng = np.random.default_rng(seed)
    layers, emb, on = qwen_weights(rng, cfg)
    write_qwen_folder(folder, cfg, layers, emb, on)
    return layers, emb, on


def test_folder_checks_every_file_before_upload(tmp_path):
    """Shape, precision and group mismatches are reported with the file name
    before any device work (these run without a GPU)."""
    from cactus_amd import cact
    lib = _lib()
    cfg = qwen_small_config(num_layers=2, vocab=512)
    _write_small_folder(tmp_path, cfg, 3)
    h = ctypes.c_void_p()

    def expect(msg):
        assert lib.cactus_qwen_create_from_folder(str(tmp_path).encode(), 64, ctypes.byref(h)) == -1
        assert msg in _err(lib), _err(lib)

    k = tmp_path / "layer_1_attn_k.weights"
    good = k.read_bytes()
    cact.save(k, np.zeros((128, 256), np.int8), (128, 256), cact.INT8, np.zeros((128, 8), np.float16), 32)
    expect("layer_1_attn_k.weights: shape 128x256, expected 256x256")
    cact.save(k, np.zeros((256, 256), np.int8), (256, 256), cact.INT8, np.zeros((256, 4), np.float16), 64)
    expect("layer_1_attn_k.weights: group size 64")
    k.write_bytes(good)
    e = tmp_path / "token_embeddings.weights"
    cact.save(e, np.zeros((512, 256), np.int8), (512, 256), cact.INT8, np.zeros((512, 2), np.float16), 128)
    expect("token_embeddings.weights: precision INT8, this engine runs FP16")
    e.unlink()
    expect("token_embeddings.weights")
    assert lib.cactus_qwen_create_from_folder(str(tmp_path).encode(), 0, ctypes.byref(h)) == -1


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_cact_load_device_returns_every_byte(hip_ready, tmp_path):
    from cactus_amd import cact
    cm = hip_ready
    lib = _lib()
    rng = np.random.default_rng(21)
    codes = rng.integers(-127, 128, (96, 640), dtype=np.int8)
    sc = np.abs(rng.normal(0, 0.01, (96, 20))).astype(np.float16)
    p = tmp_path / "q.weights"
    cact.save(p, codes, codes.shape, cact.INT8, sc, 32)
    say("cact load_device int8 96x640 g32")
    info = cact.CactInfo()
    d, s = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.cactus_cact_load_device(str(p).encode(), ctypes.byref(info), ctypes.byref(d), ctypes.byref(s)) == 0
    back = np.zeros_like(codes)
    bsc = np.zeros_like(sc)
    cm.call("cactus_hip_memcpy_d2h", back.ctypes.data, d.value, back.nbytes, None)
    cm.call("cactus_hip_memcpy_d2h", bsc.ctypes.data, s.value, bsc.nbytes, None)
    cm.call("cactus_hip_free", d.value)
    cm.call("cactus_hip_free", s.value)
    assert (back == codes).all() and (bsc == sc).all()
    assert (info.data_bytes, info.scales_bytes, info.group_size, info.num_groups) == (96 * 640, 96 * 40, 32, 20)


def _graph_case(folder, kind, rng):
    from cactus_amd import cact
    p = Path(folder) / f"{kind}.weights"
    if kind == "int8":
        d = rng.integers(-127, 128, (64, 256), dtype=np.int8)
        cact.save(p, d, d.shape, cact.INT8, rng.random((64, 8)).astype(np.float16), 32)
    elif kind == "int4":
        d = cact.pack_int4(rng.integers(-8, 8, (32, 256), dtype=np.int8))
        cact.save(p, d, (32, 256), cact.INT4, rng.random((32, 2)).astype(np.float16), 128)
    elif kind == "fp16":
        d = rng.random((2, 3)).astype(np.float16)
        cact.save(p, d, d.shape, cact.FP16)
    else:
        d = rng.random(17).astype(np.float32)
        cact.save(p, d, d.shape, cact.FP32)
    return p


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["int8", "int4", "fp16", "fp32"])
def test_graph_load_save_roundtrip(hip_ready, tmp_path, kind):
    """test_graph.cpp:477-520: load_into_graph / save_node; the re-saved file
    is byte-identical to the loaded one, node data and scales match."""
    from cactus_amd import cact
    lib = _lib()
    rng = np.random.default_rng(len(kind))
    p = _graph_case(tmp_path, kind, rng)
    info, data, scales = cact.load(p)
    say("graph load/save", kind)
    g = ctypes.c_void_p()
    assert lib.cactus_graph_create(ctypes.byref(g)) == 0, _err(lib)
    try:
        node, node2 = ctypes.c_size_t(), ctypes.c_size_t()
        assert lib.cactus_graph_load_weights(g, str(p).encode(), ctypes.byref(node)) == 0, _err(lib)
        assert lib.cactus_graph_load_weights(g, str(p).encode(), ctypes.byref(node2)) == 0
        assert node.value == node2.value   # weight cache by file name (graph_io.cpp:48-52)
        desc = cact.GraphNodeDesc()
        assert lib.cactus_graph_node_info(g, node.value, ctypes.byref(desc)) == 0, _err(lib)
        assert list(desc.shape)[:desc.ndim] == info["shape"] and desc.precision == info["precision"]
        assert desc.data_bytes == info["data_bytes"] and desc.group_size == info["group_size"]
        out = np.zeros(info["data_bytes"], np.uint8)
        osc = np.zeros(max(info["scales_bytes"] // 2, 1), np.uint16)
        assert lib.cactus_graph_read_node(g, node.value, out.ctypes.data, out.nbytes, osc.ctypes.data,
                                          osc.nbytes) == 0, _err(lib)
        assert (out == data.view(np.uint8).reshape(-1)).all()
        if scales is not None:
            assert (osc == scales.view(np.uint16).reshape(-1)).all()
        q = tmp_path / "resaved.weights"
        assert lib.cactus_graph_save_node(g, node.value, str(q).encode()) == 0, _err(lib)
        assert q.read_bytes() == p.read_bytes()
    finally:
        lib.cactus_graph_destroy(g)


@pytest.mark.gpu
def test_graph_mmap_embeddings(hip_ready, tmp_path):
    """test_graph.cpp:733-770: a 2D embedding table loads; 1D is rejected."""
    from cactus_amd import cact
    lib = _lib()
    t = np.arange(12, dtype=np.float16).reshape(4, 3)
    p = tmp_path / "emb.weights"
    cact.save(p, t, t.shape, cact.FP16)
    v = tmp_path / "vec.weights"
    cact.save(v, t.reshape(-1), (12,), cact.FP16)
    say("graph mmap_embeddings")
    g = ctypes.c_void_p()
    assert lib.cactus_graph_create(ctypes.byref(g)) == 0, _err(lib)
    try:
        n = ctypes.c_size_t()
        assert lib.cactus_graph_mmap_embeddings(g, str(p).encode(), ctypes.byref(n)) == 0, _err(lib)
        out = np.zeros(12, np.float16)
        assert lib.cactus_graph_read_node(g, n.value, out.ctypes.data, out.nbytes, None, 0) == 0, _err(lib)
        assert (out == t.reshape(-1)).all()
        assert lib.cactus_graph_mmap_embeddings(g, str(v).encode(), ctypes.byref(n)) == -1
        assert "must be 2D" in _err(lib)
    finally:
        lib.cactus_graph_destroy(g)


@pytest.mark.gpu
@pytest.mark.parametrize("gs", [32, 128])
@pytest.mark.parametrize("mode", [0, 1])
def test_qwen_from_folder_matches_oracle(hip_ready, tmp_path, gs, mode):
    """A model folder written from host weights (group 32, and the
    converter's default group 128) loads through Model::init and generates
    the oracle's tokens; final hidden states and KV cache bit-identical."""
    import oracle
    from cactus_amd.engine import Qwen
    cfg = qwen_small_config(group_size=gs, vocab=1024)
    layers, emb, on = _write_small_folder(tmp_path, cfg, 40 + gs)
    rng = np.random.default_rng(gs)
    prompt = rng.integers(0, cfg["vocab"], 70).astype(np.uint32)
    say("qwen from folder g", gs, "mode", mode)
    m = Qwen.from_folder(tmp_path, context_size=cfg["max_seq"])
    try:
        assert m.cfg["group_size"] == gs and m.cfg["num_layers"] == cfg["num_layers"]
        if mode:
            m.set_decode_mode(mode)
        toks, _ = m.generate(prompt, 6)
        orc = oracle.OracleQwen(cfg, layers, emb, on)
        ref = orc.generate(prompt, 6, cfg["prefill_chunk"])
        assert list(toks) == list(ref)
        if mode == 0:
            assert (m.last_hidden() == orc.last_hidden()).all()
        for layer in range(cfg["num_layers"]):
            for a, b in zip(m.read_kv(layer), orc.read_kv(layer)):
                assert (a == b).all(), f"kv cache layer {layer}"
        got_layers, got_emb, got_on = m.read_weights()
        assert (got_emb == emb).all() and (got_on == on).all()
        for a, b in zip(got_layers, layers):
            for k in b:
                assert (np.asarray(a[k]).view(np.uint8) == np.asarray(b[k]).view(np.uint8)).all(), k
    finally:
        m.close()
