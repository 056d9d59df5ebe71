"""Precision inference of the node graph (CactusGraph::add_node and the
builders, engine/graph.cpp), on the host: a small C++ probe builds nodes on a
graph that never executes and prints each node's precision and byte size.

The reference types a node by its builder's requested precision, except that
a request for INT8 takes the first input's precision instead
(graph_builder.cpp:582-587).  For an FP16 graph the two agree on every node
but QUANTIZE_ACTIVATIONS: the reference asks for INT8 (graph_builder.cpp:
567-569), so the rule types the node FP16 with an FP16-sized buffer that holds
INT8 codes; here it is typed INT8 (one byte per code).  The test pins both
halves: the INT8 node, and the reference's typing of everything around it.
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "cactus_amd" / "lib"


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    if not (LIB / "libcactus_engine.so").exists():
        pytest.skip("engine library not built (run __graft_entry__.build())")
    exe = tmp_path_factory.mktemp("prec") / "graph_precision"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(ROOT / "cactus_amd" / "csrc" / "engine"),
                    "-I", str(ROOT / "include"), str(ROOT / "tests" / "graph_precision.cpp"),
                    "-L", str(LIB), "-lcactus_engine", "-lcactus_hip", f"-Wl,-rpath,{LIB}", "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120).stdout
    rows = {}
    for line in out.splitlines():
        name, rest = line.split(" ", 1)
        rows[name] = rest.split()
    return rows


def test_quantize_activations_is_int8_typed(probe):
    # 4 x 64 codes, one byte each (the reference's rule would give FP16, 512 bytes)
    assert probe["quantize_activations"] == ["INT8", "256"]
    assert probe["reshape_of_quantized"] == ["INT8", "256"]


def test_fp16_graph_nodes_follow_reference_typing(probe):
    assert probe["input_fp16"] == ["FP16", "512"]
    assert probe["matmul"] == ["FP16", str(4 * 32 * 2)]
    assert probe["rms_norm"] == ["FP16", "512"]
    assert probe["add"] == ["FP16", "512"]
    assert probe["index_of_fp16"] == ["FP16", "128"]


def test_quantize_activations_rejects_non_fp16_input(probe):
    # graph_builder.cpp:563-565 throws std::invalid_argument with this text
    assert probe["quantize_int8_input"][0] == "rejected"
    assert " ".join(probe["quantize_int8_input"][1:]) == "quantize_activations requires FP16 input"
