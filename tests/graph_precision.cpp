// Host-only probe of the node graph's precision inference: builds nodes on a
// CactusGraph (no execution, no device call) and prints, per node, its
// precision and byte size.  Compiled and run by test_graph_precision.py.
#include <cstdio>
#include <stdexcept>

#include "graph.h"

using cactus::CactusGraph;
using cactus::Precision;

static const char* pname(Precision p) {
    switch (p) {
        case Precision::INT8: return "INT8";
        case Precision::FP16: return "FP16";
        case Precision::FP32: return "FP32";
        case Precision::INT4: return "INT4";
    }
    return "?";
}

int main() {
    // never destroyed: the destructor synchronises the (absent) device stream
    CactusGraph* g = new CactusGraph(nullptr);
    auto show = [&](const char* name, size_t id) {
        const auto& b = g->get_output_buffer(id);
        std::printf("%s %s %zu\n", name, pname(b.precision), (size_t)b.byte_size);
    };
    const size_t x = g->input({4, 64}, Precision::FP16);
    const size_t w = g->input({32, 64}, Precision::INT8);
    const size_t nw = g->input({64}, Precision::FP16);
    show("input_fp16", x);
    const size_t q = g->quantize_activations(x);
    show("quantize_activations", q);
    show("reshape_of_quantized", g->reshape(q, {256}));
    show("matmul", g->matmul(x, w, true));
    show("rms_norm", g->rms_norm(x, nw, 1e-6f));
    show("add", g->add(x, x));
    show("index_of_fp16", g->index(x, 1, 0));
    try {
        g->quantize_activations(w);
        std::printf("quantize_int8_input accepted\n");
    } catch (const std::invalid_argument& e) {
        std::printf("quantize_int8_input rejected %s\n", e.what());
    }
    return 0;
}
