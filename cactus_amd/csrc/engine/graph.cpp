// graph.cpp -- builder and serial executor of the device-resident CactusGraph.
//
// Shape/precision inference follows graph_builder.cpp; node execution follows
// the per-op executors of graph_ops_nn.cpp, graph_ops_math.cpp,
// graph_ops_tensor.cpp and graph_ops_sample.cpp, with every compute step a
// call into the kernel C ABI.  RESHAPE and INDEX(dim 0) are views here (the
// reference copies for RESHAPE, graph_ops_math.cpp:265-281); values are
// identical.
#include "graph.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <numeric>

#include "cact_file.h"
#include "cactus_hip.h"
#include "loader.h"

namespace cactus {

void check_hip(int rc, const char* what) {
    if (rc != CACTUS_HIP_OK)
        throw std::runtime_error(std::string(what) + ": " + cactus_hip_last_error());
}

size_t precision_size(Precision p) {
    switch (p) {
        case Precision::INT8: return 1;
        case Precision::FP16: return 2;
        case Precision::FP32: return 4;
        case Precision::INT4: return 1;
    }
    return 1;
}

static size_t numel(const std::vector<size_t>& s) {
    return std::accumulate(s.begin(), s.end(), (size_t)1, std::multiplies<size_t>());
}

// ------------------------------------------------------------------ BufferPool
size_t BufferPool::round_up(size_t b) {
    if (b <= 256) return 256;
    size_t p = 256;
    while (p < b) p <<= 1;
    return p;
}

void* BufferPool::acquire(size_t bytes) {
    const size_t b = round_up(bytes);
    auto& fl = free_[b];
    if (!fl.empty()) {
        void* p = fl.back();
        fl.pop_back();
        return p;
    }
    void* p = nullptr;
    check_hip(cactus_hip_malloc(&p, b), "BufferPool::acquire");
    pool_bytes_ += b;
    return p;
}

void BufferPool::release(void* ptr, size_t bytes) {
    if (ptr) free_[round_up(bytes)].push_back(ptr);
}

void BufferPool::clear() {
    for (auto& kv : free_)
        for (void* p : kv.second) cactus_hip_free(p);
    free_.clear();
    pool_bytes_ = 0;
}

BufferPool::~BufferPool() { clear(); }

// ------------------------------------------------------------------ CactusGraph
CactusGraph::CactusGraph(void* stream) : stream_(stream) {}

CactusGraph::~CactusGraph() {
    cactus_hip_stream_sync(stream_);
    hard_reset();
    if (quant_codes_) cactus_hip_free(quant_codes_);
    if (quant_scales_) cactus_hip_free(quant_scales_);
    if (embed_err_) cactus_hip_free(embed_err_);
}

GraphNode& CactusGraph::node(size_t id) {
    auto it = index_.find(id);
    if (it == index_.end()) throw std::runtime_error("unknown node " + std::to_string(id));
    return *nodes_[it->second];
}
const GraphNode& CactusGraph::node(size_t id) const {
    auto it = index_.find(id);
    if (it == index_.end()) throw std::runtime_error("unknown node " + std::to_string(id));
    return *nodes_[it->second];
}

size_t CactusGraph::add_node(OpType op, const std::vector<size_t>& inputs,
                             const std::vector<size_t>& shape, Precision precision,
                             const OpParams& params) {
    auto n = std::make_unique<GraphNode>();
    n->id = next_id_++;
    n->op = op;
    n->inputs = inputs;
    n->params = params;
    n->out.shape = shape;
    n->out.precision = precision;
    n->out.total_size = numel(shape);
    n->out.byte_size = n->out.total_size * precision_size(precision);
    index_[n->id] = nodes_.size();
    nodes_.push_back(std::move(n));
    return nodes_.back()->id;
}

const BufferDesc& CactusGraph::get_output_buffer(size_t id) const { return node(id).out; }

size_t CactusGraph::input(const std::vector<size_t>& shape, Precision precision) {
    return add_node(OpType::INPUT, {}, shape, precision);
}

size_t CactusGraph::matmul(size_t a, size_t b, bool pretransposed_rhs) {
    const auto& as = node(a).out.shape;
    const auto& bs = node(b).out.shape;
    if (as.size() < 2 || bs.size() != 2) throw std::runtime_error("matmul expects [.., M, K] x 2D");
    const size_t K = as.back();
    const size_t N = pretransposed_rhs ? bs[0] : bs[1];
    const size_t Kb = pretransposed_rhs ? bs[1] : bs[0];
    if (K != Kb) throw std::runtime_error("matmul: inner dimensions differ");
    std::vector<size_t> out(as.begin(), as.end() - 1);
    out.push_back(N);
    OpParams p;
    p.pretransposed_rhs = pretransposed_rhs;
    return add_node(OpType::MATMUL, {a, b}, out, Precision::FP16, p);
}

// The node is typed INT8 (one byte per code, plus per-row scales).  The
// reference's add_node re-types any node asked for INT8 to its first input's
// precision (graph_builder.cpp:582-587), so there this node reports FP16 and
// its codes sit in an FP16-sized buffer; consumers here read the INT8 type.
size_t CactusGraph::quantize_activations(size_t input) {
    if (node(input).out.precision != Precision::FP16)
        throw std::invalid_argument("quantize_activations requires FP16 input");   // graph_builder.cpp:563-565
    return add_node(OpType::QUANTIZE_ACTIVATIONS, {input}, node(input).out.shape, Precision::INT8);
}

size_t CactusGraph::rms_norm(size_t input, size_t weight, float epsilon) {
    OpParams p;
    p.epsilon = epsilon;
    return add_node(OpType::RMS_NORM, {input, weight}, node(input).out.shape, Precision::FP16, p);
}

size_t CactusGraph::rms_norm_quantize(size_t input, size_t weight, float epsilon) {
    OpParams p;
    p.epsilon = epsilon;
    return add_node(OpType::RMS_NORM_QUANTIZE, {input, weight}, node(input).out.shape, Precision::INT8, p);
}

size_t CactusGraph::silu_mul_quantize(size_t gate, size_t up) {
    if (node(gate).out.total_size != node(up).out.total_size)
        throw std::runtime_error("multiply: broadcasting is not built (shapes must match)");
    return add_node(OpType::SILU_MUL_QUANTIZE, {gate, up}, node(gate).out.shape, Precision::INT8);
}

size_t CactusGraph::matmul_add(size_t a, size_t b, size_t residual) {
    const size_t mm = matmul(a, b, true);
    GraphNode& m = node(mm);
    if (node(residual).out.shape != m.out.shape) throw std::runtime_error("matmul_add: residual shape mismatch");
    m.op = OpType::MATMUL_ADD;
    m.inputs.push_back(residual);
    return mm;
}

size_t CactusGraph::rms_norm_rope(size_t input, size_t weight, float epsilon, float theta, size_t position_offset) {
    if (node(input).out.shape.size() < 4) throw std::runtime_error("RoPE operation requires 4D tensor");
    OpParams p;
    p.epsilon = epsilon;
    p.theta = theta;
    p.position_offset = position_offset;
    return add_node(OpType::RMS_NORM_ROPE, {input, weight}, node(input).out.shape, Precision::FP16, p);
}

size_t CactusGraph::rope(size_t input, float theta, size_t position_offset) {
    OpParams p;
    p.theta = theta;
    p.position_offset = position_offset;
    return add_node(OpType::ROPE, {input}, node(input).out.shape, Precision::FP16, p);
}

size_t CactusGraph::softmax(size_t input, int axis) {
    OpParams p;
    p.axis = axis;
    return add_node(OpType::SOFTMAX, {input}, node(input).out.shape, Precision::FP16, p);
}

size_t CactusGraph::attention(size_t q, size_t k, size_t v, float scale, size_t position_offset,
                              size_t window_size, bool is_causal) {
    OpParams p;
    p.scale = scale;
    p.position_offset = position_offset;
    p.window_size = window_size;
    p.is_causal = is_causal;
    p.tolerance = attention_tolerance_;
    return add_node(OpType::ATTENTION, {q, k, v}, node(q).out.shape, Precision::FP16, p);
}

size_t CactusGraph::attention_int8_hybrid(size_t q, size_t k_new, size_t v_new, float scale,
                                          size_t position_offset, const int8_t* ck,
                                          const int8_t* cv, const float* ks, const float* vs,
                                          size_t cache_len, size_t num_kv_heads, size_t head_dim) {
    OpParams p;
    p.scale = scale;
    p.position_offset = position_offset;
    p.cached_keys_int8 = ck;
    p.cached_values_int8 = cv;
    p.cached_k_scales = ks;
    p.cached_v_scales = vs;
    p.cache_seq_len = cache_len;
    p.num_kv_heads = num_kv_heads;
    p.head_dim = head_dim;
    p.tolerance = attention_tolerance_;
    return add_node(OpType::ATTENTION_INT8_HYBRID, {q, k_new, v_new}, node(q).out.shape,
                    Precision::FP16, p);
}

size_t CactusGraph::silu(size_t input) {
    return add_node(OpType::SILU, {input}, node(input).out.shape, Precision::FP16);
}

size_t CactusGraph::add(size_t a, size_t b) {
    if (node(a).out.total_size != node(b).out.total_size)
        throw std::runtime_error("add: broadcasting is not built (shapes must match)");
    return add_node(OpType::ADD, {a, b}, node(a).out.shape, Precision::FP16);
}

size_t CactusGraph::multiply(size_t a, size_t b) {
    if (node(a).out.total_size != node(b).out.total_size)
        throw std::runtime_error("multiply: broadcasting is not built (shapes must match)");
    return add_node(OpType::MULTIPLY, {a, b}, node(a).out.shape, Precision::FP16);
}

size_t CactusGraph::embedding(size_t table, size_t indices) {
    const auto& ts = node(table).out.shape;
    if (ts.size() != 2) throw std::runtime_error("embedding table must be 2D");
    return add_node(OpType::EMBEDDING, {table, indices}, {node(indices).out.total_size, ts[1]},
                    Precision::FP16);
}

size_t CactusGraph::embedding_checked_ids(size_t table, size_t indices) {
    const size_t id = embedding(table, indices);
    node(id).params.ids_checked = true;
    return id;
}

size_t CactusGraph::index(size_t input, size_t index_value, int dim) {
    const auto& s = node(input).out.shape;
    if (dim != 0 || s.empty()) throw std::runtime_error("index: only dim 0 is built");
    if (index_value >= s[0]) throw std::runtime_error("index out of range");
    OpParams p;
    p.index_value = index_value;
    p.axis = dim;
    std::vector<size_t> out(s.begin() + 1, s.end());
    if (out.empty()) out.push_back(1);
    return add_node(OpType::INDEX, {input}, out, node(input).out.precision, p);
}

size_t CactusGraph::reshape(size_t input, const std::vector<size_t>& new_shape) {
    if (numel(new_shape) != node(input).out.total_size)
        throw std::runtime_error("reshape: element count changes");
    OpParams p;
    p.new_shape = new_shape;
    return add_node(OpType::RESHAPE, {input}, new_shape, node(input).out.precision, p);
}

size_t CactusGraph::sample(size_t logits, float temperature, float top_p, size_t top_k, size_t random_seed,
                           const std::vector<std::pair<uint32_t, float>>& logit_bias) {
    if (node(logits).out.shape.empty()) throw std::runtime_error("Sample requires non-empty logits tensor");
    OpParams p;
    for (const auto& e : logit_bias) {
        p.bias_indices.push_back(e.first);
        p.bias_values.push_back(e.second);
    }
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.random_seed = random_seed
                        ? random_seed
                        : (size_t)std::chrono::high_resolution_clock::now().time_since_epoch().count();
    return add_node(OpType::SAMPLE, {logits}, {1}, Precision::FP32, p);
}

// ------------------------------------------------------------------ data
void CactusGraph::set_input(size_t id, const void* host, Precision precision) {
    GraphNode& n = node(id);
    if (n.op != OpType::INPUT) throw std::runtime_error("set_input on a non-input node");
    n.out.precision = precision;
    n.out.byte_size = n.out.total_size * precision_size(precision);
    if (!n.out.data || n.out.external) {
        n.out.data = pool_.acquire(n.out.byte_size);
        n.out.pooled_bytes = n.out.byte_size;
        n.out.external = false;
    }
    check_hip(cactus_hip_memcpy_h2d(n.out.data, host, n.out.byte_size, stream_), "set_input");
}

void CactusGraph::set_external_input(size_t id, void* dev, Precision precision) {
    GraphNode& n = node(id);
    if (n.op != OpType::INPUT) throw std::runtime_error("set_external_input on a non-input node");
    n.out.precision = precision;
    n.out.byte_size = n.out.total_size * precision_size(precision);
    n.out.data = dev;
    n.out.external = true;
}

void CactusGraph::set_grouped_scales(size_t id, size_t group_size, size_t num_groups,
                                     const void* scales) {
    BufferDesc& b = node(id).out;
    b.group_size = group_size;
    b.num_groups = num_groups;
    b.scales = scales;
}

void CactusGraph::set_packed_int4(size_t id, const void* packed, size_t packed_size) {
    BufferDesc& b = node(id).out;
    b.packed_int4 = packed;
    b.packed_int4_size = packed_size;
}

void* CactusGraph::get_output(size_t id) {
    const BufferDesc& b = node(id).out;
    if (!b.data) throw std::runtime_error("get_output: node has no data (not executed?)");
    auto& m = host_mirror_[id];
    m.resize(b.byte_size);
    check_hip(cactus_hip_memcpy_d2h(m.data(), b.data, b.byte_size, stream_), "get_output");
    return m.data();
}

// ------------------------------------------------------------------ tensor files
size_t CactusGraph::load_weights(const std::string& filename) {
    auto it = weight_cache_.find(filename);
    if (it != weight_cache_.end()) return it->second;
    CactFile f(filename);
    const CactHeader& h = f.header();
    const bool int4 = h.precision == static_cast<uint32_t>(Precision::INT4);
    const Precision eff = int4 ? Precision::INT8 : static_cast<Precision>(h.precision);
    const size_t elems = numel(h.shape);
    if (int4 && elems % 2) throw std::runtime_error(filename + ": INT4 tensor with an odd element count");
    const size_t want = int4 ? elems / 2 : elems * precision_size(eff);
    if (h.data_bytes != want)
        throw std::runtime_error(filename + ": " + std::to_string(h.data_bytes) + " data bytes for " +
                                 std::to_string(elems) + " elements");
    DeviceTensor t = upload_cact(f, stream_);
    owned_weights_.push_back(t.data);
    if (t.scales) owned_weights_.push_back(t.scales);
    const size_t id = input(h.shape, eff);
    set_external_input(id, t.data, eff);
    if (int4) {
        set_packed_int4(id, t.data, h.data_bytes);
        node(id).out.byte_size = h.data_bytes;
    }
    if (h.scales_bytes && h.group_size && h.num_groups) set_grouped_scales(id, h.group_size, h.num_groups, t.scales);
    weight_cache_[filename] = id;
    return id;
}

size_t CactusGraph::mmap_embeddings(const std::string& filename) {
    {
        CactFile f(filename);
        if (f.shape().size() != 2)
            throw std::runtime_error("Memory-mapped embeddings must be 2D [vocab_size, embedding_dim]");
    }
    return load_weights(filename);
}

void CactusGraph::save_node(size_t id, const std::string& filename) {
    execute();
    const BufferDesc& b = node(id).out;
    const bool packed = b.is_packed_int4();
    const void* src = packed ? b.packed_int4 : b.data;
    const size_t n = packed ? b.packed_int4_size : b.byte_size;
    if (!src) throw std::runtime_error("save_node: node has no data");
    std::vector<unsigned char> host(n);
    if (n) check_hip(cactus_hip_memcpy_d2h(host.data(), src, n, stream_), "save_node");
    std::vector<uint16_t> sc;
    const bool scaled = (b.precision == Precision::INT8) && b.group_size && b.num_groups && b.scales;
    if (scaled) {
        const size_t rows = b.shape.empty() ? 1 : b.shape[0];
        sc.resize(rows * b.num_groups);
        check_hip(cactus_hip_memcpy_d2h(sc.data(), b.scales, sc.size() * 2, stream_), "save_node scales");
    }
    check_hip(cactus_hip_stream_sync(stream_), "save_node sync");
    save_cact(filename, b.shape, packed ? Precision::INT4 : b.precision, host.data(), n,
              scaled ? sc.data() : nullptr, scaled ? b.group_size : 0, scaled ? b.num_groups : 0);
}

void CactusGraph::free_weights() {
    cactus_hip_stream_sync(stream_);
    for (void* p : owned_weights_) cactus_hip_free(p);
    owned_weights_.clear();
    weight_cache_.clear();
}

// ------------------------------------------------------------------ execution
void CactusGraph::allocate(GraphNode& n) {
    if (n.op == OpType::INPUT) {
        if (!n.out.data) throw std::runtime_error("input node " + std::to_string(n.id) + " has no data");
        return;
    }
    if (n.op == OpType::RESHAPE) {
        const BufferDesc& src = node(n.inputs[0]).out;
        n.out.data = src.data;
        n.out.external = true;
        n.out.group_size = src.group_size;
        n.out.num_groups = src.num_groups;
        n.out.scales = src.scales;
        n.out.activation_scales = src.activation_scales;
        return;
    }
    if (n.op == OpType::INDEX) {  // dim 0: a view (graph_ops_tensor.cpp:357-361)
        const BufferDesc& src = node(n.inputs[0]).out;
        const size_t slice = src.total_size / src.shape[0];
        n.out.data = static_cast<char*>(src.data) + n.params.index_value * slice * precision_size(src.precision);
        n.out.external = true;
        return;
    }
    if (!n.out.data) {
        n.out.data = pool_.acquire(n.out.byte_size);
        n.out.pooled_bytes = n.out.byte_size;
    }
    if (has_row_scales(n.op) && !n.out.activation_scales) {
        const auto& s = n.out.shape;
        const size_t rows = n.out.total_size / s.back();
        n.out.activation_scales = pool_.acquire(rows * sizeof(float));
    }
}

void CactusGraph::compute(GraphNode& n) {
    void* st = stream_;
    auto in = [&](int i) -> const BufferDesc& { return node(n.inputs[i]).out; };
    auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
    uint16_t* out16 = static_cast<uint16_t*>(n.out.data);
    switch (n.op) {
        case OpType::INPUT:
        case OpType::RESHAPE:
        case OpType::INDEX:
            return;
        case OpType::QUANTIZE_ACTIVATIONS: {  // graph_ops_nn.cpp:78-127
            const BufferDesc& x = in(0);
            if (x.precision != Precision::FP16) throw std::runtime_error("QUANTIZE_ACTIVATIONS requires FP16 input");
            const size_t K = x.shape.back(), M = x.total_size / K;
            check_hip(cactus_hip_quantize_activations(u16(x.data), static_cast<int8_t*>(n.out.data),
                                                      static_cast<float*>(n.out.activation_scales), M, K, st),
                      "quantize_activations");
            return;
        }
        case OpType::MATMUL_ADD: {
            const BufferDesc& a = in(0);
            const BufferDesc& b = in(1);
            const uint16_t* r = u16(in(2).data);
            const size_t K = a.shape.back();
            const size_t M = a.total_size / K;
            const size_t N = n.out.shape.back();
            const bool preq = a.precision == Precision::INT8 && a.activation_scales;
            if (!(b.is_packed_int4() || b.is_grouped_int8()) || (!preq && a.precision != Precision::FP16))
                throw std::runtime_error("matmul_add: needs grouped INT8/INT4 weights and INT8 or FP16 activations");
            const uint16_t* bs = u16(b.scales);
            int rc;
            if (b.is_packed_int4()) {
                const uint8_t* bp = static_cast<const uint8_t*>(b.packed_int4);
                rc = preq ? cactus_hip_matmul_int4_add(static_cast<const int8_t*>(a.data),
                                                      static_cast<const float*>(a.activation_scales), bp, bs, r,
                                                      out16, M, K, N, b.group_size, st)
                          : cactus_hip_matmul_int4_f16act_add(u16(a.data), bp, bs, r, out16, M, K, N, b.group_size,
                                                              st);
            } else {
                const int8_t* bw = static_cast<const int8_t*>(b.data);
                rc = preq ? cactus_hip_matmul_int8_add(static_cast<const int8_t*>(a.data),
                                                      static_cast<const float*>(a.activation_scales), bw, bs, r,
                                                      out16, M, K, N, b.group_size, st)
                          : cactus_hip_matmul_int8_f16act_add(u16(a.data), bw, bs, r, out16, M, K, N, b.group_size,
                                                              st);
            }
            check_hip(rc, "matmul_add");
            return;
        }
        case OpType::MATMUL: {  // graph_ops_nn.cpp:129-231
            const BufferDesc& a = in(0);
            const BufferDesc& b = in(1);
            const size_t K = a.shape.back();
            const size_t M = a.total_size / K;
            const size_t N = n.out.shape.back();
            const bool preq = a.precision == Precision::INT8 && a.activation_scales;
            if (b.is_packed_int4() || b.is_grouped_int8()) {
                if (!n.params.pretransposed_rhs)
                    throw std::runtime_error("grouped INT8/INT4 matmul requires pretransposed weights");
                if (!preq && a.precision != Precision::FP16)
                    throw std::runtime_error("grouped matmul requires INT8 (pre-quantized) or FP16 activations");
                const uint16_t* bs = u16(b.scales);
                if (b.is_packed_int4()) {
                    const uint8_t* bp = static_cast<const uint8_t*>(b.packed_int4);
                    if (preq)
                        check_hip(cactus_hip_matmul_int4(static_cast<const int8_t*>(a.data),
                                                         static_cast<const float*>(a.activation_scales),
                                                         bp, bs, out16, M, K, N, b.group_size, st),
                                  "matmul_int4");
                    else
                        check_hip(cactus_hip_matmul_int4_f16act(u16(a.data), bp, bs, out16, M, K, N,
                                                                b.group_size, st),
                                  "matmul_int4_f16act");
                } else {
                    const int8_t* bw = static_cast<const int8_t*>(b.data);
                    if (preq)
                        check_hip(cactus_hip_matmul_int8(static_cast<const int8_t*>(a.data),
                                                         static_cast<const float*>(a.activation_scales),
                                                         bw, bs, out16, M, K, N, b.group_size, st),
                                  "matmul_int8");
                    else
                        check_hip(cactus_hip_matmul_int8_f16act(u16(a.data), bw, bs, out16, M, K, N,
                                                                b.group_size, st),
                                  "matmul_int8_f16act");
                }
                return;
            }
            if (a.precision != Precision::FP16 || b.precision != Precision::FP16)
                throw std::runtime_error("FP16 matmul requires FP16 operands");
            if (n.params.pretransposed_rhs) {
                check_hip(cactus_hip_matmul_f16(u16(a.data), u16(b.data), out16, M, K, N, st), "matmul_f16");
            } else {
                void* t = pool_.acquire(b.byte_size);
                check_hip(cactus_hip_transpose_2d_f16(u16(b.data), static_cast<uint16_t*>(t), b.shape[0],
                                                      b.shape[1], st),
                          "transpose");
                check_hip(cactus_hip_matmul_f16(u16(a.data), u16(t), out16, M, K, N, st), "matmul_f16");
                check_hip(cactus_hip_stream_sync(st), "matmul_f16 sync");
                pool_.release(t, b.byte_size);
            }
            return;
        }
        case OpType::RMS_NORM: {  // graph_ops_nn.cpp:233-251
            const BufferDesc& x = in(0);
            if (x.shape.size() != 2) throw std::runtime_error("RMS normalization requires 2D input tensor");
            check_hip(cactus_hip_rms_norm_f16(u16(x.data), u16(in(1).data), out16, x.shape[0], x.shape[1],
                                              n.params.epsilon, st),
                      "rms_norm");
            return;
        }
        case OpType::RMS_NORM_QUANTIZE: {
            const BufferDesc& x = in(0);
            if (x.shape.size() != 2) throw std::runtime_error("RMS normalization requires 2D input tensor");
            check_hip(cactus_hip_rms_norm_quantize_f16(u16(x.data), u16(in(1).data), static_cast<int8_t*>(n.out.data),
                                                       static_cast<float*>(n.out.activation_scales), x.shape[0],
                                                       x.shape[1], n.params.epsilon, st),
                      "rms_norm_quantize");
            return;
        }
        case OpType::SILU_MUL_QUANTIZE: {
            const BufferDesc& gt = in(0);
            const size_t K = gt.shape.back(), M = gt.total_size / K;
            check_hip(cactus_hip_silu_mul_quantize_f16(u16(gt.data), u16(in(1).data), static_cast<int8_t*>(n.out.data),
                                                       static_cast<float*>(n.out.activation_scales), M, K, st),
                      "silu_mul_quantize");
            return;
        }
        case OpType::RMS_NORM_ROPE: {
            const auto& sh = in(0).shape;
            check_hip(cactus_hip_rms_norm_rope_f16(u16(in(0).data), u16(in(1).data), out16, sh[0], sh[1], sh[2], sh[3],
                                                   n.params.position_offset, n.params.theta, n.params.epsilon, st),
                      "rms_norm_rope");
            return;
        }
        case OpType::ROPE: {  // graph_ops_nn.cpp:253-277
            const auto& s = in(0).shape;
            if (s.size() < 4) throw std::runtime_error("RoPE operation requires 4D tensor");
            check_hip(cactus_hip_rope_f16(u16(in(0).data), out16, s[0], s[1], s[2], s[3],
                                          n.params.position_offset, n.params.theta, st),
                      "rope");
            return;
        }
        case OpType::SOFTMAX: {  // graph_ops_nn.cpp:279-300
            const auto& s = in(0).shape;
            if (s.size() < 2) throw std::runtime_error("Softmax operation requires at least 2D tensor");
            const size_t V = s.back();
            check_hip(cactus_hip_softmax_f16(u16(in(0).data), out16, in(0).total_size / V, 1, V, st),
                      "softmax");
            return;
        }
        case OpType::ATTENTION: {  // graph_ops_nn.cpp:302-338
            const auto& q = in(0).shape;
            const auto& k = in(1).shape;
            if (q.size() < 4) throw std::runtime_error("Attention operation requires 4D tensors");
            check_hip((n.params.tolerance ? cactus_hip_attention_f16_fast : cactus_hip_attention_f16)(
                          u16(in(0).data), u16(in(1).data), u16(in(2).data), out16, q[0], q[1], k[1], q[2], k[2],
                          q[3], n.params.scale, nullptr, n.params.position_offset, n.params.window_size,
                          n.params.is_causal ? 1 : 0, st),
                      "attention");
            return;
        }
        case OpType::ATTENTION_INT8_HYBRID: {  // graph_ops_nn.cpp:340-371
            const auto& q = in(0).shape;
            const auto& p = n.params;
            check_hip((p.tolerance ? cactus_hip_attention_hybrid_int8_fp16_fast
                                   : cactus_hip_attention_hybrid_int8_fp16)(
                          u16(in(0).data), p.cached_keys_int8, p.cached_values_int8, p.cached_k_scales,
                          p.cached_v_scales, u16(in(1).data), u16(in(2).data), out16, q[0], q[1],
                          p.cache_seq_len, in(1).shape[1], q[2], p.num_kv_heads, p.head_dim, p.scale,
                          p.position_offset, 1, 128, st),
                      "attention_int8_hybrid");
            return;
        }
        case OpType::SILU:
            check_hip(cactus_hip_silu_f16(u16(in(0).data), out16, in(0).total_size, st), "silu");
            return;
        case OpType::ADD:
            check_hip(cactus_hip_add_f16(u16(in(0).data), u16(in(1).data), out16, n.out.total_size, st), "add");
            return;
        case OpType::MULTIPLY:
            check_hip(cactus_hip_multiply_f16(u16(in(0).data), u16(in(1).data), out16, n.out.total_size, st),
                      "multiply");
            return;
        case OpType::EMBEDDING: {  // graph_ops_tensor.cpp:301-329 (FP16 table, FP32 ids)
            const BufferDesc& t = in(0);
            const BufferDesc& ids = in(1);
            if (t.precision != Precision::FP16 || ids.precision != Precision::FP32)
                throw std::runtime_error("embedding: FP16 table with FP32 indices only");
            int* err = nullptr;
            if (!n.params.ids_checked) {
                if (!embed_err_) check_hip(cactus_hip_malloc(reinterpret_cast<void**>(&embed_err_), 4), "malloc");
                check_hip(cactus_hip_memset(embed_err_, 0, 4, st), "memset");
                err = embed_err_;
                embed_check_pending_ = true;
            }
            check_hip(cactus_hip_embedding_f16(u16(t.data), static_cast<const float*>(ids.data), out16,
                                               ids.total_size, t.shape[1], t.shape[0], err, st),
                      "embedding");
            return;
        }
        case OpType::SAMPLE: {  // graph_ops_sample.cpp:8-39
            const BufferDesc& l = in(0);
            if (l.shape.size() != 2) throw std::runtime_error("Sample expects 2D logits tensor [seq_len, vocab_size]");
            const size_t V = l.shape[1];
            if (l.precision == Precision::FP32) {
                const float* last = static_cast<const float*>(l.data) + (l.shape[0] - 1) * V;
                const auto& bv = n.params.bias_values;
                check_hip(cactus_hip_sample_f32(last, static_cast<uint32_t*>(n.out.data), V, n.params.temperature,
                                                n.params.top_p, n.params.top_k, n.params.random_seed,
                                                bv.empty() ? nullptr : bv.data(),
                                                bv.empty() ? nullptr : n.params.bias_indices.data(), bv.size(),
                                                st),
                          "sample");
                return;
            }
            const uint16_t* last = u16(l.data) + (l.shape[0] - 1) * V;
            check_hip(cactus_hip_sample_f16(last, static_cast<uint32_t*>(n.out.data), V, n.params.temperature,
                                            n.params.top_p, n.params.top_k, n.params.random_seed, st),
                      "sample");
            return;
        }
    }
}

// Consecutive matmul nodes over one pre-quantized activation (the q/k/v and
// gate/up projections, model_qwen.cpp:55-57 and :112-113) with weights of one
// format, K and group size run as one launch; each output is what its own
// node computes.  Returns the number of nodes computed from node i (0: node
// i is not such a run).
size_t CactusGraph::compute_shared_matmuls(size_t i) {
    auto eligible = [&](const GraphNode& n) {
        if (n.op != OpType::MATMUL || !n.params.pretransposed_rhs) return false;
        const BufferDesc& a = node(n.inputs[0]).out;
        const BufferDesc& b = node(n.inputs[1]).out;
        return a.precision == Precision::INT8 && a.activation_scales && (b.is_packed_int4() || b.is_grouped_int8());
    };
    const GraphNode& n0 = *nodes_[i];
    if (!eligible(n0)) return 0;
    const BufferDesc& a = node(n0.inputs[0]).out;
    const BufferDesc& b0 = node(n0.inputs[1]).out;
    const size_t K = a.shape.back(), M = a.total_size / K;
    if (M < 32) return 0;   // decode sizes: the fused GEMV per node
    size_t count = 1;
    while (count < 3 && i + count < nodes_.size()) {
        const GraphNode& nj = *nodes_[i + count];
        if (!eligible(nj) || nj.inputs[0] != n0.inputs[0]) break;
        const BufferDesc& bj = node(nj.inputs[1]).out;
        if (bj.is_packed_int4() != b0.is_packed_int4() || bj.group_size != b0.group_size) break;
        count++;
    }
    if (count < 2) return 0;
    const void* B[3];
    const uint16_t* Bs[3];
    uint16_t* C[3];
    size_t N[3];
    for (size_t j = 0; j < count; j++) {
        GraphNode& nj = *nodes_[i + j];
        if (j > 0) allocate(nj);
        const BufferDesc& b = node(nj.inputs[1]).out;
        B[j] = b.is_packed_int4() ? b.packed_int4 : b.data;
        Bs[j] = static_cast<const uint16_t*>(b.scales);
        C[j] = static_cast<uint16_t*>(nj.out.data);
        N[j] = nj.out.shape.back();
    }
    check_hip(cactus_hip_matmul_grouped_multi(static_cast<const int8_t*>(a.data),
                                              static_cast<const float*>(a.activation_scales), count, B, Bs, C, N, M,
                                              K, b0.group_size, b0.is_packed_int4() ? 1 : 0, stream_),
              "matmul (shared activation)");
    return count;
}

// Two consecutive head RMSNorm + RoPE nodes of one sequence (q and k,
// model_qwen.cpp:63-70 and :78-80) run as one launch.  Returns 2 when nodes
// i and i + 1 were computed, else 0.
size_t CactusGraph::compute_qk_rope(size_t i) {
    if (i + 1 >= nodes_.size()) return 0;
    GraphNode& a = *nodes_[i];
    GraphNode& b = *nodes_[i + 1];
    if (a.op != OpType::RMS_NORM_ROPE || b.op != OpType::RMS_NORM_ROPE) return 0;
    const auto& sa = node(a.inputs[0]).out.shape;
    const auto& sb = node(b.inputs[0]).out.shape;
    if (sa[0] != sb[0] || sa[1] != sb[1] || sa[3] != sb[3] || a.params.position_offset != b.params.position_offset ||
        a.params.theta != b.params.theta || a.params.epsilon != b.params.epsilon)
        return 0;
    allocate(b);
    auto u16 = [&](size_t id) { return static_cast<const uint16_t*>(node(id).out.data); };
    check_hip(cactus_hip_rms_norm_rope_qk_f16(u16(a.inputs[0]), u16(a.inputs[1]), static_cast<uint16_t*>(a.out.data),
                                              sa[2], u16(b.inputs[0]), u16(b.inputs[1]),
                                              static_cast<uint16_t*>(b.out.data), sb[2], sa[0], sa[1], sa[3],
                                              a.params.position_offset, a.params.theta, a.params.epsilon, stream_),
              "rms_norm_rope (q and k)");
    return 2;
}

void CactusGraph::execute() {
    const bool hooks = !before_.empty() || !after_.empty();
    auto run = [](std::unordered_map<size_t, std::function<void()>>& m, size_t id) {
        auto it = m.find(id);
        if (it != m.end()) it->second();
    };
    for (size_t i = 0; i < nodes_.size(); i++) {
        allocate(*nodes_[i]);
        if (hooks) run(before_, nodes_[i]->id);
        size_t done = compute_shared_matmuls(i);
        if (!done) done = compute_qk_rope(i);
        if (!done) {
            compute(*nodes_[i]);
            done = 1;
        }
        if (hooks)
            for (size_t j = i; j < i + done; j++) run(after_, nodes_[j]->id);
        i += done - 1;
    }
    if (embed_check_pending_) {
        embed_check_pending_ = false;
        int err = 0;
        check_hip(cactus_hip_memcpy_d2h(&err, embed_err_, 4, stream_), "embedding check");
        if (err) throw std::runtime_error("Embedding index out of bounds");
    }
}

void CactusGraph::release_outputs() {
    for (auto& n : nodes_) {
        if (n->out.pooled_bytes && !n->out.external) {
            pool_.release(n->out.data, n->out.pooled_bytes);
            n->out.data = nullptr;
            n->out.pooled_bytes = 0;
        }
        if (has_row_scales(n->op) && n->out.activation_scales) {
            const size_t rows = n->out.total_size / n->out.shape.back();
            pool_.release(n->out.activation_scales, rows * sizeof(float));
            n->out.activation_scales = nullptr;
        }
    }
}

void CactusGraph::soft_reset() {
    // graph_execute.cpp:640-675: keep INPUT nodes whose data is external
    // (weights), drop everything else; buffers go back to the pool
    check_hip(cactus_hip_stream_sync(stream_), "soft_reset sync");
    before_.clear();
    after_.clear();
    std::vector<std::unique_ptr<GraphNode>> keep;
    size_t max_id = 0;
    bool any = false;
    for (auto& n : nodes_) {
        if (n->op == OpType::INPUT && n->out.external) {
            max_id = std::max(max_id, n->id);
            any = true;
            keep.push_back(std::move(n));
        } else if (n->out.pooled_bytes && !n->out.external) {
            pool_.release(n->out.data, n->out.pooled_bytes);
            if (has_row_scales(n->op) && n->out.activation_scales)
                pool_.release(n->out.activation_scales, n->out.total_size / n->out.shape.back() * sizeof(float));
        }
    }
    nodes_ = std::move(keep);
    index_.clear();
    for (size_t i = 0; i < nodes_.size(); i++) index_[nodes_[i]->id] = i;
    next_id_ = any ? max_id + 1 : 0;
    host_mirror_.clear();
}

void CactusGraph::hard_reset() {
    release_outputs();
    before_.clear();
    after_.clear();
    nodes_.clear();
    index_.clear();
    host_mirror_.clear();
    next_id_ = 0;
    pool_.clear();
    free_weights();
}

}  // namespace cactus
