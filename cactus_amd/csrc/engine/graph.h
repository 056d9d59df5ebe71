// graph.h -- device-resident subset of the reference's CactusGraph op API
// (cactus/graph/graph.h:99-500).  Nodes are built in order, executed
// serially in insertion order (graph_execute.cpp:231-395), and every
// compute node dispatches one entry point of the kernel C ABI
// (include/cactus_hip.h) on the graph's stream.  Buffers live in device
// memory; get_output() copies a node's result to a host mirror.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <functional>
#include <unordered_map>
#include <vector>

namespace cactus {

// graph.h:99-104 (same order: INT8, FP16, FP32, INT4)
enum class Precision { INT8, FP16, FP32, INT4 };

enum class OpType {
    INPUT, MATMUL, RMS_NORM, ROPE, SOFTMAX, ATTENTION, ATTENTION_INT8_HYBRID,
    SILU, ADD, MULTIPLY, EMBEDDING, INDEX, RESHAPE, SAMPLE, QUANTIZE_ACTIVATIONS,
    RMS_NORM_QUANTIZE,   // RMS_NORM feeding only matmuls, fused with their row quantization
    SILU_MUL_QUANTIZE,   // silu(gate) * up feeding only a matmul, fused with its row quantization
    RMS_NORM_ROPE,       // per-head RMSNorm of q or k followed by their RoPE
    MATMUL_ADD,          // grouped matmul followed by the residual add
};

// nodes whose output is INT8 codes with per-row activation scales
inline bool has_row_scales(OpType op) {
    return op == OpType::QUANTIZE_ACTIVATIONS || op == OpType::RMS_NORM_QUANTIZE ||
           op == OpType::SILU_MUL_QUANTIZE;
}

size_t precision_size(Precision p);

// graph_core.cpp:21-58: size-bucketed reuse of device allocations
class BufferPool {
public:
    BufferPool() = default;
    ~BufferPool();
    BufferPool(const BufferPool&) = delete;
    BufferPool& operator=(const BufferPool&) = delete;
    void* acquire(size_t bytes);
    void release(void* ptr, size_t bytes);
    void clear();
    size_t pool_bytes() const { return pool_bytes_; }

private:
    static size_t round_up(size_t b);
    std::map<size_t, std::vector<void*>> free_;
    size_t pool_bytes_ = 0;
};

struct BufferDesc {
    std::vector<size_t> shape;
    size_t total_size = 0;       // elements
    size_t byte_size = 0;
    Precision precision = Precision::FP16;
    void* data = nullptr;        // device
    bool external = false;       // not owned (weights, views, caller memory)
    size_t pooled_bytes = 0;     // >0 when taken from the pool

    // grouped-quantized weights (graph.h:234-250)
    size_t group_size = 0;
    size_t num_groups = 0;
    const void* scales = nullptr;       // device fp16 [rows][num_groups]
    const void* packed_int4 = nullptr;  // device [rows][K/2]
    size_t packed_int4_size = 0;

    // activation row scales of a QUANTIZE_ACTIVATIONS node
    void* activation_scales = nullptr;  // device f32 [rows]

    bool is_grouped_int8() const { return precision == Precision::INT8 && group_size > 0; }
    bool is_packed_int4() const { return packed_int4 != nullptr && packed_int4_size > 0; }
};

struct OpParams {
    float scale = 1.0f;
    float theta = 10000.0f;
    float epsilon = 1e-6f;
    int axis = -1;
    bool pretransposed_rhs = false;
    size_t position_offset = 0;
    size_t window_size = 0;
    bool is_causal = true;
    std::vector<size_t> new_shape;
    float temperature = 0.0f;
    float top_p = 0.0f;
    size_t top_k = 0;
    size_t random_seed = 0;   // graph_builder.cpp:408: the build time in clock ticks
    std::vector<float> bias_values;       // logit bias (graph_builder.cpp:411-418)
    std::vector<uint32_t> bias_indices;
    size_t index_value = 0;
    bool ids_checked = false;   // EMBEDDING: indices validated on the host (no device check)
    // ATTENTION_INT8_HYBRID (graph_builder.cpp:301-316)
    const int8_t* cached_keys_int8 = nullptr;
    const int8_t* cached_values_int8 = nullptr;
    const float* cached_k_scales = nullptr;
    const float* cached_v_scales = nullptr;
    size_t cache_seq_len = 0;
    size_t num_kv_heads = 0;
    size_t head_dim = 0;
    // attention nodes: the tolerance-mode split-K kernels for decode-shaped
    // queries (cactus_hip_attention_*_fast) instead of the exact ones
    bool tolerance = false;
};

struct GraphNode {
    size_t id;
    OpType op;
    std::vector<size_t> inputs;
    BufferDesc out;
    OpParams params;
};

class CactusGraph {
public:
    explicit CactusGraph(void* stream = nullptr);
    // attention nodes built from now on run the tolerance-mode kernels
    void set_attention_tolerance(bool on) { attention_tolerance_ = on; }
    ~CactusGraph();
    CactusGraph(const CactusGraph&) = delete;
    CactusGraph& operator=(const CactusGraph&) = delete;

    // --- builders (graph.h:386-460)
    size_t input(const std::vector<size_t>& shape, Precision precision = Precision::INT8);
    size_t matmul(size_t a, size_t b, bool pretransposed_rhs = false);
    size_t quantize_activations(size_t input);
    size_t rms_norm(size_t input, size_t weight, float epsilon = 1e-5f);
    // rms_norm + quantize_activations in one node (same codes and scales)
    size_t rms_norm_quantize(size_t input, size_t weight, float epsilon = 1e-5f);
    // multiply(silu(gate), up) + quantize_activations in one node
    size_t silu_mul_quantize(size_t gate, size_t up);
    // rms_norm over head rows of a [B][S][H][d] tensor, then rope
    size_t rms_norm_rope(size_t input, size_t weight, float epsilon, float theta, size_t position_offset);
    // add(residual, matmul(a, b)) for pretransposed grouped INT8/INT4 weights
    size_t matmul_add(size_t a, size_t b, size_t residual);
    size_t rope(size_t input, float theta, size_t position_offset = 0);
    size_t softmax(size_t input, int axis = -1);
    size_t attention(size_t q, size_t k, size_t v, float scale, size_t position_offset = 0,
                     size_t window_size = 0, bool is_causal = true);
    size_t attention_int8_hybrid(size_t q, size_t k_new, size_t v_new, float scale,
                                 size_t position_offset, const int8_t* cached_keys,
                                 const int8_t* cached_values, const float* k_scales,
                                 const float* v_scales, size_t cache_len, size_t num_kv_heads,
                                 size_t head_dim);
    size_t silu(size_t input);
    size_t add(size_t a, size_t b);
    size_t multiply(size_t a, size_t b);
    size_t embedding(size_t table, size_t indices);
    // the same node for indices the caller has already checked against the
    // table's row count on the host: execute() then needs no device read-back
    size_t embedding_checked_ids(size_t table, size_t indices);
    size_t index(size_t input, size_t index_value, int dim);
    size_t reshape(size_t input, const std::vector<size_t>& new_shape);
    // random_seed 0: the reference's seed, the clock at build time
    // logit_bias reaches only FP32 logits: the FP16 sampler discards it
    size_t sample(size_t logits, float temperature = 0.6f, float top_p = 0.95f, size_t top_k = 20,
                  size_t random_seed = 0, const std::vector<std::pair<uint32_t, float>>& logit_bias = {});

    // --- data
    void set_input(size_t node, const void* host_data, Precision precision);
    void set_external_input(size_t node, void* device_data, Precision precision);
    void set_grouped_scales(size_t node, size_t group_size, size_t num_groups,
                            const void* device_scales);
    void set_packed_int4(size_t node, const void* device_packed, size_t packed_size);
    void* get_output(size_t node);                      // host mirror (synchronous)
    const BufferDesc& get_output_buffer(size_t node) const;

    // --- tensor files (graph_io.cpp:25-101, :228-320): a CACT file becomes an
    // INPUT node over a device copy the graph owns.  INT4 stays packed, the
    // node keeping its shape in elements with precision INT8 (graph.h:526-528).
    // Cached by file name; soft_reset keeps them, hard_reset frees them.
    size_t load_weights(const std::string& filename);
    size_t mmap_weights(const std::string& filename) { return load_weights(filename); }
    size_t mmap_embeddings(const std::string& filename);   // 2D [vocab][dim] only
    // GraphFile::save_node (graph_io.cpp:145-222): executes the graph, then
    // writes the node's data (and INT8 group scales) with alignment 32
    void save_node(size_t node, const std::string& filename);

    // --- execution
    // Callbacks run by execute() on the host around a node's launch: `before`
    // just before it is enqueued, `after` once it (with the nodes the
    // executor merges into the same launch) has been enqueued.  Keyed by node
    // id; soft_reset drops them.  Used to order work across streams.
    void before_node(size_t id, std::function<void()> f) { before_[id] = std::move(f); }
    void after_node(size_t id, std::function<void()> f) { after_[id] = std::move(f); }
    void execute();
    void soft_reset();   // drop all non-INPUT nodes (weights stay)
    void hard_reset();
    void* stream() const { return stream_; }
    size_t node_count() const { return nodes_.size(); }

private:
    bool attention_tolerance_ = false;
    size_t add_node(OpType op, const std::vector<size_t>& inputs, const std::vector<size_t>& shape,
                    Precision precision, const OpParams& params = {});
    GraphNode& node(size_t id);
    const GraphNode& node(size_t id) const;
    void allocate(GraphNode& n);
    void compute(GraphNode& n);
    size_t compute_shared_matmuls(size_t i);
    size_t compute_qk_rope(size_t i);
    void release_outputs();

    void* stream_;
    std::unordered_map<size_t, std::function<void()>> before_, after_;
    size_t next_id_ = 0;
    std::vector<std::unique_ptr<GraphNode>> nodes_;
    std::unordered_map<size_t, size_t> index_;
    BufferPool pool_;
    std::unordered_map<size_t, std::vector<unsigned char>> host_mirror_;
    // activation quantization reuse across matmuls with the same lhs
    // (graph_ops_nn.cpp:15-17, 36-38), keyed by the lhs node id
    size_t quant_src_ = SIZE_MAX;
    void* quant_codes_ = nullptr;
    void* quant_scales_ = nullptr;
    size_t quant_cap_ = 0, quant_rows_cap_ = 0;
    int* embed_err_ = nullptr;
    bool embed_check_pending_ = false;   // an unchecked embedding ran in this execute()
    // device copies of loaded tensor files
    std::unordered_map<std::string, size_t> weight_cache_;
    std::vector<void*> owned_weights_;
    void free_weights();
};

void check_hip(int rc, const char* what);

}  // namespace cactus
