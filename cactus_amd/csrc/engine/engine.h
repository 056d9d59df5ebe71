// engine.h -- device KV cache and the Qwen3 model over the device graph
// (reference: cactus/engine/engine.h KVCache :325-382, Model :473-577;
// cactus/models/model_qwen.cpp).
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

#include "cactus_engine.h"
#include "graph.h"

namespace cactus {

// Device buffer owned by the engine (weights, cache).
struct DevBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    explicit DevBuf(size_t n);
    ~DevBuf();
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; o.bytes = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept;
    void upload(const void* host, size_t n, void* stream);
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
};

// INT8 KV cache, one per-token/per-kv-head scale per 128 dims
// (KV_QUANT_GROUP_SIZE, kernel.h:18; engine/engine_cache.cpp), with the
// reference's sliding window and attention sinks.  Storage holds max_seq
// tokens per layer (the context size); a window, when set, is at most that.
class KVCache {
public:
    static constexpr size_t GROUP = 128;
    void init(size_t layers, size_t max_seq, size_t kv_heads, size_t head_dim);
    // KVCache::set_window_size (engine_cache.cpp:25-46): window 0 = none;
    // the first `window` slots become codes 0, scales 1.0
    void set_window(size_t window, size_t sink, void* stream);
    void reset() { current_seq_len = 0; total_seq_len = 0; }
    bool is_empty() const { return current_seq_len == 0; }
    // KVCache::update_from_graph (engine_cache.cpp:103-330): k[l], v[l] are
    // the fp16 rows [seq][kv_heads][head_dim] of layer l's new tokens.
    // Throws where the reference's update is undefined (a sliding step
    // longer than window - sink) or the storage would overflow.
    void update(const std::vector<const void*>& k, const std::vector<const void*>& v, size_t seq, void* stream);
    // The non-sliding append of update() split in two, for a prefill whose
    // chunks overlap on several streams: put_layer writes layer l's seq new rows
    // at slot `at` (the cache length before the chunk), appended() then
    // advances the lengths once for the chunk.  Callers check fits(seq).
    bool fits(size_t seq) const { return window_size == 0 && current_seq_len + seq <= max_seq_len; }
    void put_layer(size_t l, const void* k, const void* v, size_t seq, size_t at, void* stream);
    void appended(size_t seq);
    // After a one-token decode step into a full window (the fused path):
    // the step attended over all `window` cached tokens plus its own and
    // appended at slot `window` (the spare slot); tokens [sink + 1, window + 1)
    // move down by one in every layer and the device step state's cache
    // length returns to `window` -- the content update_from_graph leaves.
    void slide_after_step(uint32_t* state, void* stream);
    bool step_slides() const { return window_size > 0 && current_seq_len + 1 > window_size; }
    const int8_t* keys(size_t l) const { return k_[l].as<int8_t>(); }
    const int8_t* values(size_t l) const { return v_[l].as<int8_t>(); }
    const float* key_scales(size_t l) const { return ks_[l].as<float>(); }
    const float* value_scales(size_t l) const { return vs_[l].as<float>(); }
    int8_t* keys_mut(size_t l) { return k_[l].as<int8_t>(); }
    int8_t* values_mut(size_t l) { return v_[l].as<int8_t>(); }
    float* key_scales_mut(size_t l) { return ks_[l].as<float>(); }
    float* value_scales_mut(size_t l) { return vs_[l].as<float>(); }
    // fp32 product tiles of the values (cactus_hip_kv_shadow_update)
    float* value_products(size_t l) { return vsh_[l].as<float>(); }
    size_t groups() const { return (head_dim + GROUP - 1) / GROUP; }

    size_t current_seq_len = 0, total_seq_len = 0;
    size_t max_seq_len = 0, num_layers = 0, num_kv_heads = 0, head_dim = 0;
    size_t slots = 0;      // storage tokens per layer: max_seq_len + 1 (the fused step's spare slot)
    size_t window_size = 0, sink_size = 0;
    size_t resident = 0;   // tokens the reference's per-layer vectors would hold

private:
    void put(const std::vector<const void*>& k, const std::vector<const void*>& v, size_t row0, size_t n, size_t at,
             void* stream);
    void shift(size_t dst, size_t src, size_t count, uint32_t* state, uint32_t len, void* stream);
    std::vector<DevBuf> k_, v_, ks_, vs_, vsh_;
    DevBuf table_, temp_;   // device layer records and move buffer of cactus_hip_kv_window_shift
};

struct QwenLayer {
    DevBuf input_norm, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s, q_norm, k_norm, post_norm;
    DevBuf gate_w, gate_s, up_w, up_s, down_w, down_s;
    // graph node ids of the weights
    size_t n_input_norm, n_q, n_k, n_v, n_o, n_q_norm, n_k_norm, n_post_norm, n_gate, n_up, n_down;
};

class FusedDecoder;  // fused per-layer decode path (decode_fused.cpp)

class QwenModel {
public:
    QwenModel(const cactus_qwen_config& cfg, const cactus_qwen_layer_weights* layers,
              const uint16_t* embedding, const uint16_t* output_norm);
    ~QwenModel();

    void reset();
    void prefill(const std::vector<uint32_t>& tokens);
    uint32_t decode(uint32_t token);
    // n greedy steps from `token` (decode mode 1 keeps them on the device)
    void decode_many(uint32_t token, size_t n, uint32_t* out);
    void set_decode_mode(int mode);
    // 0: exact attention (bit-identical to the reference); 1: tolerance
    // mode for every attention node: split-K kernels for decode steps, FP16
    // MFMA flash attention for prefill chunks (within 1e-3 + 1e-2 |ref|)
    void set_attention_mode(int mode);
    int attention_mode() const { return attention_mode_; }
    void set_kv_window(size_t window, size_t sink);
    // Model::decode's temperature / top_p / top_k (engine_model.cpp:221-250);
    // all zero = greedy.  seed 0 = the reference's clock seed per step
    void set_sampling(float temperature, float top_p, size_t top_k, size_t seed);
    bool greedy() const { return temperature_ == 0.0f && top_p_ <= 0.0f && top_k_ == 0; }
    int decode_mode() const { return decode_mode_; }

    const cactus_qwen_config& config() const { return cfg_; }
    KVCache& cache() { return cache_; }
    CactusGraph& graph() { return *graph_; }
    void* stream() const { return stream_; }
    size_t last_hidden_node() const { return last_hidden_; }
    size_t last_logits_node() const { return last_logits_; }
    // fp16 logits [vocab] of the last decode step, wherever that step kept
    // them (the graph's logits node, or the fused decoder's buffer); null if
    // none was kept since the last reset or prefill
    const void* last_logits_data() const;
    const QwenLayer& layer(size_t i) const { return layers_[i]; }
    const DevBuf& embedding() const { return embedding_; }
    const DevBuf& output_norm() const { return out_norm_; }
    float attention_scale() const { return attn_scale_; }

private:
    size_t forward(const std::vector<uint32_t>& tokens);
    // the reference's embedding range check, on the host ids
    void check_token_ids(const std::vector<uint32_t>& tokens) const;
    size_t shared_matmul_input(size_t x);
    size_t norm_for_matmuls(size_t h, size_t weight);
    static constexpr size_t NO_RESIDUAL = ~(size_t)0;
    // residual: a node added to the last matmul's output (fused), or NO_RESIDUAL
    size_t build_attention(size_t x, uint32_t l, size_t pos, size_t residual = NO_RESIDUAL);
    size_t build_mlp(size_t x, uint32_t l, size_t residual = NO_RESIDUAL);
    size_t build_block(size_t h, uint32_t l, size_t pos);
    void update_kv_cache(size_t seq);

    cactus_qwen_config cfg_;
    void* stream_ = nullptr;
    std::unique_ptr<CactusGraph> graph_;
    std::vector<QwenLayer> layers_;
    DevBuf embedding_, out_norm_;
    size_t n_embedding_ = 0, n_out_norm_ = 0;
    KVCache cache_;
    float attn_scale_ = 0.0f;
    std::vector<size_t> k_nodes_, v_nodes_, att_nodes_;
    // Prefill with consecutive chunks overlapping on kPrefillStreams streams:
    // chunk i of n runs on stream (n - 1 - i) % kPrefillStreams, stream 0
    // being the model's own with graph_ (so the last chunk is there), the
    // others pf_streams_ with pf_graphs_.  Each chunk appends layer l's KV
    // rows as soon as they exist and records kv_ev_[stream][l]; the next
    // chunk's layer-l attention waits for that event.
    // three measured fastest on MI355X (4096-token prefill: 29 ms against
    // 31-35 ms with two and 37 ms with four, tolerance mode)
    static constexpr int kPrefillStreams = 3;
    void prefill_overlapped(const std::vector<uint32_t>& tokens, size_t chunk);
    void add_weight_nodes(CactusGraph& g);
    CactusGraph* cur_ = nullptr;   // the graph the builders extend
    std::vector<void*> pf_streams_;
    std::vector<std::unique_ptr<CactusGraph>> pf_graphs_;
    std::vector<std::vector<void*>> kv_ev_;
    std::vector<void*> join_ev_;
    size_t last_hidden_ = SIZE_MAX, last_logits_ = SIZE_MAX;
    bool fused_logits_ = false;   // the last step was a fused one (logits in fused_->logits())
    int decode_mode_ = 0;
    int attention_mode_ = 0;
    float temperature_ = 0.0f, top_p_ = 0.0f;
    size_t top_k_ = 0, seed_ = 0;
    std::unique_ptr<FusedDecoder> fused_;
    friend class FusedDecoder;
};

}  // namespace cactus
