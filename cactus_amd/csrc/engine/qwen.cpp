// qwen.cpp -- KV cache and the Qwen3 block over the device graph.
//
//   QwenModel::build_attention/build_mlp/build_transformer_block/forward
//                                   models/model_qwen.cpp:51-172
//   Model::prefill                  engine/engine_model.cpp:170-219
//   Model::decode (greedy)          engine/engine_model.cpp:221-297
//   KVCache::update_from_graph      engine/engine_cache.cpp:101-337 (append)
#include <cmath>
#include <cstring>

#include "cactus_hip.h"
#include "engine.h"
#include "fused.h"

namespace cactus {

// ------------------------------------------------------------------ DevBuf
DevBuf::DevBuf(size_t n) : bytes(n) {
    check_hip(cactus_hip_malloc(&ptr, n ? n : 1), "DevBuf");
}
DevBuf::~DevBuf() {
    if (ptr) cactus_hip_free(ptr);
}
DevBuf& DevBuf::operator=(DevBuf&& o) noexcept {
    if (this != &o) {
        if (ptr) cactus_hip_free(ptr);
        ptr = o.ptr;
        bytes = o.bytes;
        o.ptr = nullptr;
        o.bytes = 0;
    }
    return *this;
}
void DevBuf::upload(const void* host, size_t n, void* stream) {
    check_hip(cactus_hip_memcpy_h2d(ptr, host, n, stream), "upload");
}

// ------------------------------------------------------------------ KVCache
void KVCache::init(size_t layers, size_t max_seq, size_t kv_heads, size_t hd) {
    num_layers = layers;
    max_seq_len = max_seq;
    num_kv_heads = kv_heads;
    head_dim = hd;
    slots = max_seq + 1;
    const size_t codes = slots * kv_heads * hd;
    const size_t scales = slots * kv_heads * groups() * sizeof(float);
    size_t shadow = 0;
    check_hip(cactus_hip_kv_shadow_bytes(slots, kv_heads, hd, &shadow), "kv shadow size");
    k_.clear(); v_.clear(); ks_.clear(); vs_.clear(); vsh_.clear();
    std::vector<cactus_hip_kv_layer> recs(layers);
    for (size_t l = 0; l < layers; l++) {
        k_.emplace_back(codes);
        v_.emplace_back(codes);
        ks_.emplace_back(scales);
        vs_.emplace_back(scales);
        vsh_.emplace_back(shadow);
        recs[l] = {keys_mut(l), values_mut(l), key_scales_mut(l), value_scales_mut(l), value_products(l)};
    }
    table_ = DevBuf(layers * sizeof(cactus_hip_kv_layer));
    table_.upload(recs.data(), table_.bytes, nullptr);
    check_hip(cactus_hip_stream_sync(nullptr), "kv table upload");
    window_size = sink_size = resident = 0;
    reset();
}

// engine_cache.cpp:25-46
void KVCache::set_window(size_t window, size_t sink, void* stream) {
    if (window > max_seq_len)
        throw std::runtime_error("KV window " + std::to_string(window) + " exceeds the cache capacity " +
                                 std::to_string(max_seq_len));
    if (window && sink >= window) throw std::runtime_error("KV sink size must be smaller than the window");
    window_size = window;
    sink_size = sink;
    if (!window) return;
    const std::vector<float> ones(window * num_kv_heads * groups(), 1.0f);
    size_t shadow = 0;
    check_hip(cactus_hip_kv_shadow_bytes(slots, num_kv_heads, head_dim, &shadow), "kv shadow size");
    for (size_t l = 0; l < num_layers; l++) {
        check_hip(cactus_hip_memset(keys_mut(l), 0, window * num_kv_heads * head_dim, stream), "kv window");
        check_hip(cactus_hip_memset(values_mut(l), 0, window * num_kv_heads * head_dim, stream), "kv window");
        check_hip(cactus_hip_memcpy_h2d(key_scales_mut(l), ones.data(), ones.size() * 4, stream), "kv window");
        check_hip(cactus_hip_memcpy_h2d(value_scales_mut(l), ones.data(), ones.size() * 4, stream), "kv window");
        check_hip(cactus_hip_memset(value_products(l), 0, shadow, stream), "kv window");   // products of zeros
    }
    size_t tb = 0;
    check_hip(cactus_hip_kv_shift_temp_bytes(num_layers, window + 1, num_kv_heads, head_dim, &tb), "kv temp size");
    if (temp_.bytes < tb) temp_ = DevBuf(tb);
    check_hip(cactus_hip_stream_sync(stream), "kv window sync");
    resident = window;
}

// quantize rows [row0, row0 + n) of every layer's new K/V into slots
// [at, at + n), with their value products: one launch for all layers
void KVCache::put(const std::vector<const void*>& k, const std::vector<const void*>& v, size_t row0, size_t n,
                  size_t at, void* stream) {
    if (n == 0) return;
    const size_t row = num_kv_heads * head_dim;
    std::vector<const uint16_t*> kr(num_layers), vr(num_layers);
    for (size_t l = 0; l < num_layers; l++) {
        kr[l] = static_cast<const uint16_t*>(k[l]) + row0 * row;
        vr[l] = static_cast<const uint16_t*>(v[l]) + row0 * row;
    }
    check_hip(cactus_hip_kv_append_layers(table_.as<cactus_hip_kv_layer>(), kr.data(), vr.data(), num_layers, n, at,
                                          num_kv_heads, head_dim, GROUP, slots, stream),
              "kv update");
}

void KVCache::shift(size_t dst, size_t src, size_t count, uint32_t* state, uint32_t len, void* stream) {
    check_hip(cactus_hip_kv_window_shift(table_.as<cactus_hip_kv_layer>(), num_layers, num_kv_heads, head_dim,
                                         slots, dst, src, count, temp_.ptr, temp_.bytes, state, len, stream),
              "kv window shift");
}

// engine_cache.cpp:103-330.  All layers take the same branch; the reference
// shifts and appends layer by layer, here every layer shifts first (one
// launch pair), then each appends -- the layers are independent.
void KVCache::update(const std::vector<const void*>& k, const std::vector<const void*>& v, size_t seq,
                     void* stream) {
    if (seq == 0) return;
    const size_t old = current_seq_len, nt = old + seq, W = window_size, S = sink_size;
    const bool sliding = W > 0 && nt > W;
    if (!sliding && nt > max_seq_len)
        throw std::runtime_error("KV cache capacity exceeded (" + std::to_string(nt) + " > " +
                                 std::to_string(max_seq_len) + " tokens; set a window or a larger context)");
    if (old == 0) {
        // the K/V nodes hold all new_total rows (:131-232)
        if (!sliding) {
            put(k, v, 0, nt, 0, stream);
            resident = nt;
        } else {
            // sinks are written only when the storage was not window-sized
            const bool first = resident != W;
            const size_t skip = nt - W;
            if (first) put(k, v, 0, S, 0, stream);
            put(k, v, S + skip, W - S, S, stream);
            resident = W;
        }
    } else if (!sliding) {
        put(k, v, 0, seq, old, stream);
        resident = nt;   // std::vector::resize to the new total (:238-240)
    } else {
        // window full: keep the sinks, slide the rest (:268-327); the
        // reference's size_t arithmetic wraps for a step longer than W - S
        if (seq > W - S)
            throw std::runtime_error("KV update of " + std::to_string(seq) + " tokens into a full window of " +
                                     std::to_string(W) + " with " + std::to_string(S) +
                                     " sinks (the step must not exceed window - sink)");
        const size_t tts = W - S - seq;
        if (tts > 0 && old > S && old - tts > S) shift(S, old - tts, tts, nullptr, 0, stream);
        put(k, v, 0, seq, W - seq, stream);
        resident = W;
    }
    current_seq_len = sliding ? W : nt;
    total_seq_len += seq;
}

void KVCache::put_layer(size_t l, const void* k, const void* v, size_t seq, size_t at, void* stream) {
    if (seq == 0) return;
    const uint16_t* kr = static_cast<const uint16_t*>(k);
    const uint16_t* vr = static_cast<const uint16_t*>(v);
    check_hip(cactus_hip_kv_append_layers(table_.as<cactus_hip_kv_layer>() + l, &kr, &vr, 1, seq, at, num_kv_heads,
                                          head_dim, GROUP, slots, stream),
              "kv update (layer)");
}

void KVCache::appended(size_t seq) {
    if (!fits(seq)) throw std::runtime_error("KV cache: overlapped append beyond the capacity or into a window");
    current_seq_len += seq;
    total_seq_len += seq;
    resident = current_seq_len;
}

void KVCache::slide_after_step(uint32_t* state, void* stream) {
    const size_t W = window_size, S = sink_size;
    if (W == 0 || current_seq_len != W) throw std::runtime_error("slide_after_step: the window is not full");
    // update_from_graph with seq 1 moves [S + 1, W) to [S, W - 1) and appends
    // at W - 1; the step already appended at W, so W - S tokens move
    shift(S, S + 1, W - S, state, (uint32_t)W, stream);
}

// ------------------------------------------------------------------ QwenModel
static DevBuf upload_buf(const void* host, size_t bytes, void* stream) {
    if (!host) throw std::runtime_error("missing weight tensor");
    DevBuf b(bytes);
    b.upload(host, bytes, stream);
    return b;
}

QwenModel::QwenModel(const cactus_qwen_config& cfg, const cactus_qwen_layer_weights* lw,
                     const uint16_t* embedding, const uint16_t* output_norm)
    : cfg_(cfg) {
    if (cfg.hidden % cfg.group_size || cfg.ffn % cfg.group_size ||
        (cfg.heads * cfg.head_dim) % cfg.group_size)
        throw std::runtime_error("group_size must divide every projection's input dimension");
    if (cfg.heads % cfg.kv_heads) throw std::runtime_error("heads must be a multiple of kv_heads");
    check_hip(cactus_hip_stream_create(&stream_), "stream_create");
    graph_ = std::make_unique<CactusGraph>(stream_);
    const size_t H = cfg.hidden, F = cfg.ffn, hd = cfg.head_dim, gs = cfg.group_size;
    const size_t nq = (size_t)cfg.heads * hd, nkv = (size_t)cfg.kv_heads * hd;
    // engine_model.cpp:125-129
    attn_scale_ = 1.0f / std::sqrt(static_cast<float>(hd));

    embedding_ = upload_buf(embedding, (size_t)cfg.vocab * H * 2, stream_);
    out_norm_ = upload_buf(output_norm, H * 2, stream_);
    layers_.resize(cfg.num_layers);
    for (uint32_t l = 0; l < cfg.num_layers; l++) {
        const cactus_qwen_layer_weights& w = lw[l];
        QwenLayer& L = layers_[l];
        L.input_norm = upload_buf(w.input_norm, H * 2, stream_);
        L.post_norm = upload_buf(w.post_norm, H * 2, stream_);
        L.q_norm = upload_buf(w.q_norm, hd * 2, stream_);
        L.k_norm = upload_buf(w.k_norm, hd * 2, stream_);
        L.q_w = upload_buf(w.q_w, nq * H, stream_);
        L.q_s = upload_buf(w.q_s, nq * (H / gs) * 2, stream_);
        L.k_w = upload_buf(w.k_w, nkv * H, stream_);
        L.k_s = upload_buf(w.k_s, nkv * (H / gs) * 2, stream_);
        L.v_w = upload_buf(w.v_w, nkv * H, stream_);
        L.v_s = upload_buf(w.v_s, nkv * (H / gs) * 2, stream_);
        L.o_w = upload_buf(w.o_w, H * nq, stream_);
        L.o_s = upload_buf(w.o_s, H * (nq / gs) * 2, stream_);
        L.gate_w = upload_buf(w.gate_w, F * H / 2, stream_);
        L.gate_s = upload_buf(w.gate_s, F * (H / gs) * 2, stream_);
        L.up_w = upload_buf(w.up_w, F * H / 2, stream_);
        L.up_s = upload_buf(w.up_s, F * (H / gs) * 2, stream_);
        L.down_w = upload_buf(w.down_w, H * F / 2, stream_);
        L.down_s = upload_buf(w.down_s, H * (F / gs) * 2, stream_);
    }
    add_weight_nodes(*graph_);
    cur_ = graph_.get();
    cache_.init(cfg.num_layers, cfg.max_seq, cfg.kv_heads, hd);
    check_hip(cactus_hip_rope_reserve(cfg.max_seq + 1, hd, cfg.rope_theta), "rope_reserve");
    check_hip(cactus_hip_stream_sync(stream_), "init sync");
    k_nodes_.assign(cfg.num_layers, SIZE_MAX);
    v_nodes_.assign(cfg.num_layers, SIZE_MAX);
    att_nodes_.assign(cfg.num_layers, SIZE_MAX);
}

// QwenModel::load_weights_to_graph (model_qwen.cpp:17-49): the weights as
// external INPUT nodes.  A fresh graph gets the same node ids in the same
// order, so the layers' ids hold for graph_ and the prefill graphs alike.
void QwenModel::add_weight_nodes(CactusGraph& g) {
    const cactus_qwen_config& cfg = cfg_;
    const size_t H = cfg.hidden, F = cfg.ffn, hd = cfg.head_dim, gs = cfg.group_size;
    const size_t nq = (size_t)cfg.heads * hd, nkv = (size_t)cfg.kv_heads * hd;
    const bool first = &g == graph_.get();
    auto weight = [&](size_t& id_out, const std::vector<size_t>& shape, Precision p, void* dev) {
        const size_t id = g.input(shape, p);
        g.set_external_input(id, dev, p);
        if (first) id_out = id;
        else if (id != id_out) throw std::runtime_error("second prefill graph: weight node ids differ");
        return id;
    };
    weight(n_embedding_, {cfg.vocab, H}, Precision::FP16, embedding_.ptr);
    weight(n_out_norm_, {H}, Precision::FP16, out_norm_.ptr);
    for (uint32_t l = 0; l < cfg.num_layers; l++) {
        QwenLayer& L = layers_[l];
        weight(L.n_input_norm, {H}, Precision::FP16, L.input_norm.ptr);
        weight(L.n_post_norm, {H}, Precision::FP16, L.post_norm.ptr);
        weight(L.n_q_norm, {hd}, Precision::FP16, L.q_norm.ptr);
        weight(L.n_k_norm, {hd}, Precision::FP16, L.k_norm.ptr);
        g.set_grouped_scales(weight(L.n_q, {nq, H}, Precision::INT8, L.q_w.ptr), gs, H / gs, L.q_s.ptr);
        g.set_grouped_scales(weight(L.n_k, {nkv, H}, Precision::INT8, L.k_w.ptr), gs, H / gs, L.k_s.ptr);
        g.set_grouped_scales(weight(L.n_v, {nkv, H}, Precision::INT8, L.v_w.ptr), gs, H / gs, L.v_s.ptr);
        g.set_grouped_scales(weight(L.n_o, {H, nq}, Precision::INT8, L.o_w.ptr), gs, nq / gs, L.o_s.ptr);
        // packed INT4 MLP weights keep their shape in elements
        const size_t ng = weight(L.n_gate, {F, H}, Precision::INT8, L.gate_w.ptr);
        g.set_grouped_scales(ng, gs, H / gs, L.gate_s.ptr);
        g.set_packed_int4(ng, L.gate_w.ptr, F * H / 2);
        const size_t nu = weight(L.n_up, {F, H}, Precision::INT8, L.up_w.ptr);
        g.set_grouped_scales(nu, gs, H / gs, L.up_s.ptr);
        g.set_packed_int4(nu, L.up_w.ptr, F * H / 2);
        const size_t nd = weight(L.n_down, {H, F}, Precision::INT8, L.down_w.ptr);
        g.set_grouped_scales(nd, gs, F / gs, L.down_s.ptr);
        g.set_packed_int4(nd, L.down_w.ptr, H * F / 2);
    }
}

QwenModel::~QwenModel() {
    cactus_hip_stream_sync(stream_);
    for (void* st : pf_streams_) cactus_hip_stream_sync(st);
    fused_.reset();
    graph_.reset();
    pf_graphs_.clear();
    layers_.clear();
    for (auto& evs : kv_ev_)
        for (void* e : evs) cactus_hip_event_destroy(e);
    for (void* e : join_ev_) cactus_hip_event_destroy(e);
    for (void* st : pf_streams_) cactus_hip_stream_destroy(st);
    cactus_hip_stream_destroy(stream_);
}

void QwenModel::reset() {
    cache_.reset();
    graph_->soft_reset();
    last_hidden_ = last_logits_ = SIZE_MAX;
    fused_logits_ = false;
}

const void* QwenModel::last_logits_data() const {
    if (last_logits_ != SIZE_MAX) return graph_->get_output_buffer(last_logits_).data;
    if (fused_logits_ && fused_) return fused_->logits().ptr;
    return nullptr;
}

// Input of matmuls that share it: at prefill sizes its per-row INT8
// quantization (graph_ops_nn.cpp:35-66, the same codes and scales every
// matmul node would compute for itself) runs once as a node of its own;
// a decode-sized GEMV quantizes inside its kernel at no extra launch.
size_t QwenModel::shared_matmul_input(size_t x) {
    CactusGraph& g = *cur_;
    const BufferDesc& b = g.get_output_buffer(x);
    if (b.precision == Precision::INT8) return x;   // already codes with row scales
    return b.shape[0] >= 32 ? g.quantize_activations(x) : x;
}

// The RMSNorm in front of q/k/v and of gate/up feeds only those matmuls: at
// prefill sizes it is one node with their row quantization.
size_t QwenModel::norm_for_matmuls(size_t h, size_t weight) {
    CactusGraph& g = *cur_;
    if (g.get_output_buffer(h).shape[0] >= 32) return g.rms_norm_quantize(h, weight, cfg_.eps);
    return g.rms_norm(h, weight, cfg_.eps);
}

// model_qwen.cpp:51-106
size_t QwenModel::build_attention(size_t x, uint32_t l, size_t pos, size_t residual) {
    CactusGraph& g = *cur_;
    const QwenLayer& L = layers_[l];
    const size_t hd = cfg_.head_dim, nh = cfg_.heads, nkv = cfg_.kv_heads;
    const size_t xq = shared_matmul_input(x);
    size_t q = g.matmul(xq, L.n_q, true);
    size_t k = g.matmul(xq, L.n_k, true);
    size_t v = g.matmul(xq, L.n_v, true);
    const size_t S = g.get_output_buffer(q).shape[0];
    size_t q4, k4;
    size_t v4 = g.reshape(v, {1, S, nkv, hd});
    if (cfg_.rope_theta > 0) {
        // the head RMSNorm and RoPE of q and of k, one node each (adjacent:
        // the executor runs the pair as one launch)
        const size_t q_in = g.reshape(q, {1, S, nh, hd}), k_in = g.reshape(k, {1, S, nkv, hd});
        q4 = g.rms_norm_rope(q_in, L.n_q_norm, cfg_.eps, cfg_.rope_theta, pos);
        k4 = g.rms_norm_rope(k_in, L.n_k_norm, cfg_.eps, cfg_.rope_theta, pos);
    } else {
        q = g.reshape(q, {S * nh, hd});
        q = g.rms_norm(q, L.n_q_norm, cfg_.eps);
        k = g.reshape(k, {S * nkv, hd});
        k = g.rms_norm(k, L.n_k_norm, cfg_.eps);
        q4 = g.reshape(q, {1, S, nh, hd});
        k4 = g.reshape(k, {1, S, nkv, hd});
    }
    k_nodes_[l] = k4;
    v_nodes_[l] = v4;
    size_t att;
    if (!cache_.is_empty())
        att = g.attention_int8_hybrid(q4, k4, v4, attn_scale_, pos, cache_.keys(l), cache_.values(l),
                                      cache_.key_scales(l), cache_.value_scales(l),
                                      cache_.current_seq_len, nkv, hd);
    else
        att = g.attention(q4, k4, v4, attn_scale_, pos);
    att_nodes_[l] = att;
    att = g.reshape(att, {S, hd * nh});
    if (residual != NO_RESIDUAL) return g.matmul_add(att, L.n_o, residual);
    return g.matmul(att, L.n_o, true);
}

// model_qwen.cpp:109-117
size_t QwenModel::build_mlp(size_t x, uint32_t l, size_t residual) {
    CactusGraph& g = *cur_;
    const QwenLayer& L = layers_[l];
    const size_t xq = shared_matmul_input(x);
    size_t gate = g.matmul(xq, L.n_gate, true);
    size_t up = g.matmul(xq, L.n_up, true);
    // at prefill sizes the SwiGLU product is one node with the down
    // projection's row quantization
    if (g.get_output_buffer(gate).shape[0] >= 32) {
        const size_t q = g.silu_mul_quantize(gate, up);
        if (residual != NO_RESIDUAL) return g.matmul_add(q, L.n_down, residual);
        return g.matmul(q, L.n_down, true);
    }
    size_t act = g.silu(gate);
    size_t m = g.multiply(act, up);
    if (residual != NO_RESIDUAL) return g.matmul_add(m, L.n_down, residual);
    return g.matmul(m, L.n_down, true);
}

// model_qwen.cpp:120-129
size_t QwenModel::build_block(size_t h, uint32_t l, size_t pos) {
    CactusGraph& g = *cur_;
    const QwenLayer& L = layers_[l];
    size_t x = norm_for_matmuls(h, L.n_input_norm);
    // at prefill sizes the residual adds ride on the o-proj and down matmuls
    const bool fuse = g.get_output_buffer(h).shape[0] >= 32;
    size_t h1 = build_attention(x, l, pos, fuse ? h : NO_RESIDUAL);
    if (!fuse) h1 = g.add(h, h1);
    size_t x2 = norm_for_matmuls(h1, L.n_post_norm);
    size_t out = build_mlp(x2, l, fuse ? h1 : NO_RESIDUAL);
    return fuse ? out : g.add(h1, out);
}

void QwenModel::check_token_ids(const std::vector<uint32_t>& tokens) const {
    for (uint32_t t : tokens)
        if (t >= cfg_.vocab)
            throw std::runtime_error("Embedding index out of bounds: " + std::to_string(t) + " >= " +
                                     std::to_string(cfg_.vocab));
}

// model_qwen.cpp:132-172 (use_cache = true)
size_t QwenModel::forward(const std::vector<uint32_t>& tokens) {
    if (tokens.empty()) throw std::runtime_error("Token sequence cannot be empty");
    CactusGraph& g = *cur_;
    g.soft_reset();
    const size_t S = tokens.size();
    const size_t pos = cache_.total_seq_len;
    // the reference's out-of-range check (graph_ops_tensor.cpp:256-263), on
    // the host ids before anything is launched
    check_token_ids(tokens);
    size_t ids = g.input({S}, Precision::FP32);
    size_t h = g.embedding_checked_ids(n_embedding_, ids);
    std::vector<float> idf(S);
    for (size_t i = 0; i < S; i++) idf[i] = static_cast<float>(tokens[i]);
    g.set_input(ids, idf.data(), Precision::FP32);
    for (uint32_t l = 0; l < cfg_.num_layers; l++) h = build_block(h, l, pos);
    return g.rms_norm(h, n_out_norm_, cfg_.eps);
}

// engine_model.cpp:317-321 -> engine_cache.cpp:234-267 (append branch)
void QwenModel::update_kv_cache(size_t seq) {
    std::vector<const void*> k(cfg_.num_layers), v(cfg_.num_layers);
    for (uint32_t l = 0; l < cfg_.num_layers; l++) {
        k[l] = graph_->get_output_buffer(k_nodes_[l]).data;
        v[l] = graph_->get_output_buffer(v_nodes_[l]).data;
    }
    cache_.update(k, v, seq, stream_);
}

// KVCache::set_window_size through the model (engine_model.cpp:136-146)
void QwenModel::set_kv_window(size_t window, size_t sink) {
    check_hip(cactus_hip_stream_sync(stream_), "sync");
    cache_.set_window(window, sink, stream_);
}

// engine_model.cpp:170-219
void QwenModel::prefill(const std::vector<uint32_t>& tokens) {
    if (tokens.empty()) return;
    // every id is checked before the first chunk is queued: a bad id in a
    // later chunk must not leave earlier chunks' KV appends in flight on the
    // overlapped streams (the reference raises the same error from its
    // embedding node, graph_ops_tensor.cpp:256-263)
    check_token_ids(tokens);
    const size_t chunk = cfg_.prefill_chunk ? cfg_.prefill_chunk : 256;
    if (tokens.size() > chunk && cache_.fits(tokens.size())) {
        prefill_overlapped(tokens, chunk);
        return;
    }
    // the graph is rebuilt per chunk: no logits node survives a prefill
    last_logits_ = SIZE_MAX;
    fused_logits_ = false;
    auto process = [&](size_t b, size_t e) {
        std::vector<uint32_t> c(tokens.begin() + b, tokens.begin() + e);
        last_hidden_ = forward(c);
        graph_->execute();
        update_kv_cache(c.size());
    };
    if (tokens.size() <= chunk) {
        process(0, tokens.size());
        return;
    }
    const size_t full = (tokens.size() - 1) / chunk;
    for (size_t i = 0; i < full; i++) process(i * chunk, (i + 1) * chunk);
    process(full * chunk, tokens.size());
}

// The chunks of engine_model.cpp:170-219 (the same boundaries and the
// same nodes as prefill's serial loop) with consecutive chunks overlapping
// on several streams.  A chunk reads the earlier chunks' KV rows only in its
// attention nodes, so chunk c appends each layer's rows right after that
// layer's k/v nodes (one launch per layer instead of one per chunk, the same
// bytes); before its attention node of the layer it waits for chunk c - 1's
// event of the layer and then records its own, which therefore follows the
// appends of chunks 0..c of that layer.  Every kernel sees the inputs of the
// serial order: the results are bit-identical to it.
void QwenModel::prefill_overlapped(const std::vector<uint32_t>& tokens, size_t chunk) {
    const size_t L = cfg_.num_layers;
    constexpr int NS = kPrefillStreams;
    if (pf_graphs_.empty()) {
        for (int p = 1; p < NS; p++) {
            void* st = nullptr;
            check_hip(cactus_hip_stream_create(&st), "stream_create");
            pf_streams_.push_back(st);
            pf_graphs_.push_back(std::make_unique<CactusGraph>(st));
            add_weight_nodes(*pf_graphs_.back());
        }
        kv_ev_.assign(NS, std::vector<void*>(L, nullptr));
        for (auto& evs : kv_ev_)
            for (void*& e : evs) check_hip(cactus_hip_event_create(&e), "event_create");
        join_ev_.assign(NS, nullptr);
        for (void*& e : join_ev_) check_hip(cactus_hip_event_create(&e), "event_create");
    }
    auto graph_of = [&](int p) -> CactusGraph& { return p == 0 ? *graph_ : *pf_graphs_[p - 1]; };
    auto stream_of = [&](int p) { return p == 0 ? stream_ : pf_streams_[p - 1]; };
    // the other streams start after everything already queued on stream_
    // (the cache contents the first chunk attends to)
    check_hip(cactus_hip_event_record(join_ev_[0], stream_), "event_record");
    for (int p = 1; p < NS; p++) {
        graph_of(p).set_attention_tolerance(attention_mode_ == 1);
        check_hip(cactus_hip_stream_wait_event(stream_of(p), join_ev_[0]), "stream_wait_event");
    }
    last_logits_ = SIZE_MAX;
    fused_logits_ = false;
    std::vector<std::pair<size_t, size_t>> bounds;
    const size_t full = (tokens.size() - 1) / chunk;
    for (size_t i = 0; i < full; i++) bounds.emplace_back(i * chunk, (i + 1) * chunk);
    bounds.emplace_back(full * chunk, tokens.size());
    const size_t n = bounds.size();
    try {
        for (size_t i = 0; i < n; i++) {
            const int par = (int)((n - 1 - i) % NS), prev = (par + 1) % NS;
            CactusGraph& g = graph_of(par);
            void* st = stream_of(par);
            cur_ = &g;
            const std::vector<uint32_t> c(tokens.begin() + bounds[i].first, tokens.begin() + bounds[i].second);
            last_hidden_ = forward(c);
            const size_t at = cache_.current_seq_len, seq = c.size();
            for (size_t l = 0; l < L; l++) {
                const size_t kn = k_nodes_[l], vn = v_nodes_[l];
                void* ev = kv_ev_[par][l];
                void* pe = i > 0 ? kv_ev_[prev][l] : nullptr;
                g.after_node(kn, [this, &g, l, kn, vn, seq, at, st] {
                    cache_.put_layer(l, g.get_output_buffer(kn).data, g.get_output_buffer(vn).data, seq, at, st);
                });
                // the layer's event is recorded after this chunk's own wait
                // for the previous chunk's event, so it covers the appends of
                // every earlier chunk, not only this one's: a later chunk's
                // attention reads all of them
                g.before_node(att_nodes_[l], [st, pe, ev] {
                    if (pe) check_hip(cactus_hip_stream_wait_event(st, pe), "stream_wait_event");
                    check_hip(cactus_hip_event_record(ev, st), "event_record");
                });
            }
            g.execute();
            cache_.appended(seq);
        }
    } catch (...) {
        cur_ = graph_.get();
        // whatever the other streams queued (KV appends included) stays
        // ordered before later work on stream_; errors of the join itself
        // are dropped so the original exception propagates
        for (int p = 1; p < NS; p++) {
            if (cactus_hip_event_record(join_ev_[p], stream_of(p)) == 0)
                (void)cactus_hip_stream_wait_event(stream_, join_ev_[p]);
            else
                (void)cactus_hip_stream_sync(stream_of(p));
        }
        throw;
    }
    cur_ = graph_.get();
    // later work on stream_ (decode, reset) follows all of the other streams'
    for (int p = 1; p < NS; p++) {
        check_hip(cactus_hip_event_record(join_ev_[p], stream_of(p)), "event_record");
        check_hip(cactus_hip_stream_wait_event(stream_, join_ev_[p]), "stream_wait_event");
    }
}

// engine_model.cpp:221-297, greedy
void QwenModel::set_sampling(float temperature, float top_p, size_t top_k, size_t seed) {
    if (!(temperature >= 0.0f)) throw std::runtime_error("temperature must be >= 0");
    temperature_ = temperature;
    top_p_ = top_p;
    top_k_ = top_k;
    seed_ = seed;
}

uint32_t QwenModel::decode(uint32_t token) {
    // the fused step ends in the greedy LM head; other settings run the
    // node graph's sample node (its draw is made on the host per step)
    if (decode_mode_ == 1 && fused_ && greedy()) {
        return fused_decode(*this, *fused_, token);
    }
    CactusGraph& g = *graph_;
    fused_logits_ = false;
    size_t fin = forward({token});
    last_hidden_ = fin;
    size_t last = g.index(fin, 0, 0);
    last = g.reshape(last, {1, cfg_.hidden});
    last_logits_ = g.matmul(last, n_embedding_, true);
    size_t tok = g.sample(last_logits_, temperature_, top_p_, top_k_, seed_);
    g.execute();
    update_kv_cache(1);
    uint32_t id = 0;
    std::memcpy(&id, g.get_output(tok), 4);
    return id;
}

}  // namespace cactus
