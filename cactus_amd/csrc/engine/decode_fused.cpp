// decode_fused.cpp -- fused decode path of QwenModel (decode mode 1).
//
// Per layer: qkv (RMSNorm + INT8 GEMV x3), attn_prep (q/k RMSNorm, RoPE,
// INT8 KV append) and attention (scores + value chains) -- for head_dim 64
// or 128 with one or two query heads per KV head, the prep runs inside the
// score kernel --, o-proj + residual, mlp_up (RMSNorm + INT4 gate/up +
// SiLU*mul), down + residual.  Then the LM
// head with the fused argmax advances the device step state.  Bit-identical
// to decode mode 0 (the node-by-node graph).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <stdexcept>

#include "cactus_hip.h"
#include "fused.h"

namespace cactus {

FusedDecoder::FusedDecoder(QwenModel& m) : m_(m) {
    const cactus_qwen_config& c = m.config();
    const size_t H = c.hidden, F = c.ffn, hd = c.head_dim;
    const size_t nq = (size_t)c.heads * hd, nkv = (size_t)c.kv_heads * hd;
    state_ = DevBuf(16);
    h_ = DevBuf(H * 2);
    q_raw_ = DevBuf(nq * 2);
    k_raw_ = DevBuf(nkv * 2);
    v_raw_ = DevBuf(nkv * 2);
    q_rot_ = DevBuf(nq * 2);
    k_rot_ = DevBuf(nkv * 2);
    attn_ = DevBuf(nq * 2);
    mlp_ = DevBuf(F * 2);
    max_steps_ = c.max_seq + 1;
    tokens_ = DevBuf(max_steps_ * 4);
    // covers the scratch contracts of cactus_hip_decode_lm_head (>= 256) and
    // cactus_hip_decode_lm_head_tiled (>= 1024 + 8 * ceil(vocab / 640))
    const size_t blocks = (c.vocab + 127) / 128;
    lm_scratch_ = DevBuf(1024 + 8 * blocks);
    logits_ = DevBuf((size_t)c.vocab * 2);
    check_hip(cactus_hip_memset(lm_scratch_.ptr, 0, lm_scratch_.bytes, m.stream()), "memset");
    // the LM head reads the embedding through its 64-row tiles (a second
    // copy, built once: the weights do not change after loading)
    size_t tile_bytes = 0;
    check_hip(cactus_hip_lm_tiles_bytes(H, c.vocab, &tile_bytes), "lm_tiles_bytes");
    lm_tiles_ = DevBuf(tile_bytes);
    check_hip(cactus_hip_lm_tiles_build(m.embedding().as<uint16_t>(), H, c.vocab, lm_tiles_.as<uint16_t>(), m.stream()),
              "lm_tiles_build");
    // split-K attention workspace (tolerance mode): counters zeroed once
    attn_ws_ = DevBuf(cactus_hip_decode_attention_fast_workspace(c.heads, c.kv_heads, hd, m.cache().slots));
    check_hip(cactus_hip_memset(attn_ws_.ptr, 0, attn_ws_.bytes, m.stream()), "memset");
    // the decode entry points ask for max_cache + 1 positions, max_cache
    // being the cache's slot count (context + 1)
    rope_pos_ = m.cache().slots + 1;
    check_hip(cactus_hip_rope_reserve(rope_pos_, hd, c.rope_theta), "rope_reserve");
    check_hip(cactus_hip_stream_sync(m.stream()), "sync");
}

void FusedDecoder::reserve(size_t positions, size_t steps) {
    const cactus_qwen_config& c = m_.config();
    bool grown = false;
    if (positions + 1 > rope_pos_ || steps > max_steps_) {
        // nothing queued may still read the buffers being replaced
        check_hip(cactus_hip_stream_sync(m_.stream()), "sync");
    }
    if (positions + 1 > rope_pos_) {
        rope_pos_ = std::max(positions + 1, 2 * rope_pos_);
        check_hip(cactus_hip_rope_reserve(rope_pos_, c.head_dim, c.rope_theta), "rope_reserve");
        grown = true;
    }
    if (steps > max_steps_) {
        max_steps_ = std::max(steps, 2 * max_steps_);
        tokens_ = DevBuf(max_steps_ * 4);
        grown = true;
    }
    if (grown && graph_) {
        cactus_hip_graph_destroy(graph_);
        graph_ = nullptr;
    }
}

FusedDecoder::~FusedDecoder() {
    if (graph_) cactus_hip_graph_destroy(graph_);
}

void FusedDecoder::invalidate() {
    check_hip(cactus_hip_stream_sync(m_.stream()), "sync");
    if (graph_) cactus_hip_graph_destroy(graph_);
    graph_ = nullptr;
}

void FusedDecoder::enqueue() {
    const cactus_qwen_config& c = m_.config();
    void* st = m_.stream();
    const size_t H = c.hidden, F = c.ffn, hd = c.head_dim, gs = c.group_size;
    const size_t nq = (size_t)c.heads * hd, nkv = (size_t)c.kv_heads * hd;
    uint32_t* state = state_.as<uint32_t>();
    uint16_t* h = h_.as<uint16_t>();
    KVCache& kv = m_.cache();
    auto u16 = [](const DevBuf& b) { return b.as<uint16_t>(); };
    // head preparation inside the attention's score kernel where the shape
    // allows (one kernel fewer per layer)
    const size_t gqa = c.heads / c.kv_heads;
    const bool fused_prep = (hd == 64 || hd == 128) && (gqa == 1 || gqa == 2);
    const bool tolerance = m_.attention_mode() == 1 && (hd == 64 || hd == 128) && (gqa == 1 || gqa == 2 || gqa == 4);
    // h holds the step's input row: embedded by run() for the first step,
    // then by the LM head of the step before
    for (uint32_t l = 0; l < c.num_layers; l++) {
        const QwenLayer& L = m_.layer(l);
        check_hip(cactus_hip_decode_qkv(h, u16(L.input_norm), c.eps, H, gs, L.q_w.as<int8_t>(), u16(L.q_s),
                                        q_raw_.as<uint16_t>(), nq, L.k_w.as<int8_t>(), u16(L.k_s),
                                        k_raw_.as<uint16_t>(), nkv, L.v_w.as<int8_t>(), u16(L.v_s),
                                        v_raw_.as<uint16_t>(), nkv, st),
                  "decode_qkv");
        if (tolerance) {
            check_hip(cactus_hip_decode_prep_attention_fast(
                          q_raw_.as<uint16_t>(), k_raw_.as<uint16_t>(), v_raw_.as<uint16_t>(), u16(L.q_norm),
                          u16(L.k_norm), c.eps, c.heads, c.kv_heads, hd, c.rope_theta, state, kv.keys_mut(l),
                          kv.values_mut(l), kv.key_scales_mut(l), kv.value_scales_mut(l), kv.slots,
                          kv.value_products(l), m_.attention_scale(), attn_.as<uint16_t>(), attn_ws_.ptr,
                          attn_ws_.bytes, st),
                      "decode_prep_attention_fast");
        } else if (fused_prep) {
            check_hip(cactus_hip_decode_prep_attention(
                          q_raw_.as<uint16_t>(), k_raw_.as<uint16_t>(), v_raw_.as<uint16_t>(), u16(L.q_norm),
                          u16(L.k_norm), c.eps, c.heads, c.kv_heads, hd, c.rope_theta, state, kv.keys_mut(l),
                          kv.values_mut(l), kv.key_scales_mut(l), kv.value_scales_mut(l), kv.slots,
                          kv.value_products(l), m_.attention_scale(), attn_.as<uint16_t>(), st),
                      "decode_prep_attention");
        } else {
            check_hip(cactus_hip_decode_attn_prep(q_raw_.as<uint16_t>(), k_raw_.as<uint16_t>(),
                                                  v_raw_.as<uint16_t>(), u16(L.q_norm), u16(L.k_norm), c.eps,
                                                  c.heads, c.kv_heads, hd, c.rope_theta, state,
                                                  q_rot_.as<uint16_t>(), k_rot_.as<uint16_t>(), kv.keys_mut(l),
                                                  kv.values_mut(l), kv.key_scales_mut(l), kv.value_scales_mut(l),
                                                  kv.slots, kv.value_products(l), st),
                      "decode_attn_prep");
            check_hip(cactus_hip_decode_attention(q_rot_.as<uint16_t>(), kv.keys(l), kv.values(l),
                                                  kv.key_scales(l), kv.value_scales(l), k_rot_.as<uint16_t>(),
                                                  v_raw_.as<uint16_t>(), attn_.as<uint16_t>(), c.heads,
                                                  c.kv_heads, hd, m_.attention_scale(), state, kv.slots,
                                                  kv.value_products(l), st),
                      "decode_attention");
        }
        check_hip(cactus_hip_decode_matmul_residual(attn_.as<uint16_t>(), nq, gs, L.o_w.ptr, u16(L.o_s), H, 0, h,
                                                    st),
                  "decode_o_proj");
        check_hip(cactus_hip_decode_mlp_up(h, u16(L.post_norm), c.eps, H, gs, L.gate_w.as<uint8_t>(),
                                           u16(L.gate_s), L.up_w.as<uint8_t>(), u16(L.up_s), F,
                                           mlp_.as<uint16_t>(), st),
                  "decode_mlp_up");
        check_hip(cactus_hip_decode_matmul_residual(mlp_.as<uint16_t>(), F, gs, L.down_w.ptr, u16(L.down_s), H, 1,
                                                    h, st),
                  "decode_down");
    }
    // the LM head's last workgroup also embeds the token it picks into h
    check_hip(cactus_hip_decode_lm_head_tiled_embed(h, u16(m_.output_norm()), c.eps, lm_tiles_.as<uint16_t>(),
                                                    u16(m_.embedding()), H, c.vocab, state, tokens_.as<uint32_t>(),
                                                    max_steps_, logits_.as<uint16_t>(), h, lm_scratch_.ptr,
                                                    lm_scratch_.bytes, st),
              "decode_lm_head");
}

void FusedDecoder::set_state(uint32_t token) {
    const KVCache& kv = m_.cache();
    const uint32_t s[4] = {token, (uint32_t)kv.total_seq_len, (uint32_t)kv.current_seq_len, 0u};
    check_hip(cactus_hip_memcpy_h2d(state_.ptr, s, sizeof(s), m_.stream()), "state upload");
}

void FusedDecoder::ensure_graph() {
    if (graph_) return;
    void* st = m_.stream();
    check_hip(cactus_hip_graph_capture_begin(st), "capture begin");
    try {
        enqueue();
    } catch (...) {
        void* g = nullptr;
        cactus_hip_graph_capture_end(st, &g);
        if (g) cactus_hip_graph_destroy(g);
        throw;
    }
    check_hip(cactus_hip_graph_capture_end(st, &graph_), "capture end");
}

void FusedDecoder::run(uint32_t token, size_t n, uint32_t* out) {
    if (n == 0) return;
    KVCache& kv = m_.cache();
    if (kv.window_size == 0 && kv.current_seq_len + n > kv.max_seq_len)
        throw std::runtime_error("KV cache capacity exceeded (" + std::to_string(kv.current_seq_len + n) + " > " +
                                 std::to_string(kv.max_seq_len) + " tokens; set a window or a larger context)");
    reserve(kv.total_seq_len + n, n);
    set_state(token);
    check_hip(cactus_hip_decode_embed(m_.embedding().as<uint16_t>(), state_.as<uint32_t>(), h_.as<uint16_t>(),
                                      m_.config().hidden, m_.config().vocab, m_.stream()),
              "decode_embed");
    // the fused step keeps the last step's logits (in logits_), not the
    // final hidden state
    m_.last_hidden_ = SIZE_MAX;
    m_.last_logits_ = SIZE_MAX;
    m_.fused_logits_ = false;
    // CACTUS_DECODE_EAGER=1 enqueues the step's kernels directly instead of
    // replaying the graph (same kernels and results; for kernel tracers)
    static const bool eager = [] {
        const char* e = std::getenv("CACTUS_DECODE_EAGER");
        return e && e[0] == '1';
    }();
    for (size_t done = 0; done < n; done++) {
        // into a full window the step attends over the whole window plus its
        // own token and appends at slot `window`; the slide follows
        // (engine_cache.cpp:268-327 for seq_len 1)
        const bool slides = kv.step_slides();
        if (!warmed_ || eager) {
            // the first step runs eagerly: it allocates the library's
            // scratch buffers outside of any capture
            enqueue();
            warmed_ = true;
        } else {
            ensure_graph();
            check_hip(cactus_hip_graph_launch(graph_, m_.stream()), "graph launch");
        }
        if (slides) kv.slide_after_step(state_.as<uint32_t>(), m_.stream());
        else kv.current_seq_len += 1;
        kv.total_seq_len += 1;
        if (slides) kv.resident = kv.window_size;
        else kv.resident = std::max(kv.resident, kv.current_seq_len);
    }
    check_hip(cactus_hip_memcpy_d2h(out, tokens_.ptr, n * 4, m_.stream()), "tokens");
    m_.fused_logits_ = true;
}

uint32_t FusedDecoder::step(uint32_t token) {
    uint32_t t = 0;
    run(token, 1, &t);
    return t;
}

uint32_t fused_decode(QwenModel& m, FusedDecoder& f, uint32_t token) {
    (void)m;
    return f.step(token);
}

void QwenModel::set_attention_mode(int mode) {
    if (mode != 0 && mode != 1) throw std::runtime_error("attention mode must be 0 (exact) or 1 (tolerance)");
    check_hip(cactus_hip_stream_sync(stream_), "sync");
    attention_mode_ = mode;
    graph_->set_attention_tolerance(mode == 1);
    if (fused_) fused_->invalidate();
}

void QwenModel::set_decode_mode(int mode) {
    if (mode != 0 && mode != 1) throw std::runtime_error("decode mode must be 0 or 1");
    check_hip(cactus_hip_stream_sync(stream_), "sync");
    if (mode == 1 && !fused_) fused_ = std::make_unique<FusedDecoder>(*this);
    decode_mode_ = mode;
}

void QwenModel::decode_many(uint32_t token, size_t n, uint32_t* out) {
    if (decode_mode_ == 1 && fused_ && greedy()) {
        fused_->run(token, n, out);
        return;
    }
    for (size_t i = 0; i < n; i++) {
        token = decode(token);
        out[i] = token;
    }
}

}  // namespace cactus
