/*
 * qwen_oracle.c -- CPU restatement of the Qwen3 block and the engine's
 * prefill/decode flow, composed from the kernel restatements in
 * cactus_oracle.c (test infrastructure; see cactus_oracle.h).
 *
 *   QwenModel::build_attention / build_mlp / build_transformer_block /
 *   forward                       models/model_qwen.cpp:51-172
 *   Model::prefill                engine/engine_model.cpp:170-219
 *   Model::decode (greedy)        engine/engine_model.cpp:221-297
 *   KVCache update (INT8)         engine/engine_cache.cpp:103-330 (kv_oracle.c)
 *
 * The graph's reshape nodes are copies in the reference and views here;
 * neither changes a value.  Positions (RoPE and the attention's causal
 * offset) are total_seq_len, the cache length current_seq_len
 * (model_qwen.cpp:85-99, :141-145); with a sliding window the two differ.
 */
#include "cactus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define KV_GROUP 128

struct orc_qwen {
    orc_qwen_config cfg;
    orc_qwen_layer* layers;
    const uint16_t* embedding;
    const uint16_t* out_norm;
    float attn_scale;
    /* KV cache, INT8 per token/head/128-dim group */
    orc_kv* kv;
    /* final hidden state of the last forward */
    uint16_t* last_hidden; size_t last_rows;
};

orc_qwen* orc_qwen_create(const orc_qwen_config* cfg, const orc_qwen_layer* layers,
                          const uint16_t* embedding, const uint16_t* output_norm) {
    orc_qwen* m = (orc_qwen*)calloc(1, sizeof(orc_qwen));
    m->cfg = *cfg;
    m->layers = (orc_qwen_layer*)malloc(sizeof(orc_qwen_layer) * cfg->num_layers);
    memcpy(m->layers, layers, sizeof(orc_qwen_layer) * cfg->num_layers);
    m->embedding = embedding;
    m->out_norm = output_norm;
    /* engine_model.cpp:125-129 */
    m->attn_scale = 1.0f / sqrtf((float)cfg->head_dim);
    m->kv = orc_kv_create(cfg->num_layers, cfg->max_seq, cfg->kv_heads, cfg->head_dim);
    return m;
}

void orc_qwen_destroy(orc_qwen* m) {
    if (!m) return;
    orc_kv_destroy(m->kv);
    free(m->layers);
    free(m->last_hidden);
    free(m);
}

void orc_qwen_reset(orc_qwen* m) { orc_kv_reset(m->kv); }
size_t orc_qwen_cache_len(const orc_qwen* m) { return orc_kv_len(m->kv); }
int orc_qwen_set_window(orc_qwen* m, size_t window, size_t sink) { return orc_kv_set_window(m->kv, window, sink); }

void orc_qwen_kv(const orc_qwen* m, size_t l, const int8_t** k, const int8_t** v,
                 const float** ks, const float** vs) {
    orc_kv_layer(m->kv, l, k, v, ks, vs);
}

const uint16_t* orc_qwen_last_hidden(const orc_qwen* m, size_t* rows) {
    if (rows) *rows = m->last_rows;
    return m->last_hidden;
}

/* matmul node on FP16 activations: per-row quantization then the grouped
 * kernel (graph_ops_nn.cpp:129-231) */
static void mm_int8(const uint16_t* x, size_t S, size_t K, const int8_t* w, const uint16_t* s,
                    size_t N, size_t gs, uint16_t* y, int8_t* qbuf, float* sbuf) {
    orc_quantize_activations(x, qbuf, sbuf, S, K);
    orc_matmul_int8(qbuf, sbuf, w, s, y, S, K, N, gs);
}
static void mm_int4(const uint16_t* x, size_t S, size_t K, const uint8_t* w, const uint16_t* s,
                    size_t N, size_t gs, uint16_t* y, int8_t* qbuf, float* sbuf) {
    orc_quantize_activations(x, qbuf, sbuf, S, K);
    orc_matmul_int4(qbuf, sbuf, w, s, y, S, K, N, gs);
}

/* One forward over S tokens with use_cache=true (model_qwen.cpp:132-172)
 * followed by the KV-cache append (engine_cache.cpp:234-267). */
static int qwen_forward(orc_qwen* m, const uint32_t* tok, size_t S) {
    const orc_qwen_config* c = &m->cfg;
    const size_t H = c->hidden, F = c->ffn, hd = c->head_dim;
    const size_t nq = (size_t)c->heads * hd, nkv = (size_t)c->kv_heads * hd;
    const size_t gs = c->group_size;
    const size_t pos = orc_kv_total(m->kv);
    const size_t cache_len = orc_kv_len(m->kv);

    size_t maxK = H > F ? H : F;
    if (nq > maxK) maxK = nq;
    uint16_t* h = (uint16_t*)malloc(2 * S * H);
    uint16_t* x = (uint16_t*)malloc(2 * S * H);
    uint16_t* q = (uint16_t*)malloc(2 * S * nq);
    uint16_t* q2 = (uint16_t*)malloc(2 * S * nq);
    uint16_t* at = (uint16_t*)malloc(2 * S * nq);
    uint16_t* t = (uint16_t*)malloc(2 * S * H);
    uint16_t* g = (uint16_t*)malloc(2 * S * F);
    uint16_t* u = (uint16_t*)malloc(2 * S * F);
    int8_t* qbuf = (int8_t*)malloc(S * maxK);
    float* sbuf = (float*)malloc(sizeof(float) * S);
    float* ids = (float*)malloc(sizeof(float) * S);
    uint16_t** kl = (uint16_t**)calloc(c->num_layers, sizeof(void*));
    uint16_t** vl = (uint16_t**)calloc(c->num_layers, sizeof(void*));

    for (size_t i = 0; i < S; i++) ids[i] = (float)tok[i];
    int rc = orc_embedding_f16(m->embedding, ids, h, S, H, c->vocab);

    for (size_t l = 0; rc == 0 && l < c->num_layers; l++) {
        const orc_qwen_layer* L = &m->layers[l];
        uint16_t* k = (uint16_t*)malloc(2 * S * nkv);
        uint16_t* k2 = (uint16_t*)malloc(2 * S * nkv);
        uint16_t* v = (uint16_t*)malloc(2 * S * nkv);
        orc_rms_norm_f16(h, L->input_norm, x, S, H, c->eps);
        mm_int8(x, S, H, L->q_w, L->q_s, nq, gs, q, qbuf, sbuf);
        mm_int8(x, S, H, L->k_w, L->k_s, nkv, gs, k, qbuf, sbuf);
        mm_int8(x, S, H, L->v_w, L->v_s, nkv, gs, v, qbuf, sbuf);
        orc_rms_norm_f16(q, L->q_norm, q2, S * c->heads, hd, c->eps);
        orc_rms_norm_f16(k, L->k_norm, k2, S * c->kv_heads, hd, c->eps);
        orc_rope_f16(q2, q, 1, S, c->heads, hd, pos, c->rope_theta);
        orc_rope_f16(k2, k, 1, S, c->kv_heads, hd, pos, c->rope_theta);
        free(k2);
        if (cache_len == 0) {
            orc_attention_f16(q, k, v, at, 1, S, S, c->heads, c->kv_heads, hd, m->attn_scale,
                              NULL, pos, 0, 1);
        } else {
            const int8_t *kc, *vc;
            const float *ks, *vs;
            orc_kv_layer(m->kv, l, &kc, &vc, &ks, &vs);
            orc_attention_hybrid_int8_fp16(q, kc, vc, ks, vs, k, v, at, 1, S, cache_len, S, c->heads,
                                           c->kv_heads, hd, m->attn_scale, pos, 1, KV_GROUP);
        }
        kl[l] = k; vl[l] = v;
        mm_int8(at, S, nq, L->o_w, L->o_s, H, gs, t, qbuf, sbuf);
        orc_add_f16(h, t, h, S * H);
        orc_rms_norm_f16(h, L->post_norm, x, S, H, c->eps);
        mm_int4(x, S, H, L->gate_w, L->gate_s, F, gs, g, qbuf, sbuf);
        mm_int4(x, S, H, L->up_w, L->up_s, F, gs, u, qbuf, sbuf);
        orc_silu_f16(g, g, S * F);
        orc_multiply_f16(g, u, g, S * F);
        mm_int4(g, S, F, L->down_w, L->down_s, H, gs, t, qbuf, sbuf);
        orc_add_f16(h, t, h, S * H);
    }
    if (rc == 0) {
        free(m->last_hidden);
        m->last_hidden = (uint16_t*)malloc(2 * S * H);
        m->last_rows = S;
        orc_rms_norm_f16(h, m->out_norm, m->last_hidden, S, H, c->eps);
        /* KV update after the graph executes (engine_model.cpp:317-321) */
        rc = orc_kv_update(m->kv, (const uint16_t* const*)kl, (const uint16_t* const*)vl, S);
    }
    for (size_t l = 0; l < c->num_layers; l++) {
        free(kl[l]);
        free(vl[l]);
    }
    free(h); free(x); free(q); free(q2); free(at); free(t); free(g); free(u);
    free(qbuf); free(sbuf); free(ids); free(kl); free(vl);
    return rc;
}

int orc_qwen_prefill(orc_qwen* m, const uint32_t* tokens, size_t n, size_t chunk) {
    if (n == 0) return 0;
    if (n <= chunk) return qwen_forward(m, tokens, n);
    const size_t full = (n - 1) / chunk;
    for (size_t i = 0; i < full; i++) {
        int rc = qwen_forward(m, tokens + i * chunk, chunk);
        if (rc) return rc;
    }
    return qwen_forward(m, tokens + full * chunk, n - full * chunk);
}

uint32_t orc_qwen_decode(orc_qwen* m, uint32_t token, uint16_t* logits_out) {
    const orc_qwen_config* c = &m->cfg;
    if (qwen_forward(m, &token, 1) != 0) return UINT32_MAX;
    uint16_t* logits = logits_out ? logits_out : (uint16_t*)malloc(2 * (size_t)c->vocab);
    /* tied LM head: FP16 matmul against the embedding table (engine_model.cpp:241-246) */
    orc_matmul_f16(m->last_hidden + (m->last_rows - 1) * c->hidden, m->embedding, logits, 1,
                   c->hidden, c->vocab);
    uint32_t id = orc_argmax_f16(logits, c->vocab);
    if (!logits_out) free(logits);
    return id;
}
