/*
 * kv_oracle.c -- CPU restatement of the engine's INT8 KV cache with the
 * sliding window and attention sinks (test infrastructure; see
 * cactus_oracle.h):
 *
 *   KVCache::init                      engine/engine_cache.cpp:11-23
 *   KVCache::set_window_size           engine/engine_cache.cpp:25-46
 *   KVCache::reset                     engine/engine_cache.cpp:48-51
 *   KVCache::update_from_graph         engine/engine_cache.cpp:103-330
 *
 * The reference keeps each layer's cache in std::vectors that are resized
 * as the sequence grows and slides; what a resize keeps matters once, in
 * the sliding branch of a full rewrite (a first update longer than the
 * window), which writes the sink rows only when the vectors were not
 * already window-sized (:167-197).  This restatement therefore tracks the
 * vectors' size in tokens ("resident") and their contents exactly: growth
 * value-initialises (codes 0, scales 0.0f), set_window_size fills codes
 * with 0 and scales with 1.0f.
 *
 * The sliding append computes window - sink - seq in size_t (:268-270); a
 * step longer than window - sink wraps around and the memmove that follows
 * is undefined.  orc_kv_update returns -1 for it instead.
 */
#include "cactus_oracle.h"

#include <stdlib.h>
#include <string.h>

#define KV_GROUP 128

struct orc_kv {
    size_t layers, kv_heads, head_dim, groups;
    size_t cap;                  /* allocated tokens */
    size_t window, sink;
    size_t resident;             /* tokens the reference's vectors hold */
    size_t len, total;           /* current_seq_len, total_seq_len */
    int8_t** k; int8_t** v; float** ks; float** vs;
};

static size_t tok_codes(const orc_kv* c) { return c->kv_heads * c->head_dim; }
static size_t tok_scales(const orc_kv* c) { return c->kv_heads * c->groups; }

static int reserve(orc_kv* c, size_t tokens) {
    if (tokens <= c->cap) return 0;
    for (size_t l = 0; l < c->layers; l++) {
        int8_t* k = (int8_t*)realloc(c->k[l], tokens * tok_codes(c));
        int8_t* v = (int8_t*)realloc(c->v[l], tokens * tok_codes(c));
        float* ks = (float*)realloc(c->ks[l], tokens * tok_scales(c) * sizeof(float));
        float* vs = (float*)realloc(c->vs[l], tokens * tok_scales(c) * sizeof(float));
        if (k) c->k[l] = k;
        if (v) c->v[l] = v;
        if (ks) c->ks[l] = ks;
        if (vs) c->vs[l] = vs;
        if (!k || !v || !ks || !vs) return -1;
    }
    c->cap = tokens;
    return 0;
}

/* std::vector::resize of every layer's four vectors to `tokens` tokens */
static int resize(orc_kv* c, size_t tokens) {
    if (reserve(c, tokens)) return -1;
    if (tokens > c->resident) {
        const size_t a = c->resident, n = tokens - a;
        for (size_t l = 0; l < c->layers; l++) {
            memset(c->k[l] + a * tok_codes(c), 0, n * tok_codes(c));
            memset(c->v[l] + a * tok_codes(c), 0, n * tok_codes(c));
            memset(c->ks[l] + a * tok_scales(c), 0, n * tok_scales(c) * sizeof(float));
            memset(c->vs[l] + a * tok_scales(c), 0, n * tok_scales(c) * sizeof(float));
        }
    }
    c->resident = tokens;
    return 0;
}

orc_kv* orc_kv_create(size_t layers, size_t max_seq, size_t kv_heads, size_t head_dim) {
    orc_kv* c = (orc_kv*)calloc(1, sizeof(orc_kv));
    c->layers = layers;
    c->kv_heads = kv_heads;
    c->head_dim = head_dim;
    c->groups = (head_dim + KV_GROUP - 1) / KV_GROUP;
    c->k = (int8_t**)calloc(layers, sizeof(void*));
    c->v = (int8_t**)calloc(layers, sizeof(void*));
    c->ks = (float**)calloc(layers, sizeof(void*));
    c->vs = (float**)calloc(layers, sizeof(void*));
    if (reserve(c, max_seq ? max_seq : 1)) {
        orc_kv_destroy(c);
        return NULL;
    }
    return c;
}

void orc_kv_destroy(orc_kv* c) {
    if (!c) return;
    for (size_t l = 0; l < c->layers; l++) {
        free(c->k[l]); free(c->v[l]); free(c->ks[l]); free(c->vs[l]);
    }
    free(c->k); free(c->v); free(c->ks); free(c->vs);
    free(c);
}

int orc_kv_set_window(orc_kv* c, size_t window, size_t sink) {
    c->window = window;
    c->sink = sink;
    if (window == 0) return 0;
    if (resize(c, window)) return -1;
    for (size_t l = 0; l < c->layers; l++) {
        memset(c->k[l], 0, window * tok_codes(c));
        memset(c->v[l], 0, window * tok_codes(c));
        for (size_t i = 0; i < window * tok_scales(c); i++) {
            c->ks[l][i] = 1.0f;
            c->vs[l][i] = 1.0f;
        }
    }
    return 0;
}

void orc_kv_reset(orc_kv* c) { c->len = 0; c->total = 0; }
size_t orc_kv_len(const orc_kv* c) { return c->len; }
size_t orc_kv_total(const orc_kv* c) { return c->total; }

void orc_kv_layer(const orc_kv* c, size_t l, const int8_t** k, const int8_t** v, const float** ks,
                  const float** vs) {
    *k = c->k[l]; *v = c->v[l]; *ks = c->ks[l]; *vs = c->vs[l];
}

/* quantize rows [r0, r0 + n) of one layer's fp16 K and V into tokens [t, t + n) */
static void put(orc_kv* c, size_t l, const uint16_t* kf, const uint16_t* vf, size_t r0, size_t n, size_t t) {
    if (n == 0) return;
    orc_quantize_kv_fp16_to_int8(kf + r0 * tok_codes(c), c->k[l] + t * tok_codes(c),
                                 c->ks[l] + t * tok_scales(c), n, c->kv_heads, c->head_dim, KV_GROUP);
    orc_quantize_kv_fp16_to_int8(vf + r0 * tok_codes(c), c->v[l] + t * tok_codes(c),
                                 c->vs[l] + t * tok_scales(c), n, c->kv_heads, c->head_dim, KV_GROUP);
}

int orc_kv_update(orc_kv* c, const uint16_t* const* kl, const uint16_t* const* vl, size_t seq) {
    const size_t old = c->len, nt = old + seq;
    const int sliding = c->window > 0 && nt > c->window;
    const size_t W = c->window, snk = c->sink;
    if (seq == 0) return 0;
    if (sliding && snk > W) return -1;
    if (sliding && old > 0 && seq > W - snk) return -1;    /* size_t wrap in the reference */
    if (old == 0) {
        /* full rewrite: the K/V nodes hold all new_total rows (:131-232) */
        if (!sliding) {
            if (resize(c, nt)) return -1;
            for (size_t l = 0; l < c->layers; l++) put(c, l, kl[l], vl[l], 0, nt, 0);
        } else {
            const int first = c->resident != W;
            const size_t skip = nt - W;
            if (first && resize(c, W)) return -1;
            for (size_t l = 0; l < c->layers; l++) {
                if (first) put(c, l, kl[l], vl[l], 0, snk, 0);
                put(c, l, kl[l], vl[l], snk + skip, W - snk, snk);
            }
        }
    } else if (!sliding) {
        /* append (:234-267) */
        if (resize(c, nt)) return -1;
        for (size_t l = 0; l < c->layers; l++) put(c, l, kl[l], vl[l], 0, seq, old);
    } else {
        /* append with the window full: keep the sinks, slide the rest (:268-327) */
        if (c->resident != W && resize(c, W)) return -1;
        const size_t shift = W - snk - seq;
        for (size_t l = 0; l < c->layers; l++) {
            if (shift > 0 && old > snk) {
                const size_t src = old - shift;
                if (src > snk) {
                    memmove(c->k[l] + snk * tok_codes(c), c->k[l] + src * tok_codes(c), shift * tok_codes(c));
                    memmove(c->v[l] + snk * tok_codes(c), c->v[l] + src * tok_codes(c), shift * tok_codes(c));
                    memmove(c->ks[l] + snk * tok_scales(c), c->ks[l] + src * tok_scales(c),
                            shift * tok_scales(c) * sizeof(float));
                    memmove(c->vs[l] + snk * tok_scales(c), c->vs[l] + src * tok_scales(c),
                            shift * tok_scales(c) * sizeof(float));
                }
            }
            put(c, l, kl[l], vl[l], 0, seq, W - seq);
        }
    }
    c->len = sliding ? W : nt;
    c->total += seq;
    return 0;
}
