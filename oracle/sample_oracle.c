/*
 * sample_oracle.c -- CPU restatement of the reference's non-greedy FP16
 * sampler and its random draw (test infrastructure; see cactus_oracle.h):
 *
 *   cactus_sample_f16                 kernel/kernel_nn.cpp:446-651
 *   cactus_sample_f32                 kernel/kernel_nn.cpp:253-444
 *   std::mt19937 + uniform_real_distribution<float>(0, 1), first draw
 *                                     kernel/kernel_nn.cpp:609-612
 *
 * Behaviour restated on purpose:
 *   - the logit bias is added and then overwritten: the temperature step
 *     reads the raw logits again (:501-511) and without a temperature they
 *     are copied back (:512-514), so the bias never reaches the result;
 *   - the f16 sampler has no min-p step (only cactus_sample_f32 does);
 *   - the repetition penalty (1.1) walks a history of the last 128 tokens
 *     this sampler returned, in order, once per occurrence (:516-529);
 *     greedy calls do not record;
 *   - top-k keeps every logit >= the k-th largest value (ties included);
 *   - top-p sorts the surviving logits descending, turns them into
 *     probabilities with expf in that order, and cuts after the first
 *     position j > 0 whose running sum exceeds top_p (:550-590).
 * The order std::sort gives equal logits is unspecified; here ties keep
 * ascending token order (parity unpinned where two equal logits straddle
 * the top-p cut).
 *
 * The draw: MT19937 (Matsumoto & Nishimura 1998, the C++ standard's
 * std::mt19937) seeded with the 32-bit seed, first output x, then
 * u = (float)x / 2^32 -- libc++'s generate_canonical<float, 24> for a 32-bit
 * engine, times (b - a) = 1, plus a = 0.
 */
#include "cactus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define MT_N 624
#define MT_M 397

uint32_t orc_mt19937_nth(uint32_t seed, size_t n) {
    uint32_t mt[MT_N];
    mt[0] = seed;
    for (uint32_t i = 1; i < MT_N; i++) mt[i] = 1812433253u * (mt[i - 1] ^ (mt[i - 1] >> 30)) + i;
    size_t idx = MT_N;
    uint32_t y = 0;
    for (size_t k = 0; k < n; k++) {
        if (idx >= MT_N) {
            for (int i = 0; i < MT_N; i++) {
                const uint32_t v = (mt[i] & 0x80000000u) | (mt[(i + 1) % MT_N] & 0x7fffffffu);
                mt[i] = mt[(i + MT_M) % MT_N] ^ (v >> 1) ^ ((v & 1u) ? 0x9908b0dfu : 0u);
            }
            idx = 0;
        }
        y = mt[idx++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9d2c5680u;
        y ^= (y << 15) & 0xefc60000u;
        y ^= y >> 18;
    }
    return y;
}

float orc_sample_uniform(uint32_t seed) {
    return (float)orc_mt19937_nth(seed, 1) / 4294967296.0f;
}

#define NEG_INF_H 0xFC00u

typedef struct {
    uint16_t v;
    uint32_t i;
} cand;

static int cand_desc(const void* a, const void* b) {
    const cand* x = (const cand*)a;
    const cand* y = (const cand*)b;
    const float fx = orc_h2f(x->v), fy = orc_h2f(y->v);
    if (fx > fy) return -1;
    if (fx < fy) return 1;
    return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

static void push_history(uint32_t* hist, size_t* n, uint32_t tok) {
    if (*n == ORC_SAMPLE_HISTORY) {
        memmove(hist, hist + 1, (ORC_SAMPLE_HISTORY - 1) * sizeof(uint32_t));
        *n = ORC_SAMPLE_HISTORY - 1;
    }
    hist[(*n)++] = tok;
}

uint32_t orc_sample_f16(const uint16_t* logits, size_t V, float temperature, float top_p, size_t top_k,
                        float u, uint32_t* hist, size_t* hist_n) {
    if (temperature == 0.0f && top_p <= 0.0f && top_k == 0) return V ? orc_argmax_f16(logits, V) : 0;
    if (V == 0) return 0;
    uint16_t* f = (uint16_t*)malloc(V * sizeof(uint16_t));
    /* :501-514 -- the bias is lost either way */
    if (temperature > 0) {
        const uint16_t inv = orc_f2h(1.0f / temperature);
        for (size_t i = 0; i < V; i++) f[i] = orc_hmul(logits[i], inv);
    } else {
        memcpy(f, logits, V * sizeof(uint16_t));
    }
    /* :516-529 */
    if (*hist_n > 0) {
        const uint16_t pen_inv = orc_f2h(1.0f / 1.1f), pen = orc_f2h(1.1f);
        for (size_t j = 0; j < *hist_n; j++) {
            const uint32_t t = hist[j];
            if (t < V) f[t] = orc_h2f(f[t]) > 0.0f ? orc_hmul(f[t], pen_inv) : orc_hmul(f[t], pen);
        }
    }
    /* :531-548 */
    if (top_k > 0 && top_k < V) {
        cand* c = (cand*)malloc(V * sizeof(cand));
        for (size_t i = 0; i < V; i++) { c[i].v = f[i]; c[i].i = (uint32_t)i; }
        qsort(c, V, sizeof(cand), cand_desc);
        const float kth = orc_h2f(c[top_k - 1].v);
        free(c);
        for (size_t i = 0; i < V; i++)
            if (orc_h2f(f[i]) < kth) f[i] = NEG_INF_H;
    }
    /* :550-590 */
    if (top_p > 0.0f && top_p < 1.0f) {
        cand* c = (cand*)malloc(V * sizeof(cand));
        size_t n = 0;
        for (size_t i = 0; i < V; i++)
            if (orc_h2f(f[i]) != orc_h2f(NEG_INF_H)) { c[n].v = f[i]; c[n].i = (uint32_t)i; n++; }
        qsort(c, n, sizeof(cand), cand_desc);
        if (n > 0) {
            const float mx = orc_h2f(c[0].v);
            float* p = (float*)malloc(n * sizeof(float));
            float sum = 0.0f;
            for (size_t j = 0; j < n; j++) {
                p[j] = orc_expf(orc_h2f(c[j].v) - mx);
                sum += p[j];
            }
            for (size_t j = 0; j < n; j++) p[j] /= sum;
            float cum = 0.0f;
            int reached = 0;
            for (size_t j = 0; j < n; j++) {
                cum += p[j];
                if (cum > top_p && j > 0) reached = 1;
                if (reached && j > 0) f[c[j].i] = NEG_INF_H;
            }
            free(p);
        }
        free(c);
    }
    /* :592-633 */
    uint16_t mxh = f[0];
    for (size_t i = 1; i < V; i++)
        if (orc_h2f(f[i]) > orc_h2f(mxh)) mxh = f[i];
    if (orc_h2f(mxh) == orc_h2f(NEG_INF_H)) {
        free(f);
        return 0;
    }
    const float mx = orc_h2f(mxh);
    float* p = (float*)malloc(V * sizeof(float));
    float sum = 0.0f;
    for (size_t i = 0; i < V; i++) {
        if (orc_h2f(f[i]) == orc_h2f(NEG_INF_H)) {
            p[i] = 0.0f;
        } else {
            p[i] = orc_expf(orc_h2f(f[i]) - mx);
            sum += p[i];
        }
    }
    free(f);
    if (sum == 0.0f) {
        free(p);
        return 0;
    }
    for (size_t i = 0; i < V; i++) p[i] /= sum;
    float cum = 0.0f;
    uint32_t tok = 0;
    int found = 0;
    for (size_t i = 0; i < V && !found; i++) {
        cum += p[i];
        if (cum >= u) { tok = (uint32_t)i; found = 1; }
    }
    for (size_t i = V; i > 0 && !found; i--)
        if (p[i - 1] > 0.0f) { tok = (uint32_t)(i - 1); found = 1; }
    free(p);
    push_history(hist, hist_n, tok);
    return tok;
}

/* Model::decode's out_entropy (engine/engine_model.cpp:255-290): softmax
 * entropy of the fp16 logits in double, sequential in token order, divided
 * by log(vocab), returned as float.  exp and log are the host libm's. */
float orc_logits_entropy_f16(const uint16_t* logits, size_t V) {
    float mx = orc_h2f(logits[0]);
    for (size_t i = 1; i < V; i++)
        if (orc_h2f(logits[i]) > mx) mx = orc_h2f(logits[i]);
    double sum_exp = 0.0;
    for (size_t i = 0; i < V; i++) sum_exp += exp((double)(orc_h2f(logits[i]) - mx));
    const double lse = (double)mx + log(sum_exp);
    double ent = 0.0;
    for (size_t i = 0; i < V; i++) {
        const double lp = (double)orc_h2f(logits[i]) - lse;
        const double p = exp(lp);
        if (p > 1e-10) ent -= p * lp;
    }
    return (float)(ent / log((double)V));
}

/* cactus_sample_f32 (kernel_nn.cpp:253-444).  Unlike the f16 sampler: the
 * logit bias is added (entry by entry, in order, :280-288) and kept; the
 * temperature divides (:290-294); a min-p step with min_p = 0.15 runs
 * between top-k and top-p (:316-346); there is no repetition penalty and no
 * history.  Both infinities count as removed (std::isinf).  expf is the
 * libm boundary of the f16 sampler.  Ties in the top-p sort keep ascending
 * token order (parity unpinned where equal logits straddle the cut). */
static int isinf_f(float x) { return x == INFINITY || x == -INFINITY; }

typedef struct {
    float v;
    uint32_t i;
} cand32;

static int cand32_desc(const void* a, const void* b) {
    const cand32* x = (const cand32*)a;
    const cand32* y = (const cand32*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

uint32_t orc_sample_f32(const float* logits, size_t V, float temperature, float top_p, size_t top_k,
                        const float* bias_values, const uint32_t* bias_indices, size_t bias_count, float u) {
    if (temperature == 0.0f && top_p <= 0.0f && top_k == 0) {
        if (V == 0) return 0;
        size_t best = 0;
        float bv = logits[0];
        for (size_t i = 1; i < V; i++)
            if (logits[i] > bv) { bv = logits[i]; best = i; }
        return (uint32_t)best;
    }
    float* f = (float*)malloc((V ? V : 1) * sizeof(float));
    memcpy(f, logits, V * sizeof(float));
    if (bias_values && bias_indices)
        for (size_t j = 0; j < bias_count; j++)
            if (bias_indices[j] < V) f[bias_indices[j]] += bias_values[j];
    if (temperature > 0)
        for (size_t i = 0; i < V; i++) f[i] /= temperature;
    /* :296-313 -- top_k >= vocab keeps everything */
    if (top_k > 0 && top_k < V) {
        cand32* c = (cand32*)malloc(V * sizeof(cand32));
        for (size_t i = 0; i < V; i++) { c[i].v = f[i]; c[i].i = (uint32_t)i; }
        qsort(c, V, sizeof(cand32), cand32_desc);
        const float kth = c[top_k - 1].v;
        free(c);
        for (size_t i = 0; i < V; i++)
            if (f[i] < kth) f[i] = -INFINITY;
    }
    /* :316-346 */
    {
        const float min_p = 0.15f;
        float mx = V ? f[0] : 0.0f;
        for (size_t i = 1; i < V; i++)
            if (f[i] > mx) mx = f[i];
        if (V && !isinf_f(mx)) {
            float* tp = (float*)malloc(V * sizeof(float));
            float sum = 0.0f;
            for (size_t i = 0; i < V; i++) {
                if (!isinf_f(f[i])) {
                    tp[i] = orc_expf(f[i] - mx);
                    sum += tp[i];
                } else {
                    tp[i] = 0.0f;
                }
            }
            if (sum > 0.0f) {
                float mp = 0.0f;
                for (size_t i = 0; i < V; i++) {
                    tp[i] /= sum;
                    if (i == 0 || tp[i] > mp) mp = tp[i];
                }
                const float thr = mp * min_p;
                for (size_t i = 0; i < V; i++)
                    if (tp[i] < thr) f[i] = -INFINITY;
            }
            free(tp);
        }
    }
    /* :348-392 */
    if (top_p > 0.0f && top_p < 1.0f) {
        cand32* c = (cand32*)malloc((V ? V : 1) * sizeof(cand32));
        size_t n = 0;
        for (size_t i = 0; i < V; i++)
            if (!isinf_f(f[i])) { c[n].v = f[i]; c[n].i = (uint32_t)i; n++; }
        qsort(c, n, sizeof(cand32), cand32_desc);
        if (n > 0) {
            const float mx = c[0].v;
            float* p = (float*)malloc(n * sizeof(float));
            float sum = 0.0f;
            for (size_t j = 0; j < n; j++) {
                p[j] = orc_expf(c[j].v - mx);
                sum += p[j];
            }
            for (size_t j = 0; j < n; j++) p[j] /= sum;
            /* remove from the first position whose running sum exceeds
             * top_p on, but never position 0 (:373-386) */
            float cum = 0.0f;
            size_t cut = n;
            for (size_t j = 0; j < n; j++) {
                cum += p[j];
                if (cum > top_p) { cut = j; break; }
            }
            if (cut == 0) cut = 1;
            for (size_t j = cut; j < n; j++) f[c[j].i] = -INFINITY;
            free(p);
        }
        free(c);
    }
    /* :394-444 */
    float mx = V ? f[0] : 0.0f;
    for (size_t i = 1; i < V; i++)
        if (f[i] > mx) mx = f[i];
    if (V == 0 || isinf_f(mx)) {
        free(f);
        return 0;
    }
    float* p = (float*)malloc(V * sizeof(float));
    float sum = 0.0f;
    for (size_t i = 0; i < V; i++) {
        if (isinf_f(f[i])) {
            p[i] = 0.0f;
        } else {
            p[i] = orc_expf(f[i] - mx);
            sum += p[i];
        }
    }
    free(f);
    if (sum == 0.0f) {
        free(p);
        return 0;
    }
    for (size_t i = 0; i < V; i++) p[i] /= sum;
    float cum = 0.0f;
    uint32_t tok = 0;
    int found = 0;
    for (size_t i = 0; i < V && !found; i++) {
        cum += p[i];
        if (cum >= u) { tok = (uint32_t)i; found = 1; }
    }
    for (size_t i = V; i > 0 && !found; i--)
        if (p[i - 1] > 0.0f) { tok = (uint32_t)(i - 1); found = 1; }
    free(p);
    return tok;
}
