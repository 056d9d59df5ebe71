/*
 * cactus_oracle.h -- CPU restatement of the Cactus quantized kernel layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * HIP kernels in cactus_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never links it.
 *
 * Every function restates one reference function (cited file:line, paths
 * relative to the reference repository root) with its exact arithmetic:
 * the same fp32 operation order, the same fused multiply-adds, the same
 * fp16 roundings.  fp16 values travel as raw uint16_t bit patterns.
 *
 * Libm boundary: the reference calls the platform expf/powf/cosf/sinf.
 *   - expf is replaced (here and in the HIP library) by orc_expf, a
 *     double-precision Cody-Waite + Taylor evaluation rounded once to
 *     float; it is checked against glibc expf in tests.
 *   - powf/cosf/sinf are only used to build the RoPE tables; both this
 *     oracle and the HIP library build those tables on the host with the
 *     host libm, so both sides see identical fp16 tables.
 */
#ifndef CACTUS_ORACLE_H
#define CACTUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 and exact fp16 arithmetic ---------------------------- */
float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);                 /* round to nearest even */
uint16_t orc_d2h(double d);                /* round to nearest even, single rounding */
uint16_t orc_hadd(uint16_t a, uint16_t b); /* fp16 add, RNE */
uint16_t orc_hmul(uint16_t a, uint16_t b); /* fp16 mul, RNE */
uint16_t orc_hfma(uint16_t a, uint16_t b, uint16_t c); /* fused a*b+c, one fp16 rounding */

/* ---- transcendental helpers --------------------------------------------- */
float orc_expf(float x);        /* libm expf substitute (see header) */
float orc_fast_exp(float x);    /* fast_exp_f32x4 lane, kernel_utils.h:108-141 */
float orc_poly_exp_weight(float score, float block_max); /* kernel_attention.cpp:174-195 */

/* ---- a1: activation quantization ---------------------------------------- */
float orc_fp16_max_abs(const uint16_t* src, size_t count);
void  orc_fp16_to_int8(const uint16_t* src, int8_t* dst, size_t count, float scale);
void  orc_quantize_activations(const uint16_t* x, int8_t* q, float* scales,
                               size_t M, size_t K);

/* ---- a2/a3: grouped integer matmul -------------------------------------- */
void orc_matmul_int8(const int8_t* A, const float* A_scales,
                     const int8_t* B, const uint16_t* B_scales,
                     uint16_t* C, size_t M, size_t K, size_t N, size_t group_size);
void orc_matmul_int4(const int8_t* A, const float* A_scales,
                     const uint8_t* B_packed, const uint16_t* B_scales,
                     uint16_t* C, size_t M, size_t K, size_t N, size_t group_size);
/* int32 per-group accumulators acc[m][n][g] (the bit-exact intermediate) */
void orc_group_sums_int8(const int8_t* A, const int8_t* B, int32_t* acc,
                         size_t M, size_t K, size_t N, size_t group_size);
void orc_unpack_int4_to_int8(const uint8_t* packed, int8_t* unpacked, size_t count);
/* threaded variants used only as the timed CPU baseline */
/* Worker threads of the row/head loops (1 = serial, the default); results
 * do not depend on it. */
void orc_set_threads(int n);

void orc_matmul_int8_mt(const int8_t* A, const float* A_scales,
                        const int8_t* B, const uint16_t* B_scales,
                        uint16_t* C, size_t M, size_t K, size_t N, size_t group_size,
                        int num_threads);

/* ---- a4: FP16 matmul with FP16 accumulation ----------------------------- */
void orc_matmul_f16(const uint16_t* a, const uint16_t* b_transposed, uint16_t* c,
                    size_t M, size_t K, size_t N);

/* ---- a5/a6: attention ----------------------------------------------------- */
void orc_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       uint16_t* o, size_t batch, size_t seq_len, size_t kv_seq_len,
                       size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                       float scale, const uint16_t* mask, size_t position_offset,
                       size_t window_size, int is_causal);
void orc_attention_hybrid_int8_fp16(const uint16_t* q, const int8_t* k_cached,
                                    const int8_t* v_cached, const float* k_scales,
                                    const float* v_scales, const uint16_t* k_new,
                                    const uint16_t* v_new, uint16_t* o, size_t batch,
                                    size_t seq_len, size_t cache_len, size_t new_len,
                                    size_t num_q_heads, size_t num_kv_heads,
                                    size_t head_dim, float scale, size_t position_offset,
                                    int is_causal, size_t quant_group_size);

/* ---- a7: KV quantization -------------------------------------------------- */
void orc_quantize_kv_fp16_to_int8(const uint16_t* src, int8_t* dst, float* scales,
                                  size_t seq_len, size_t kv_heads, size_t head_dim,
                                  size_t group_size);

/* ---- a8-a12: norm, rope, softmax, silu, elementwise --------------------- */
void orc_rms_norm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y,
                      size_t rows, size_t dims, float eps);
void orc_rope_tables(uint16_t* cos_tab, uint16_t* sin_tab, size_t num_pos,
                     size_t head_dim, float theta);
void orc_rope_f16(const uint16_t* x, uint16_t* y, size_t batch, size_t seq_len,
                  size_t num_heads, size_t head_dim, size_t start_pos, float theta);
void orc_softmax_f16(const uint16_t* x, uint16_t* y, size_t rows, size_t vocab);
void orc_silu_f16(const uint16_t* x, uint16_t* y, size_t n);
void orc_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n);
void orc_multiply_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n);

/* ---- a13/a14: embedding gather, greedy sample --------------------------- */
int      orc_embedding_f16(const uint16_t* table, const float* ids, uint16_t* out,
                           size_t num_ids, size_t hidden, size_t vocab);
uint32_t orc_argmax_f16(const uint16_t* logits, size_t vocab);

/* ---- f3: non-greedy FP16 sampler (sample_oracle.c) ----------------------- */
#define ORC_SAMPLE_HISTORY 128
/* the n-th output (n >= 1) of std::mt19937 seeded with `seed` */
uint32_t orc_mt19937_nth(uint32_t seed, size_t n);
/* uniform_real_distribution<float>(0, 1) over the first mt19937(seed) draw */
float    orc_sample_uniform(uint32_t seed);
/* cactus_sample_f16 (kernel_nn.cpp:446-651) with the draw `u` given and the
 * token history explicit (hist holds up to ORC_SAMPLE_HISTORY entries,
 * *hist_n of them used; updated like the reference's static history) */
uint32_t orc_sample_f16(const uint16_t* logits, size_t vocab, float temperature, float top_p,
                        size_t top_k, float u, uint32_t* hist, size_t* hist_n);

/* cactus_sample_f32 (kernel_nn.cpp:253-444) with the draw `u` given: bias
 * added, temperature divided, top-k, min-p 0.15, top-p, draw; no history */
uint32_t orc_sample_f32(const float* logits, size_t vocab, float temperature, float top_p, size_t top_k,
                        const float* bias_values, const uint32_t* bias_indices, size_t bias_count, float u);

/* Model::decode's normalised entropy of the logits (engine_model.cpp:255-290) */
float    orc_logits_entropy_f16(const uint16_t* logits, size_t vocab);

/* ---- f4: ops of other model families (family_oracle.c) ------------------ */
float orc_fast_tanh(float x);                                  /* kernel_utils.h:143-163 */
void  orc_gelu_f16(const uint16_t* in, uint16_t* out, size_t n);
void  orc_gelu_erf_f16(const uint16_t* in, uint16_t* out, size_t n);
void  orc_layer_norm_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y,
                         size_t rows, size_t features, float eps);
void  orc_conv1d_causal_depthwise_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t N,
                                      size_t L, size_t C, size_t K, size_t dilation);
void  orc_conv1d_f16_k3(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t N, size_t L,
                        size_t C_in, size_t C_out, size_t stride);

/* ---- a15: Qwen3-architecture forward ------------------------------------ */
typedef struct {
    uint32_t num_layers, hidden, ffn, heads, kv_heads, head_dim, vocab;
    uint32_t group_size;       /* weight quant group (attention INT8 and MLP INT4) */
    float eps, rope_theta;
    uint32_t max_seq;          /* KV cache tokens allocated up front (grows on demand) */
} orc_qwen_config;

typedef struct {
    const uint16_t* input_norm;      /* [hidden] */
    const int8_t*   q_w;  const uint16_t* q_s;   /* [heads*hd][hidden], [..][G] */
    const int8_t*   k_w;  const uint16_t* k_s;
    const int8_t*   v_w;  const uint16_t* v_s;
    const int8_t*   o_w;  const uint16_t* o_s;   /* [hidden][heads*hd] */
    const uint16_t* q_norm;          /* [hd] */
    const uint16_t* k_norm;          /* [hd] */
    const uint16_t* post_norm;       /* [hidden] */
    const uint8_t*  gate_w; const uint16_t* gate_s; /* packed int4 [ffn][hidden/2] */
    const uint8_t*  up_w;   const uint16_t* up_s;
    const uint8_t*  down_w; const uint16_t* down_s; /* packed int4 [hidden][ffn/2] */
} orc_qwen_layer;

typedef struct orc_qwen orc_qwen;   /* opaque: config, weights, KV cache */

orc_qwen* orc_qwen_create(const orc_qwen_config* cfg, const orc_qwen_layer* layers,
                          const uint16_t* embedding, const uint16_t* output_norm);
void      orc_qwen_destroy(orc_qwen* m);
void      orc_qwen_reset(orc_qwen* m);
/* Model::prefill (engine_model.cpp:170-219), chunked */
int       orc_qwen_prefill(orc_qwen* m, const uint32_t* tokens, size_t n, size_t chunk);
/* Model::decode greedy (engine_model.cpp:221-297); returns the token id */
uint32_t  orc_qwen_decode(orc_qwen* m, uint32_t token, uint16_t* logits_out);
/* final hidden state (after output norm) of the last forward, [rows][hidden] */
const uint16_t* orc_qwen_last_hidden(const orc_qwen* m, size_t* rows);
size_t    orc_qwen_cache_len(const orc_qwen* m);
/* KV cache read-back for one layer: pointers into the oracle's own cache */
void      orc_qwen_kv(const orc_qwen* m, size_t layer, const int8_t** k, const int8_t** v,
                      const float** ks, const float** vs);
/* KVCache::set_window_size on the model's cache (engine_model.cpp:136-146) */
int       orc_qwen_set_window(orc_qwen* m, size_t window, size_t sink);

/* ---- f2: INT8 KV cache with sliding window and sinks (kv_oracle.c) ------- */
typedef struct orc_kv orc_kv;
orc_kv* orc_kv_create(size_t layers, size_t max_seq, size_t kv_heads, size_t head_dim);
void    orc_kv_destroy(orc_kv* c);
/* KVCache::set_window_size (engine_cache.cpp:25-46): window 0 = no window */
int     orc_kv_set_window(orc_kv* c, size_t window, size_t sink);
void    orc_kv_reset(orc_kv* c);
/* KVCache::update_from_graph (engine_cache.cpp:103-330) with the K and V
 * rows of `seq` new tokens per layer ([seq][kv_heads][head_dim] fp16); -1
 * where the reference's update is undefined (see kv_oracle.c) */
int     orc_kv_update(orc_kv* c, const uint16_t* const* k_layers, const uint16_t* const* v_layers,
                      size_t seq);
size_t  orc_kv_len(const orc_kv* c);     /* current_seq_len */
size_t  orc_kv_total(const orc_kv* c);   /* total_seq_len */
void    orc_kv_layer(const orc_kv* c, size_t layer, const int8_t** k, const int8_t** v,
                     const float** ks, const float** vs);

#ifdef __cplusplus
}
#endif
#endif
