/*
 * cactus_engine.h -- C ABI of the graph/engine layer (libcactus_engine.so).
 *
 * The engine drives the Qwen3-architecture model through the device graph of
 * cactus_amd/csrc/engine, which dispatches every node to the kernel ABI of
 * cactus_hip.h.  The entry points mirror the reference's Model interface
 * (cactus/engine/engine.h:473-577: init / prefill / decode / reset) and the
 * order in which the reference FFI drives it (cactus/ffi/cactus_complete.cpp:
 * 185-298: prefill the prompt minus its last token in 256-token chunks, then
 * decode from the last prompt token).  Decoding is greedy: argmax of the
 * logits with the first index winning ties (kernel_nn.cpp:451-466).
 *
 * Host pointers are host memory; the engine uploads weights once.
 * Every call returns 0 on success or -1 with cactus_engine_last_error().
 */
#ifndef CACTUS_ENGINE_H
#define CACTUS_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Qwen3 configuration (engine/engine.h:43-116 defaults for Qwen3-0.6B). */
typedef struct {
    uint32_t num_layers, hidden, ffn, heads, kv_heads, head_dim, vocab;
    uint32_t group_size;     /* quantization group of the INT8 / INT4 weights */
    float eps, rope_theta;
    uint32_t max_seq;        /* KV-cache capacity in tokens (no eviction) */
    uint32_t prefill_chunk;  /* Model::get_prefill_chunk_size() = 256 */
} cactus_qwen_config;

/* One decoder layer, host memory.  Attention projections are grouped INT8
 * ([out][in] codes + [out][in/group] fp16 scales); the MLP is packed INT4
 * ([out][in/2] bytes, low nibble = even input index) with fp16 scales;
 * norms are fp16. */
typedef struct {
    const uint16_t* input_norm;
    const int8_t* q_w;  const uint16_t* q_s;
    const int8_t* k_w;  const uint16_t* k_s;
    const int8_t* v_w;  const uint16_t* v_s;
    const int8_t* o_w;  const uint16_t* o_s;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    const uint16_t* post_norm;
    const uint8_t* gate_w; const uint16_t* gate_s;
    const uint8_t* up_w;   const uint16_t* up_s;
    const uint8_t* down_w; const uint16_t* down_s;
} cactus_qwen_layer_weights;

typedef struct {
    double prefill_ms;       /* wall time of Model::prefill over the prompt minus one */
    double first_decode_ms;  /* decode of the last prompt token */
    double decode_ms;        /* the remaining decode steps */
    uint32_t prefill_tokens, decode_tokens;
} cactus_qwen_timing;

const char* cactus_engine_last_error(void);

/* Model::init with caller-provided weights (tie_word_embeddings: the
 * embedding table [vocab][hidden] is also the LM head). */
int cactus_qwen_create(const cactus_qwen_config* cfg, const cactus_qwen_layer_weights* layers,
                       const uint16_t* embedding, const uint16_t* output_norm, void** model);
/* Random-init weights of the same architecture, generated on the host from
 * `seed` (codes uniform, scales |N(0,0.02)|/qmax, norms 1+N(0,0.02),
 * embeddings N(0,0.02)). */
int cactus_qwen_create_random(const cactus_qwen_config* cfg, uint64_t seed, void** model);
int cactus_qwen_destroy(void* model);
int cactus_qwen_reset(void* model);
/* Selects the decode path: 0 = node-by-node graph (one C-ABI call per node,
 * the reference's structure), 1 = fused per-layer kernels replayed as one
 * HIP graph per token.  Both are bit-identical. */
int cactus_qwen_set_decode_mode(void* model, int mode);
int cactus_qwen_prefill(void* model, const uint32_t* tokens, size_t n);
int cactus_qwen_decode(void* model, uint32_t token, uint32_t* next_token);
/* FFI flow: prefill prompt[:-1], decode prompt[-1], then feed back
 * max_new - 1 more greedy tokens; out_tokens receives max_new ids. */
int cactus_qwen_generate(void* model, const uint32_t* prompt, size_t n, size_t max_new,
                         uint32_t* out_tokens, cactus_qwen_timing* timing);
/* Final hidden state (after the output norm) of the last forward, fp16
 * [rows][hidden] copied into `out` (capacity max_rows rows). */
int cactus_qwen_last_hidden(void* model, uint16_t* out, size_t max_rows, size_t* rows);
/* Logits of the last decode step, fp16 [vocab] (decode mode 0 only). */
int cactus_qwen_last_logits(void* model, uint16_t* out);
int cactus_qwen_cache_len(void* model, size_t* len);
/* Copies layer `layer` of the INT8 KV cache (first cache_len tokens). */
int cactus_qwen_read_kv(void* model, size_t layer, int8_t* k, int8_t* v, float* k_scales,
                        float* v_scales);
/* Host copies of the weights the model holds (for random-init models). */
int cactus_qwen_read_weights(void* model, cactus_qwen_layer_weights* layers_out_buffers,
                             uint16_t* embedding, uint16_t* output_norm);

#ifdef __cplusplus
}
#endif
#endif
