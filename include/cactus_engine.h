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
    uint32_t max_seq;        /* KV-cache capacity in tokens (the context size) */
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
 * `seed`: codes uniform, group scales |N(0,0.02)|/qmax (down projection
 * |N(0,0.1)|/qmax), norms 1+N(0,0.02), embeddings N(0,0.005).  The two wider
 * or narrower scales keep greedy decode from repeating one token (with all
 * at 0.02 the residual stream of a deep random model loses its dependence on
 * the input token).  Deterministic for a seed, whatever the host's core
 * count. */
int cactus_qwen_create_random(const cactus_qwen_config* cfg, uint64_t seed, void** model);
/* The weights cactus_qwen_create_random(cfg, seed) uploads, written into
 * caller-provided host buffers (the shapes of cactus_qwen_layer_weights; the
 * const pointers of each layer entry name writable buffers).  Host only: no
 * device is touched, so the same weights can feed a CPU model. */
int cactus_qwen_random_weights(const cactus_qwen_config* cfg, uint64_t seed,
                               cactus_qwen_layer_weights* layers_out_buffers, uint16_t* embedding,
                               uint16_t* output_norm);
int cactus_qwen_destroy(void* model);
int cactus_qwen_reset(void* model);
/* Selects the decode path: 0 = node-by-node graph (one C-ABI call per node,
 * the reference's structure), 1 = fused per-layer kernels replayed as one
 * HIP graph per token.  Both are bit-identical. */
int cactus_qwen_set_decode_mode(void* model, int mode);
/* Selects the attention arithmetic: 0 = exact (the reference's operation
 * order, bit-identical; the default), 1 = tolerance mode: every attention
 * node runs the _fast kernels -- decode steps the split-K kernels of
 * cactus_hip_attention_*_fast / cactus_hip_decode_prep_attention_fast,
 * prefill chunks the FP16-MFMA flash attention of
 * cactus_hip_attention_hybrid_int8_fp16_fast -- within 1e-3 + 1e-2 |ref| of
 * the reference per fp16 output, and the softmax (not the reference's zero
 * row) where the reference's block rescale overflows.  Greedy tokens are
 * therefore not guaranteed to equal the reference's.  Applies to both
 * decode modes. */
int cactus_qwen_set_attention_mode(void* model, int mode);
/* KVCache::set_window_size (engine/engine_cache.cpp:25-46): keep at most
 * `window` cached tokens -- the first `sink` of the sequence and the most
 * recent window - sink (update_from_graph, :103-330) -- while positions keep
 * counting (RoPE and the attention's causal offset use the total length).
 * window 0 = no window (the cache must then hold the whole sequence).  The
 * first `window` slots are reset to codes 0, scales 1.0, as in the
 * reference; call it before the first token.  Models from
 * cactus_qwen_create / _create_random start without a window;
 * cactus_qwen_create_from_folder applies Model::init's default
 * (min(context, 512), 4 sinks, CACTUS_KV_WINDOW_SIZE / CACTUS_KV_SINK_SIZE,
 * engine_model.cpp:136-146).  A step that would add more than
 * window - sink tokens to a full window is an error (the reference's
 * arithmetic wraps there). */
int cactus_qwen_set_kv_window(void* model, size_t window, size_t sink);
/* Model::decode's sampling settings (engine_model.cpp:221-250 ->
 * cactus_hip_sample_f16): all zero = greedy (the default).  Non-greedy steps
 * run the node graph's sample node in either decode mode; random_seed 0
 * draws the reference's seed (the clock) per step, a nonzero seed is used
 * for every step. */
int cactus_qwen_set_sampling(void* model, float temperature, float top_p, size_t top_k, size_t random_seed);
/* total_seq_len: tokens processed since the last reset */
int cactus_qwen_total_len(void* model, size_t* len);
int cactus_qwen_prefill(void* model, const uint32_t* tokens, size_t n);
int cactus_qwen_decode(void* model, uint32_t token, uint32_t* next_token);
/* FFI flow: prefill prompt[:-1], decode prompt[-1], then feed back
 * max_new - 1 more greedy tokens; out_tokens receives max_new ids. */
int cactus_qwen_generate(void* model, const uint32_t* prompt, size_t n, size_t max_new,
                         uint32_t* out_tokens, cactus_qwen_timing* timing);
/* Final hidden state (after the output norm) of the last forward, fp16
 * [rows][hidden] copied into `out` (capacity max_rows rows). */
int cactus_qwen_last_hidden(void* model, uint16_t* out, size_t max_rows, size_t* rows);
/* Logits of the last decode step, fp16 [vocab] (either decode mode; an
 * error before the first step after a reset or prefill). */
int cactus_qwen_last_logits(void* model, uint16_t* out);
/* Model::decode's out_entropy (engine_model.cpp:255-290) for the last
 * decode step's logits: normalised softmax entropy in [0, 1], the
 * confidence signal of the reference's cloud handoff. */
int cactus_qwen_last_entropy(void* model, float* entropy);
int cactus_qwen_cache_len(void* model, size_t* len);
/* Copies layer `layer` of the INT8 KV cache (first cache_len tokens). */
int cactus_qwen_read_kv(void* model, size_t layer, int8_t* k, int8_t* v, float* k_scales,
                        float* v_scales);
/* Host copies of the weights the model holds (for random-init models). */
int cactus_qwen_read_weights(void* model, cactus_qwen_layer_weights* layers_out_buffers,
                             uint16_t* embedding, uint16_t* output_norm);

/* ---- CACT tensor files (cactus/graph/graph_io.cpp) -------------------------
 * One tensor per file: an 80-byte little-endian header (magic "CACT",
 * version, flags, alignment, ndim, dims[4] as u64, precision, data bytes,
 * scales bytes, group size, group count), fp16 group scales [rows][groups]
 * at align(80, alignment), data at align(end of scales, alignment).
 * Precision: 0 INT8, 1 FP16, 2 FP32, 3 INT4 (two codes per byte, low nibble
 * = even column) -- graph.h:99-104. */
typedef struct {
    uint32_t version, flags, alignment, ndim;
    uint64_t shape[4];
    uint32_t precision, group_size, num_groups;
    uint64_t data_bytes, scales_bytes, scales_offset, data_offset;
} cactus_cact_info;

/* MappedFile::parse_header (graph_io.cpp:497-566); host only.  Fails on a
 * short file, a wrong magic, scales or data past the end of the file, or an
 * unknown precision. */
int cactus_cact_read_info(const char* path, cactus_cact_info* info);
/* GraphFile::save_node's layout (graph_io.cpp:145-222), alignment 32, from
 * host buffers; scales may be NULL (then group_size and num_groups are
 * written as 0).  Host only. */
int cactus_cact_save(const char* path, const uint64_t* shape, uint32_t ndim, uint32_t precision,
                     const void* data, uint64_t data_bytes, const uint16_t* scales, uint32_t group_size,
                     uint32_t num_groups);
/* GraphFile::load_into_graph (graph_io.cpp:228-320) to device memory: the
 * data (INT4 stays packed) and the scales (NULL when the file has none),
 * each from cactus_hip_malloc; release them with cactus_hip_free.  With
 * scales == NULL the scales are not kept. */
int cactus_cact_load_device(const char* path, cactus_cact_info* info, void** data, void** scales);

/* Config::from_json over folder/config.txt (engine_model.cpp:403-520):
 * key=value lines, '#' comments; keys not present keep the reference's
 * defaults (engine.h:42-58).  group_size is read from
 * layer_0_attn_q.weights; max_seq is 0.  Fails for model types other than
 * Qwen, untied output weights and mixture-of-experts configs. */
int cactus_qwen_read_config(const char* folder, cactus_qwen_config* cfg);
/* Model::init(model_folder, context_size) (engine_model.cpp:47-160) over the
 * reference's file names (model_qwen.cpp:17-42, token_embeddings.weights):
 * FP16 embeddings and norms, grouped INT8 attention projections, packed INT4
 * MLP, one group size.  Any other precision, shape or group layout is an
 * error naming the file. */
int cactus_qwen_create_from_folder(const char* folder, size_t context_size, void** model);

/* A device graph for the file API (CactusGraph::load_weights / mmap_weights /
 * mmap_embeddings, graph_io.cpp:25-101; GraphFile::save_node). */
typedef struct {
    uint32_t ndim;
    uint64_t shape[4];
    uint32_t precision;      /* 3 for packed INT4 nodes */
    uint64_t data_bytes;
    uint32_t group_size, num_groups;
} cactus_graph_node_desc;

int cactus_graph_create(void** graph);
int cactus_graph_destroy(void* graph);
int cactus_graph_load_weights(void* graph, const char* path, size_t* node);
int cactus_graph_mmap_embeddings(void* graph, const char* path, size_t* node);
int cactus_graph_save_node(void* graph, size_t node, const char* path);
int cactus_graph_node_info(void* graph, size_t node, cactus_graph_node_desc* desc);
/* Copies a node's data (packed bytes for INT4) and, when asked, its group
 * scales to host memory. */
int cactus_graph_read_node(void* graph, size_t node, void* data, uint64_t capacity, uint16_t* scales,
                           uint64_t scales_capacity);

#ifdef __cplusplus
}
#endif
#endif
