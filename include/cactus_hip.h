/*
 * cactus_hip.h -- C ABI of the MI355X (gfx950) kernel layer.
 *
 * Each kernel entry point replaces one free function of the reference's
 * kernel layer (cactus/kernel/kernel.h) or one graph node executor that
 * wraps it (cactus/graph/graph_ops_nn.cpp); the citation on each
 * declaration names the reference interface it stands in for.
 *
 * Conventions (differences from kernel.h are deliberate):
 *   - fp16 values are passed as uint16_t bit patterns (IEEE binary16).
 *   - Every tensor pointer is a DEVICE pointer unless stated otherwise;
 *     memory is owned by the caller (cactus_hip_malloc or any HIP allocation).
 *   - `stream` is a hipStream_t (NULL = the default stream).  Kernels are
 *     enqueued on it and the call returns without waiting, except the
 *     memcpy_d2h / memcpy_h2d helpers, which wait for the copy.
 *   - Every call returns 0 on success or a negative CACTUS_HIP_E* code;
 *     cactus_hip_last_error() then holds a message for the calling thread.
 *     Bad shapes are rejected on the host before anything is launched (the
 *     reference kernels return silently on M|K|N == 0; so do these).
 *   - Results are bit-identical to the reference's arithmetic where the
 *     reference defines it (integer sums, quantized codes, fp16 roundings,
 *     operation order); see the comment on each entry point.
 */
#ifndef CACTUS_HIP_H
#define CACTUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CACTUS_HIP_OK              0
#define CACTUS_HIP_EINVAL        (-1)   /* bad argument / shape */
#define CACTUS_HIP_EUNSUPPORTED  (-2)   /* valid in the reference, not built here */
#define CACTUS_HIP_ERUNTIME      (-3)   /* HIP runtime error */
#define CACTUS_HIP_ENOMEM        (-4)

/* ---------------------------------------------------------------- runtime */
int         cactus_hip_init(int device);
const char* cactus_hip_last_error(void);
int         cactus_hip_device_count(int* count);
/* free and total device memory of the current device (hipMemGetInfo); no
 * reference counterpart: a diagnostic, e.g. to show that a call allocates
 * nothing */
int         cactus_hip_device_memory(size_t* free_bytes, size_t* total_bytes);
int         cactus_hip_malloc(void** ptr, size_t bytes);
int         cactus_hip_free(void* ptr);
int         cactus_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int         cactus_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int         cactus_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int         cactus_hip_memset(void* dst, int byte_value, size_t bytes, void* stream);
int         cactus_hip_stream_create(void** stream);
int         cactus_hip_stream_destroy(void* stream);
int         cactus_hip_stream_sync(void* stream);
int         cactus_hip_event_create(void** event);
int         cactus_hip_event_destroy(void* event);
int         cactus_hip_event_record(void* event, void* stream);
/* later work on `stream` waits for the event's last record (cross-stream
 * ordering; no reference counterpart) */
int         cactus_hip_stream_wait_event(void* stream, void* event);
int         cactus_hip_event_elapsed_ms(void* start, void* end, float* ms);
/* Stream capture into a HIP graph (the fused decode step is captured once
 * and replayed per token).  No reference counterpart. */
int         cactus_hip_graph_capture_begin(void* stream);
int         cactus_hip_graph_capture_end(void* stream, void** graph_exec);
int         cactus_hip_graph_launch(void* graph_exec, void* stream);
int         cactus_hip_graph_destroy(void* graph_exec);

/* ------------------------------------------------ a1: activation quantization */
/* cactus_fp16_max_abs (kernel/kernel.h:147, kernel_quants.cpp:196):
 * writes max|src| as one float to *out (device). */
int cactus_hip_fp16_max_abs(const uint16_t* src, size_t count, float* out, void* stream);
/* cactus_fp16_to_int8 (kernel/kernel.h:146, kernel_quants.cpp:158):
 * q = sat8(rne(clamp(x * (1/scale), -128, 127))); count%8 tail rounds ties away. */
int cactus_hip_fp16_to_int8(const uint16_t* src, int8_t* dst, size_t count, float scale,
                            void* stream);
/* quantize_activations_fp16_to_int8 (graph/graph_ops_nn.cpp:35-66) and
 * compute_quantize_activations_node (:78-127): per row m of x[M][K],
 * scales[m] = max(max|x|/127, 1e-10), codes as cactus_fp16_to_int8. */
int cactus_hip_quantize_activations(const uint16_t* x, int8_t* q, float* scales,
                                    size_t M, size_t K, void* stream);

/* ------------------------------------------------ a2/a3: grouped matmul */
/* cactus_matmul_int8 (kernel/kernel.h:43, kernel_gemm.cpp:128-327):
 *   C[m][n] = fp16( fma-chain over g ascending of (float)acc[m][n][g] * Bs[n][g]
 *                   , times A_scales[m] )
 * acc = exact int32 sum over group g of A[m][k]*B[n][k].
 * A [M][K] int8, A_scales [M] f32, B [N][K] int8 (pretransposed),
 * B_scales [N][K/group_size] fp16, C [M][N] fp16.  group_size must divide K
 * and be a multiple of 16. */
int cactus_hip_matmul_int8(const int8_t* A, const float* A_scales, const int8_t* B,
                           const uint16_t* B_scales, uint16_t* C, size_t M, size_t K,
                           size_t N, size_t group_size, void* stream);
/* cactus_matmul_int4 (kernel/kernel.h:47, kernel_gemm.cpp:329-529): B_packed
 * [N][K/2], byte n*K/2 + k/2 holds k even in the low nibble, k odd in the high
 * nibble, two's-complement 4-bit.  group_size as above (multiple of 32). */
int cactus_hip_matmul_int4(const int8_t* A, const float* A_scales, const uint8_t* B_packed,
                           const uint16_t* B_scales, uint16_t* C, size_t M, size_t K,
                           size_t N, size_t group_size, void* stream);
/* compute_matmul_node with FP16 lhs (graph/graph_ops_nn.cpp:129-231): the
 * activation quantization of cactus_hip_quantize_activations fused into the
 * matmul; results identical to the unfused pair. */
int cactus_hip_matmul_int8_f16act(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                  uint16_t* C, size_t M, size_t K, size_t N, size_t group_size,
                                  void* stream);
/* No counterpart in the reference.  cactus_hip_matmul_int8_f16act for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the same kernels
 * and results, with the activation codes and row scales of the MFMA path
 * (M >= 32) in a static 4 MiB device buffer instead of a buffer the library
 * allocates.  Rejects, with CACTUS_HIP_EINVAL and before any launch, shapes
 * whose ((M*K + 255) & ~255) + 4*M bytes exceed 4 MiB (e.g. M = 4096 at
 * K = 1024).  Calls no hipMalloc / hipFree.  Every call on one GPU shares
 * that GPU's buffer: calls that overlap on one GPU (two streams, two host
 * threads) race.  Each call rewrites every byte it reads, so nothing
 * carries over from the previous call. */
int cactus_hip_matmul_int8_f16act_noalloc(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                          uint16_t* C, size_t M, size_t K, size_t N, size_t group_size,
                                          void* stream);
int cactus_hip_matmul_int4_f16act(const uint16_t* A, const uint8_t* B_packed,
                                  const uint16_t* B_scales, uint16_t* C, size_t M, size_t K,
                                  size_t N, size_t group_size, void* stream);
/* No single reference function: a grouped matmul (cactus_matmul_int8 /
 * cactus_matmul_int4, or their FP16-activation forms) followed by the
 * residual add node (model_qwen.cpp:123 and :126, cactus_add_f16):
 * C = fp16(fp16(A x B) + residual), identical to the two nodes.  residual
 * is [M][N] fp16 and may not alias C. */
int cactus_hip_matmul_int8_add(const int8_t* A, const float* A_scales, const int8_t* B, const uint16_t* B_scales,
                               const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                               size_t group_size, void* stream);
int cactus_hip_matmul_int4_add(const int8_t* A, const float* A_scales, const uint8_t* B_packed,
                               const uint16_t* B_scales, const uint16_t* residual, uint16_t* C, size_t M, size_t K,
                               size_t N, size_t group_size, void* stream);
int cactus_hip_matmul_int8_f16act_add(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                      const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                                      size_t group_size, void* stream);
int cactus_hip_matmul_int4_f16act_add(const uint16_t* A, const uint8_t* B_packed, const uint16_t* B_scales,
                                      const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                                      size_t group_size, void* stream);
/* No single reference function: `count` (1..3) grouped matmuls that share one
 * pre-quantized activation, C[i] = A x B[i]^T as cactus_hip_matmul_int8
 * (int4 = 0, B[i] [N[i]][K] int8) or cactus_hip_matmul_int4 (int4 = 1,
 * B[i] [N[i]][K/2] packed), each identical to its own call.  The q/k/v and
 * gate/up projections of model_qwen.cpp:55-57 and :112-113 run as one
 * launch instead of three or two.  B, B_scales, C and N are host arrays of
 * `count` entries; M, K and group_size are shared. */
int cactus_hip_matmul_grouped_multi(const int8_t* A, const float* A_scales, size_t count, const void* const* B,
                                    const uint16_t* const* B_scales, uint16_t* const* C, const size_t* N, size_t M,
                                    size_t K, size_t group_size, int int4, void* stream);
/* Strided-batched form of cactus_hip_matmul_int8_f16act: `batch` independent
 * problems, problem i at A + i*stride_a, B + i*stride_b, B_scales +
 * i*stride_bs, C + i*stride_c (strides in elements).  No reference
 * counterpart: it lets one launch stream many distinct weight sets (layers,
 * experts, or a cache-defeating rotation). */
int cactus_hip_matmul_int8_f16act_batched(const uint16_t* A, const int8_t* B,
                                          const uint16_t* B_scales, uint16_t* C, size_t M,
                                          size_t K, size_t N, size_t group_size, size_t batch,
                                          size_t stride_a, size_t stride_b, size_t stride_bs,
                                          size_t stride_c, void* stream);
/* The same for cactus_hip_matmul_int4_f16act (stride_b in bytes of packed
 * weights, the other strides in elements).  No reference counterpart. */
int cactus_hip_matmul_int4_f16act_batched(const uint16_t* A, const uint8_t* B_packed,
                                          const uint16_t* B_scales, uint16_t* C, size_t M,
                                          size_t K, size_t N, size_t group_size, size_t batch,
                                          size_t stride_a, size_t stride_b, size_t stride_bs,
                                          size_t stride_c, void* stream);
/* cactus_unpack_int4_to_int8 (kernel/kernel.h:162, kernel_quants.cpp:295-351) */
int cactus_hip_unpack_int4_to_int8(const uint8_t* packed, int8_t* unpacked, size_t count,
                                   void* stream);

/* ------------------------------------------------ a4: FP16 matmul */
/* cactus_matmul_f16 (kernel/kernel.h:51, kernel_gemm.cpp:17-126): FP16
 * accumulation, 8 lanes (lane j takes k = j mod 8 in increasing k, fp16 fma),
 * final sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) in fp16.  a [M][K],
 * b_transposed [N][K], c [M][N]. */
int cactus_hip_matmul_f16(const uint16_t* a, const uint16_t* b_transposed, uint16_t* c,
                          size_t M, size_t K, size_t N, void* stream);
/* LM head + greedy sample fused (engine_model.cpp:241-247 then
 * cactus_sample_f16 greedy branch): logits = cactus_hip_matmul_f16(a[1][K],
 * b_transposed) written to `logits` (may be NULL) and token = argmax with
 * the first index winning ties. */
int cactus_hip_lm_head_argmax_f16(const uint16_t* a, const uint16_t* b_transposed,
                                  uint16_t* logits, uint32_t* token, size_t K, size_t N,
                                  void* stream);

/* ------------------------------------------------ a5/a6: attention */
/* cactus_attention_f16 (kernel/kernel.h:95, kernel_attention.cpp:10-255).
 * q [B][S][Hq][d], k/v [B][Skv][Hkv][d], o like q; mask (may be NULL)
 * [B][S][Skv] fp16, 0 = masked.  Reference order of operations: 32-key
 * blocks, running max = last block max, second-order 2^x weights for the
 * first floor(n/4)*4 keys of a block and expf for the rest. */
int cactus_hip_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* o, size_t batch, size_t seq_len, size_t kv_seq_len,
                             size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                             float scale, const uint16_t* mask, size_t position_offset,
                             size_t window_size, int is_causal, void* stream);
/* cactus_attention_hybrid_int8_fp16 (kernel/kernel.h:100,
 * kernel_attention.cpp:257-482): positions < cache_len read the INT8 cache
 * (k_cached/v_cached [B][cache_len][Hkv][d], scales [cache_len][Hkv][G] --
 * one scale table for every batch row, as kernel_attention.cpp:353,424 index it),
 * later positions read k_new/v_new [B][new_len][Hkv][d] fp16. expf weights. */
int cactus_hip_attention_hybrid_int8_fp16(const uint16_t* q, const int8_t* k_cached,
                                          const int8_t* v_cached, const float* k_scales,
                                          const float* v_scales, const uint16_t* k_new,
                                          const uint16_t* v_new, uint16_t* o, size_t batch,
                                          size_t seq_len, size_t cache_len, size_t new_len,
                                          size_t num_q_heads, size_t num_kv_heads,
                                          size_t head_dim, float scale, size_t position_offset,
                                          int is_causal, size_t quant_group_size, void* stream);
/* Tolerance-mode variants of the two attention entry points above (same
 * arguments and layouts; no reference counterpart of their own).  A decode
 * query (seq_len 1, causal, no mask, head_dim 64 or 128, 1, 2 or 4 query
 * heads per KV head; hybrid: quant_group_size >= head_dim) runs as a split-K
 * reduction over 256-key splits with one combine, so the launch is bound by
 * HBM bandwidth instead of the reference's sequential value accumulation.
 * The hybrid variant also takes prefill rows (seq_len > 1, causal, 16-byte
 * aligned rows, head_dim 64 or 128): they run as flash attention on FP16
 * MFMA.  Both are the same softmax attention with a different fp32
 * summation order and exponential: within |gpu - ref| <= 1e-3 + 1e-2 |ref|
 * of the reference per output, not bit-identical.  Where the reference's
 * block rescale overflows (a later block's max more than ~88 below an
 * earlier one makes its running accumulators infinite and the row comes out
 * zero, kernel_attention.cpp:395-403, 465-469) these variants return the
 * softmax instead.  Every other shape runs the exact kernels. */
int cactus_hip_attention_f16_fast(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  uint16_t* o, size_t batch, size_t seq_len, size_t kv_seq_len,
                                  size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                  float scale, const uint16_t* mask, size_t position_offset,
                                  size_t window_size, int is_causal, void* stream);
int cactus_hip_attention_hybrid_int8_fp16_fast(const uint16_t* q, const int8_t* k_cached,
                                               const int8_t* v_cached, const float* k_scales,
                                               const float* v_scales, const uint16_t* k_new,
                                               const uint16_t* v_new, uint16_t* o, size_t batch,
                                               size_t seq_len, size_t cache_len, size_t new_len,
                                               size_t num_q_heads, size_t num_kv_heads,
                                               size_t head_dim, float scale, size_t position_offset,
                                               int is_causal, size_t quant_group_size, void* stream);

/* ------------------------------------------------ a7: KV quantization */
/* No single reference function: an RMSNorm node (cactus_rms_norm_f16,
 * kernel_attention.cpp:484-563) whose output only feeds matmuls, fused with
 * those matmuls' per-row activation quantization (graph_ops_nn.cpp:35-66):
 * codes [M][K] and row scales [M], identical to cactus_hip_rms_norm_f16
 * followed by cactus_hip_quantize_activations.  K <= 32768. */
int cactus_hip_rms_norm_quantize_f16(const uint16_t* x, const uint16_t* weight, int8_t* q, float* scales,
                                     size_t M, size_t K, float eps, void* stream);
/* No single reference function: the per-head RMSNorm of q or k (the
 * q_norm / k_norm nodes, model_qwen.cpp:63-70, cactus_rms_norm_f16 over rows
 * of head_dim) followed by their RoPE (cactus_rope_f16, model_qwen.cpp:78-81)
 * on x [batch][seq][heads][head_dim]; identical to the two nodes. */
int cactus_hip_rms_norm_rope_f16(const uint16_t* x, const uint16_t* weight, uint16_t* y, size_t batch,
                                 size_t seq_len, size_t num_heads, size_t head_dim, size_t start_pos, float theta,
                                 float eps, void* stream);
/* No single reference function: the q and k head RMSNorm + RoPE nodes of
 * model_qwen.cpp:63-70 and :78-80 in one launch, each output identical to
 * cactus_hip_rms_norm_rope_f16 on that tensor alone.  q [batch][seq_len]
 * [q_heads][head_dim] and k [..][kv_heads][head_dim] with their own norm
 * weights; either head count may be 0. */
int cactus_hip_rms_norm_rope_qk_f16(const uint16_t* q, const uint16_t* q_weight, uint16_t* q_out, size_t q_heads,
                                    const uint16_t* k, const uint16_t* k_weight, uint16_t* k_out, size_t kv_heads,
                                    size_t batch, size_t seq_len, size_t head_dim, size_t start_pos, float theta,
                                    float eps, void* stream);
/* No single reference function: the SwiGLU nodes silu(gate) * up
 * (cactus_silu_f16, kernel_nn.cpp:12-44; cactus_multiply_f16,
 * kernel_blas.cpp:291-316) fused with the row quantization of the matmul
 * they feed: codes [M][K] and row scales [M], identical to the three nodes
 * (the silu tail rule counts over the whole [M][K] tensor).  K <= 32768. */
int cactus_hip_silu_mul_quantize_f16(const uint16_t* gate, const uint16_t* up, int8_t* q, float* scales,
                                     size_t M, size_t K, void* stream);
/* cactus_quantize_kv_fp16_to_int8 (kernel/kernel.h:150, kernel_quants.cpp:223-293)
 * src [S][Hkv][d] fp16 -> dst int8 same shape, scales [S][Hkv][ceil(d/g)] f32. */
int cactus_hip_quantize_kv_fp16_to_int8(const uint16_t* src, int8_t* dst, float* scales,
                                        size_t seq_len, size_t kv_heads, size_t head_dim,
                                        size_t group_size, void* stream);

/* ------------------------------------------------ a8-a12 */
/* cactus_rms_norm_f16 (kernel/kernel.h:79, kernel_attention.cpp:484-563) */
int cactus_hip_rms_norm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows,
                            size_t dims, float eps, void* stream);
/* cactus_rope_f16 (kernel/kernel.h:82, kernel_attention.cpp:565-676): NeoX
 * half-split pairing with fp16 cos/sin tables built on the host
 * (freq = 1/powf(theta, 2i/d), angle = pos*freq) and cached per device. */
int cactus_hip_rope_f16(const uint16_t* x, uint16_t* y, size_t batch, size_t seq_len,
                        size_t num_heads, size_t head_dim, size_t start_pos, float theta,
                        void* stream);
/* Grows the cached RoPE table to at least max_pos positions so that later
 * cactus_hip_rope_f16 calls up to that position do no host work (required
 * before capturing them into a HIP graph). */
int cactus_hip_rope_reserve(size_t max_pos, size_t head_dim, float theta);
/* cactus_softmax_f16 (kernel/kernel.h:85, kernel_nn.cpp:152-251) */
int cactus_hip_softmax_f16(const uint16_t* x, uint16_t* y, size_t batch, size_t seq_len,
                           size_t vocab, void* stream);
/* cactus_silu_f16 (kernel/kernel.h:88, kernel_nn.cpp:12-44) */
int cactus_hip_silu_f16(const uint16_t* x, uint16_t* y, size_t n, void* stream);
/* cactus_add_f16 / cactus_multiply_f16 (kernel/kernel.h:22,25, kernel_blas.cpp:187,291) */
int cactus_hip_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n,
                       void* stream);
int cactus_hip_multiply_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n,
                            void* stream);

/* cactus_transpose_2d_f16 (kernel/kernel.h:54, kernel_blas.cpp): dst[c][r] = src[r][c]
 * for src [rows][cols]; used by the graph for a non-pretransposed FP16 rhs. */
int cactus_hip_transpose_2d_f16(const uint16_t* src, uint16_t* dst, size_t rows, size_t cols,
                                void* stream);

/* ------------------------------------------------ a13/a14 */
/* compute_embedding_node, FP16 table with FP32 ids
 * (graph/graph_ops_tensor.cpp:301-329): out[i] = table[(size_t)ids[i]].
 * Out-of-range ids (the reference throws) produce zero rows and set
 * *error_flag = 1 when error_flag is non-NULL (device int). */
int cactus_hip_embedding_f16(const uint16_t* table, const float* ids, uint16_t* out,
                             size_t num_ids, size_t hidden, size_t vocab, int* error_flag,
                             void* stream);
/* cactus_sample_f16 (kernel/kernel.h:127, kernel_nn.cpp:446-651): greedy
 * (temperature == 0, top_p <= 0, top_k == 0: first index of the maximum) or
 * the full sampler: fp16 temperature scaling, the repetition penalty 1.1 over
 * the last 128 tokens this sampler returned (a history kept per device, like
 * the reference's process-wide one), top-k (ties at the k-th value kept),
 * top-p (the position whose running sum first exceeds top_p, after the
 * first, and everything after it removed), and the draw u from
 * std::mt19937(random_seed) (a random seed for 0) through libc++'s
 * generate_canonical<float, 24>.  The reference's logit bias never reaches
 * its result and has no argument here; the f16 sampler has no min-p.
 * Top-p works with any top_k (0: the whole vocabulary); the reference's
 * unspecified order of tied values is taken as ascending token where a tie
 * straddles the top-p cut.  Always writes a token id < vocab (0 when every
 * logit is -inf) as one uint32 to *out (device memory), stream-ordered. */
int cactus_hip_sample_f16(const uint16_t* logits, uint32_t* out, size_t vocab,
                          float temperature, float top_p, size_t top_k, size_t random_seed,
                          void* stream);
/* cactus_sample_f32 (kernel/kernel.h:130, kernel_nn.cpp:253-444): greedy
 * (temperature == 0, top_p <= 0, top_k == 0: first index of the maximum) or
 * the full FP32 sampler: the logit bias added entry by entry in order
 * (bias_values / bias_indices in host memory, at most 128 entries, else
 * CACTUS_HIP_EUNSUPPORTED), division by the temperature, top-k (ties at the
 * k-th value kept), min-p 0.15, top-p and the draw u from
 * std::mt19937(random_seed) (a random seed for 0) through libc++'s
 * generate_canonical<float, 24>.  No repetition penalty and no history.
 * Tied values straddling the top-p cut are taken in ascending token order.
 * Always writes a token id < vocab (0 when nothing survives) as one uint32
 * to *out (device memory), stream-ordered. */
int cactus_hip_sample_f32(const float* logits, uint32_t* out, size_t vocab, float temperature, float top_p,
                          size_t top_k, size_t random_seed, const float* bias_values,
                          const uint32_t* bias_indices, size_t bias_count, void* stream);
/* Model::decode's out_entropy (engine/engine_model.cpp:255-290): the
 * softmax entropy of fp16 logits [vocab] in double, divided by log(vocab),
 * written as one float to *out (device memory).  Floating point: within a
 * few float ulp of the reference's sequential double sums. */
int cactus_hip_logits_entropy_f16(const uint16_t* logits, size_t vocab, float* out, void* stream);
/* ---- ops of other model families (kernel.h, graph_ops_nn.cpp) ----------
 * cactus_gelu_f16 (kernel_nn.cpp:46-92): the 8-element body uses
 * fast_tanh_f32x4 (kernel_utils.h:143-163), the n % 8 tail tanhf. */
int cactus_hip_gelu_f16(const uint16_t* in, uint16_t* out, size_t n, void* stream);
/* cactus_gelu_f16_erf (kernel_nn.cpp:94-150) */
int cactus_hip_gelu_erf_f16(const uint16_t* in, uint16_t* out, size_t n, void* stream);
/* compute_layernorm_node, FP16 input / weight / bias / output
 * (graph_ops_nn.cpp:373-457): rows of `features` values */
int cactus_hip_layer_norm_f16(const uint16_t* x, const uint16_t* weight, const uint16_t* bias, uint16_t* y,
                              size_t rows, size_t features, float eps, void* stream);
/* cactus_conv1d_causal_depthwise_f16 (kernel_conv.cpp:15-110): input and
 * output [N][L][C], weight [C][K], y[t] = sum_k w[K-1-k] x[t - k*dilation] */
int cactus_hip_conv1d_causal_depthwise_f16(const uint16_t* input, const uint16_t* weight, uint16_t* output,
                                           size_t N, size_t L, size_t C, size_t K, size_t dilation,
                                           void* stream);
/* cactus_conv1d_f16_k3 (kernel_conv.cpp:112-236): input [N][C_in][L], weight
 * [C_out][C_in][3], output [N][C_out][(L-1)/stride + 1], zero padding 1 */
int cactus_hip_conv1d_f16_k3(const uint16_t* input, const uint16_t* weight, uint16_t* output, size_t N,
                             size_t L, size_t C_in, size_t C_out, size_t stride, void* stream);

/* No reference counterpart (the reference's history is a static vector in
 * kernel_nn.cpp:516): read back this device's sampler history (oldest
 * first, at most 128 entries; synchronises the stream) or clear it. */
int cactus_hip_sample_history(uint32_t* tokens, size_t* count, void* stream);
int cactus_hip_sample_history_reset(void* stream);

/* ------------------------------------------------ value product tiles
 * No reference counterpart: an fp32 mirror of the INT8 value cache holding
 * each cached (float)code * scale, the operand the hybrid attention's value
 * accumulation rounds to (kernel_attention.cpp:424-441), laid out
 * [kv head][64-dim slice][key / 4][64 dims][4 keys] (a slice's keys padded
 * to whole 64-key tiles) for the decode attention: one 16-byte load per
 * lane gives a dim's products of four consecutive keys.  Batch 1,
 * head_dim % 8 == 0, 128-dim scale groups. */
int cactus_hip_kv_shadow_bytes(size_t max_seq, size_t kv_heads, size_t head_dim, size_t* bytes);
/* products of cached keys [start, start + count) from the INT8 values and
 * scales ([max_seq][kv_heads][head_dim], [max_seq][kv_heads][groups]) */
int cactus_hip_kv_shadow_update(const int8_t* v_cache, const float* v_scales, float* shadow,
                                size_t start, size_t count, size_t kv_heads, size_t head_dim,
                                size_t quant_group_size, size_t max_seq, void* stream);

/* The sliding window's memmove (KVCache::update_from_graph,
 * engine/engine_cache.cpp:268-306, std::memmove on host vectors there) on the
 * device, for every layer at once: cached tokens [src, src + count) move to
 * [dst, dst + count) (dst <= src; the ranges may overlap) -- key and value
 * codes and scales -- and the value-product tiles of the moved tokens are
 * recomputed (records with shadow == NULL skip them).  `layers` is a DEVICE
 * array of nlayers records; caches are [max_seq][kv_heads][head_dim] codes
 * and [max_seq][kv_heads][ceil(head_dim/128)] scales.  `temp` is device
 * memory of cactus_hip_kv_shift_temp_bytes(nlayers, count, ...) bytes.
 * With state != NULL, state[2] (the decode step's cache length) is set to
 * cache_len after the move (also when count == 0). */
typedef struct {
    int8_t* k;
    int8_t* v;
    float* k_scales;
    float* v_scales;
    float* shadow;
} cactus_hip_kv_layer;
int cactus_hip_kv_shift_temp_bytes(size_t nlayers, size_t count, size_t kv_heads, size_t head_dim,
                                   size_t* bytes);
/* No single reference function: the cache append of engine_cache.cpp:131-267
 * (cactus_quantize_kv_fp16_to_int8 of each layer's new K and V rows,
 * kernel_quants.cpp:223-293) for every layer in one launch, with the value
 * products of cactus_hip_kv_shadow_update for records whose shadow is not
 * NULL; identical to those calls layer by layer.  `layers` is a DEVICE array
 * of nlayers records; k_rows / v_rows are HOST arrays of nlayers device
 * pointers to [count][kv_heads][head_dim] fp16 rows, written to cache slots
 * [at, at + count).  Quantization group 128 (the cache's). */
int cactus_hip_kv_append_layers(const cactus_hip_kv_layer* layers, const uint16_t* const* k_rows,
                                const uint16_t* const* v_rows, size_t nlayers, size_t count, size_t at,
                                size_t kv_heads, size_t head_dim, size_t group_size, size_t max_seq,
                                void* stream);
int cactus_hip_kv_window_shift(const cactus_hip_kv_layer* layers, size_t nlayers, size_t kv_heads,
                               size_t head_dim, size_t max_seq, size_t dst, size_t src, size_t count,
                               void* temp, size_t temp_bytes, uint32_t* state, uint32_t cache_len,
                               void* stream);

/* ------------------------------------------------ fused decode step
 * Each entry point computes a run of consecutive graph nodes of
 * QwenModel::forward (models/model_qwen.cpp:51-172) for ONE token with the
 * reference's arithmetic; there is no single reference function for any of
 * them.  `state` is a device uint32[4] = {token, position, cache_length,
 * step}, read (and, by the LM head, advanced) on the device so the whole
 * step can be captured into a HIP graph. */
/* h = embedding[state.token] */
int cactus_hip_decode_embed(const uint16_t* table, const uint32_t* state, uint16_t* h,
                            size_t hidden, size_t vocab, void* stream);
/* x = rms_norm(h, norm_w, eps); q|k|v = matmul(x, Wq|Wk|Wv) (grouped INT8) */
int cactus_hip_decode_qkv(const uint16_t* h, const uint16_t* norm_w, float eps, size_t K,
                          size_t group_size, const int8_t* wq, const uint16_t* sq, uint16_t* q,
                          size_t nq, const int8_t* wk, const uint16_t* sk, uint16_t* k, size_t nk,
                          const int8_t* wv, const uint16_t* sv, uint16_t* v, size_t nv,
                          void* stream);
/* h = h + matmul(x, W) (grouped INT8, or packed INT4 when int4 != 0) */
int cactus_hip_decode_matmul_residual(const uint16_t* x, size_t K, size_t group_size,
                                      const void* w, const uint16_t* s, size_t N, int int4,
                                      uint16_t* h, void* stream);
/* x = rms_norm(h); m = silu(matmul(x, Wg)) * matmul(x, Wu) (packed INT4) */
int cactus_hip_decode_mlp_up(const uint16_t* h, const uint16_t* norm_w, float eps, size_t K,
                             size_t group_size, const uint8_t* wg, const uint16_t* sg,
                             const uint8_t* wu, const uint16_t* su, size_t N, uint16_t* m,
                             void* stream);
/* q/k head RMSNorm, RoPE at state.position, INT8 append of k and v at
 * state.cache_length (128-dim groups); with v_shadow (may be null) also the
 * appended value row's product tiles (cactus_hip_kv_shadow_update) */
int cactus_hip_decode_attn_prep(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                float theta, const uint32_t* state, uint16_t* q_out,
                                uint16_t* k_out, int8_t* k_cache, int8_t* v_cache,
                                float* k_scales, float* v_scales, size_t max_cache,
                                float* v_shadow, void* stream);
/* cactus_hip_attention_hybrid_int8_fp16 for one token, cache length and
 * position from `state`; v_shadow (may be null): the value product tiles of
 * the cache, capacity max_cache, which the value chains then stream */
int cactus_hip_decode_attention(const uint16_t* q, const int8_t* k_cache, const int8_t* v_cache,
                                const float* k_scales, const float* v_scales,
                                const uint16_t* k_new, const uint16_t* v_new, uint16_t* o,
                                size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                float scale, const uint32_t* state, size_t max_cache,
                                const float* v_shadow, void* stream);
/* cactus_hip_decode_attn_prep followed by cactus_hip_decode_attention (k_new =
 * the prepared key, v_new = v_raw) with the head preparation done inside
 * the attention's score kernel: one kernel fewer per layer.  head_dim 64 or
 * 128, one or two query heads per KV head. */
int cactus_hip_decode_prep_attention(const uint16_t* q_raw, const uint16_t* k_raw,
                                     const uint16_t* v_raw, const uint16_t* q_norm,
                                     const uint16_t* k_norm, float eps, size_t num_q_heads,
                                     size_t num_kv_heads, size_t head_dim, float theta,
                                     const uint32_t* state, int8_t* k_cache, int8_t* v_cache,
                                     float* k_scales, float* v_scales, size_t max_cache,
                                     float* v_shadow, float scale, uint16_t* o, void* stream);
/* cactus_hip_decode_prep_attention with the tolerance-mode split-K attention
 * of cactus_hip_attention_hybrid_int8_fp16_fast (the head preparation and
 * the KV append are bit-identical to the exact form; the attention output
 * is within tolerance).  workspace: device memory of at least
 * cactus_hip_decode_attention_fast_workspace(...) bytes, 256-byte aligned,
 * zeroed once before first use (each launch leaves it reusable); one
 * workspace per stream. */
size_t cactus_hip_decode_attention_fast_workspace(size_t num_q_heads, size_t num_kv_heads,
                                                  size_t head_dim, size_t max_cache);
int cactus_hip_decode_prep_attention_fast(const uint16_t* q_raw, const uint16_t* k_raw,
                                          const uint16_t* v_raw, const uint16_t* q_norm,
                                          const uint16_t* k_norm, float eps, size_t num_q_heads,
                                          size_t num_kv_heads, size_t head_dim, float theta,
                                          const uint32_t* state, int8_t* k_cache, int8_t* v_cache,
                                          float* k_scales, float* v_scales, size_t max_cache,
                                          float* v_shadow, float scale, uint16_t* o, void* workspace,
                                          size_t workspace_bytes, void* stream);
/* token = argmax(matmul_f16(rms_norm(h), embedding)); writes tokens_out[step]
 * and advances state; logits_out (fp16 [N], or null) receives the logits
 * row.  scratch: >= 256 bytes, zeroed once (each call leaves it zeroed);
 * calls sharing a scratch buffer must not overlap. */
int cactus_hip_decode_lm_head(const uint16_t* h, const uint16_t* norm_w, float eps,
                              const uint16_t* embedding, size_t K, size_t N, uint32_t* state,
                              uint32_t* tokens_out, size_t max_steps, uint16_t* logits_out,
                              void* scratch, size_t scratch_bytes, void* stream);
/* No reference counterpart: the embedding [N][K] fp16 (the tied LM head)
 * copied step-major, [K/8][N rounded up to 64][8 values], rows past N zero,
 * so that one 16-byte load per lane of a wave (lane = row) reads 1 KB
 * contiguous and the waves of one k-step read one contiguous band.
 * K % 8 == 0, K <= 4096; pointers 16-byte aligned. */
int cactus_hip_lm_tiles_bytes(size_t K, size_t N, size_t* bytes);
int cactus_hip_lm_tiles_build(const uint16_t* embedding, size_t K, size_t N, uint16_t* tiles, void* stream);
/* cactus_hip_decode_lm_head over the tiles of cactus_hip_lm_tiles_build:
 * the same tokens, logits and state (h, norm_w and tiles 16-byte aligned).
 * scratch: >= 1024 + 8 * ceil(N / 640) bytes, zeroed once (each call leaves
 * its counters zeroed; the rest is written before it is read). */
int cactus_hip_decode_lm_head_tiled(const uint16_t* h, const uint16_t* norm_w, float eps,
                                    const uint16_t* tiles, size_t K, size_t N, uint32_t* state,
                                    uint32_t* tokens_out, size_t max_steps, uint16_t* logits_out,
                                    void* scratch, size_t scratch_bytes, void* stream);
/* cactus_hip_decode_lm_head_tiled that also writes the next step's input,
 * h_next = embedding[token] (the greedy token just chosen; zeros for a token
 * >= N, as cactus_hip_decode_embed), from the workgroup that finishes the
 * argmax, so a step replayed back to back needs no embedding launch of its
 * own (the first step of a run still takes cactus_hip_decode_embed).
 * h_next may be h.  embedding [N][K] fp16, the table the tiles were built
 * from; every pointer 16-byte aligned. */
int cactus_hip_decode_lm_head_tiled_embed(const uint16_t* h, const uint16_t* norm_w, float eps,
                                          const uint16_t* tiles, const uint16_t* embedding, size_t K, size_t N,
                                          uint32_t* state, uint32_t* tokens_out, size_t max_steps,
                                          uint16_t* logits_out, uint16_t* h_next, void* scratch,
                                          size_t scratch_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
