// attention_args.h -- launch arguments and key ranges shared by the exact
// attention kernels (attention.hip) and the decode value-chain kernel
// (chain_stream.hip).
#pragma once
#include "hip_common.h"

namespace cactus_hip {

constexpr int ATT_BLOCK = 32;
constexpr int ATT_MAX_D = 256;
constexpr int ATT_MAX_GQ = 8;      // query heads per KV head

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;        // FP16 keys [B][Skv][Hkv][d] or new keys [B][new][Hkv][d]
    const uint16_t* v;
    const int8_t* kc;         // INT8 cache [B][cache][Hkv][d]
    const int8_t* vc;
    const float* ks;          // [B][cache][Hkv][nqg]
    const float* vs;
    const uint16_t* mask;     // [B][S][Skv] or null
    uint16_t* o;
    float* w;                 // scratch: weights [B*S*Hq][wstride]
    float* bmax;              // scratch: block max [B*S*Hq][nbstride]
    float* bsum;              // scratch: block sums
    size_t wstride;
    int nbstride;
    int B, S, Hq, Hkv, d, gq;
    size_t Skv;               // FP16: kv_seq_len; hybrid: cache_len + new_len
    size_t cache_len, new_len;
    size_t pos_off, window;
    int causal, qgs, nqg;
    float scale;
    // decode-step form: when set, cache_len = dyn[2] and position_offset =
    // dyn[1] are read from device memory (the step state of the fused
    // decode path), and the launch is sized for max_cache keys
    const uint32_t* dyn;
    size_t max_cache;
    // fp32 value-product tiles of the INT8 cache (kv_shadow.hip), or null
    const float* vsh;
    size_t sh_ntile;
    // decode score grid mapped onto the XCDs (0: plain 2-D grid): workgroup
    // i runs on XCD i % 8, kv head h's workgroups on XCD h % 8; xcd_chunks
    // workgroups per (row group, kv head), xcd_rest row groups
    int xcd_chunks, xcd_rest;
    // decode scores: the query heads of a kv head split over this many
    // workgroups per key chunk (0 or 1: one workgroup takes all gq heads);
    // the workgroups of one chunk are consecutive within xcd_chunks
    int hsplit;
    // decode step with the head preparation fused into the scores (null
    // q_raw: q and the new key row come prepared in q and k): raw q / k / v
    // rows of the step, head RMSNorm weights, RoPE tables, and the cache
    // rows the new key and value are appended to
    struct {
        const uint16_t* q_raw; const uint16_t* k_raw; const uint16_t* v_raw;
        const uint16_t* q_norm; const uint16_t* k_norm;
        const uint16_t* cos_t; const uint16_t* sin_t;
        float eps;
        uint32_t table_pos;
        int8_t* kc; int8_t* vc; float* ks; float* vs; float* vsh;
    } prep;
};

__device__ __forceinline__ AttnArgs resolve(const AttnArgs& in) {
    AttnArgs a = in;
    if (a.dyn) {
        a.cache_len = a.dyn[2];
        a.pos_off = a.dyn[1];
        a.Skv = a.cache_len + a.new_len;
    }
    return a;
}

// sign bit set on a non-negative float: a flag carried by a block sum
__device__ __forceinline__ float set_sign(float x) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) | 0x80000000u);
}

__device__ __forceinline__ float lane_f(float v, int j) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j));
}

// Key range and block limit of query position qp (kernel_attention.cpp:78-96
// for FP16, :328-337 for the hybrid).
template <bool HYBRID>
__device__ __forceinline__ void kv_range(const AttnArgs& a, size_t qp, size_t& kv_start,
                                         size_t& kv_end, size_t& blk_limit) {
    const size_t aq = a.pos_off + qp;
    kv_start = 0;
    kv_end = a.Skv;
    blk_limit = a.Skv;
    if (!HYBRID) {
        if (a.window > 0 && a.window < a.Skv) {
            if (aq > a.window) kv_start = aq - a.window;
            if (a.causal && aq + 1 < kv_end) kv_end = aq + 1;
        } else if (a.causal && aq + 1 < kv_end) {
            kv_end = aq + 1;
        }
    } else {
        if (a.causal && aq + 1 < kv_end) kv_end = aq + 1;
        blk_limit = kv_end;
    }
}


// The decode value chains over the value product tiles (chain_stream.hip):
// one batch, at most two query rows and two new rows, head_dim <= 256,
// nbmax <= 1024 blocks.
int launch_chain_stream(const AttnArgs& a, int nbmax, void* stream);

}  // namespace cactus_hip
