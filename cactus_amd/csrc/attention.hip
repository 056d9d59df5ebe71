// attention.hip -- KV-cache attention (a5 FP16 KV, a6 INT8 cache + FP16 new)
// in the reference's order of operations (kernel_attention.cpp:10-482).
//
// One wave per (batch, query position, query head).  Keys are walked in the
// reference's 32-key blocks; for each block:
//   * lane j (< 32) runs the "low" FMA chains of key j's score (dims 8c+0..3)
//     and lane j+32 the "high" chains (dims 8c+4..7); the pair is combined as
//     (t0+t1)+(t2+t3) with t_l = low_l + high_l, then multiplied by `scale`;
//   * the block max becomes the running max (even when smaller), the running
//     sum and accumulators are rescaled by expf(old_max - block_max);
//   * weights are the second-order 2^x polynomial for the first
//     floor(n/4)*4 keys and expf for the rest (FP16 variant), or expf for all
//     keys (hybrid variant); the block sum adds ((y0+y1)+(y2+y3)) per group of
//     four in order, then the tail;
//   * each lane owns head_dim/64 output dims and applies acc = fma(v, w, acc)
//     key by key in increasing position.
// Output = fp16(acc * (1/sum)) on the 8-aligned prefix of head_dim, zero
// elsewhere or when the sum is not positive.
#include "hip_common.h"

namespace cactus_hip {

constexpr int ATT_BLOCK = 32;
constexpr int ATT_MAX_D = 256;
constexpr int ATT_DPL = ATT_MAX_D / 64;   // max dims per lane

// value of v in lane j (j wave-uniform), via v_readlane_b32
__device__ __forceinline__ float lane_f(float v, int j) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), j));
}

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
    int B, S, Hq, Hkv, d;
    size_t Skv;               // FP16: kv_seq_len; hybrid: cache_len + new_len
    size_t cache_len, new_len;
    size_t pos_off, window;
    int causal, qgs, nqg;
    float scale;
};

template <bool HYBRID>
__global__ void __launch_bounds__(256) attention_ref_kernel(AttnArgs a) {
    __shared__ float qsh[4][ATT_MAX_D];
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t item = (size_t)blockIdx.x * 4 + wid;
    const size_t total = (size_t)a.B * a.S * a.Hq;
    const bool live = item < total;
    // work order of the reference: batch, then head, then query position
    const size_t b = live ? item / ((size_t)a.Hq * a.S) : 0;
    const size_t rem = live ? item % ((size_t)a.Hq * a.S) : 0;
    const int h = (int)(rem / a.S);
    const size_t qp = rem % a.S;
    const int kvh = h / (a.Hq / a.Hkv);
    const int d = a.d, da = (d / 8) * 8;
    float* qs = qsh[wid];
    const uint16_t* qv = a.q + ((b * a.S + qp) * a.Hq + h) * (size_t)d;
    if (live)
        for (int i = lane; i < d; i += 64) qs[i] = h2f(qv[i]);
    __syncthreads();
    if (!live) return;

    const bool high = lane >= 32;
    const int jl = lane & 31;
    const size_t aq = a.pos_off + qp;
    const bool is_decode = (!HYBRID) && (qp == (size_t)a.S - 1) && a.S > 1;
    size_t kv_start = 0, kv_end = a.Skv, blk_limit = a.Skv;
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

    float acc[ATT_DPL];
#pragma unroll
    for (int i = 0; i < ATT_DPL; i++) acc[i] = 0.0f;
    float rmax = -__builtin_inff(), rsum = 0.0f;
    const float NEG_INF = -__builtin_inff();

    for (size_t bs0 = kv_start; bs0 < kv_end; bs0 += ATT_BLOCK) {
        const size_t be = (bs0 + ATT_BLOCK < blk_limit) ? bs0 + ATT_BLOCK : blk_limit;
        const int bsz = (int)(be - bs0);
        if (!HYBRID && !is_decode && a.causal && bs0 > aq) continue;
        // ---- scores: lane jl computes key bs0+jl, low or high half
        const size_t kp = bs0 + jl;
        bool masked = jl >= bsz;
        if (!masked && a.causal && kp > aq && (HYBRID || !is_decode)) masked = true;
        float c[4] = {0.f, 0.f, 0.f, 0.f};
        if (!masked) {
            const int off = high ? 4 : 0;
            if (HYBRID && kp < a.cache_len) {
                const int8_t* kr = a.kc + ((b * a.cache_len + kp) * a.Hkv + kvh) * (size_t)d;
                const float* sr = a.ks + ((b * a.cache_len + kp) * a.Hkv + kvh) * (size_t)a.nqg;
                for (int cb = 0; cb < da; cb += 8) {
                    const float s = sr[cb / a.qgs];
                    const uint32_t w = *reinterpret_cast<const uint32_t*>(kr + cb + off);
#pragma unroll
                    for (int l = 0; l < 4; l++) {
                        const float kk = (float)(int8_t)((w >> (8 * l)) & 0xFF) * s;
                        c[l] = __builtin_fmaf(qs[cb + off + l], kk, c[l]);
                    }
                }
            } else {
                const size_t kpos = HYBRID ? kp - a.cache_len : kp;
                const size_t klen = HYBRID ? a.new_len : a.Skv;
                const uint16_t* kr = a.k + ((b * klen + kpos) * a.Hkv + kvh) * (size_t)d;
                for (int cb = 0; cb < da; cb += 8) {
                    const uint2 w = *reinterpret_cast<const uint2*>(kr + cb + off);
                    c[0] = __builtin_fmaf(qs[cb + off + 0], h2f((uint16_t)(w.x & 0xFFFF)), c[0]);
                    c[1] = __builtin_fmaf(qs[cb + off + 1], h2f((uint16_t)(w.x >> 16)), c[1]);
                    c[2] = __builtin_fmaf(qs[cb + off + 2], h2f((uint16_t)(w.y & 0xFFFF)), c[2]);
                    c[3] = __builtin_fmaf(qs[cb + off + 3], h2f((uint16_t)(w.y >> 16)), c[3]);
                }
            }
        }
        // combine low (lane jl) with high (lane jl+32)
        float hi0 = __shfl(c[0], jl + 32, 64), hi1 = __shfl(c[1], jl + 32, 64);
        float hi2 = __shfl(c[2], jl + 32, 64), hi3 = __shfl(c[3], jl + 32, 64);
        float score = NEG_INF;
        if (!high && !masked) {
            const float t0 = c[0] + hi0, t1 = c[1] + hi1, t2 = c[2] + hi2, t3 = c[3] + hi3;
            float s = (t0 + t1) + (t2 + t3);
            if (!HYBRID) {
                // dims beyond the 8-aligned prefix (kernel_attention.cpp:139-141)
                const uint16_t* kr = a.k + ((b * a.Skv + kp) * a.Hkv + kvh) * (size_t)d;
                for (int i = da; i < d; i++) s = __builtin_fmaf(qs[i], h2f(kr[i]), s);
            }
            s = s * a.scale;
            if (!HYBRID) {
                if (a.causal && kp > aq) s = NEG_INF;
                else if (a.window > 0 && kp < aq && (aq - kp) > a.window) s = NEG_INF;
                else if (a.mask && h2f(a.mask[(b * a.S + qp) * a.Skv + kp]) == 0.0f) s = NEG_INF;
            }
            score = s;
        }
        // ---- block max (lanes 0..31 hold scores, others -inf)
        const float bmax = wave_max(score);
        if (bmax > NEG_INF) {
            const float corr = cactus_expf(rmax - bmax);
            rsum = rsum * corr;
#pragma unroll
            for (int i = 0; i < ATT_DPL; i++) acc[i] = acc[i] * corr;
            rmax = bmax;
        }
        // ---- weights
        float w = 0.0f;
        const int vs4 = HYBRID ? 0 : (bsz / 4) * 4;
        if (!high && jl < bsz) {
            if (jl < vs4) w = poly_exp_weight(score, bmax);
            else w = (score != NEG_INF) ? cactus_expf(score - bmax) : 0.0f;
        }
        // block sum: ((y0+y1)+(y2+y3)) per group of four in order, then the
        // tail; weights are broadcast from lane j with v_readlane
        float bsum = 0.0f;
        for (int j = 0; j < vs4; j += 4) {
            const float y0 = lane_f(w, j), y1 = lane_f(w, j + 1);
            const float y2 = lane_f(w, j + 2), y3 = lane_f(w, j + 3);
            bsum = bsum + ((y0 + y1) + (y2 + y3));
        }
        for (int j = vs4; j < bsz; j++) bsum = bsum + lane_f(w, j);
        // ---- weighted values
        for (int j = 0; j < bsz; j++) {
            const float wj = lane_f(w, j);
            if (wj == 0.0f) continue;
            const size_t vp = bs0 + j;
            if (HYBRID && vp < a.cache_len) {
                const int8_t* vr = a.vc + ((b * a.cache_len + vp) * a.Hkv + kvh) * (size_t)d;
                const float* sr = a.vs + ((b * a.cache_len + vp) * a.Hkv + kvh) * (size_t)a.nqg;
#pragma unroll
                for (int i = 0; i < ATT_DPL; i++) {
                    const int dim = lane + 64 * i;
                    if (dim < da) {
                        const float vv = (float)vr[dim] * sr[((dim / 8) * 8) / a.qgs];
                        acc[i] = __builtin_fmaf(vv, wj, acc[i]);
                    }
                }
            } else {
                const size_t vpos = HYBRID ? vp - a.cache_len : vp;
                const size_t vlen = HYBRID ? a.new_len : a.Skv;
                const uint16_t* vr = a.v + ((b * vlen + vpos) * a.Hkv + kvh) * (size_t)d;
#pragma unroll
                for (int i = 0; i < ATT_DPL; i++) {
                    const int dim = lane + 64 * i;
                    if (dim < da) acc[i] = __builtin_fmaf(h2f(vr[dim]), wj, acc[i]);
                }
            }
        }
        rsum = rsum + bsum;
    }

    uint16_t* ov = a.o + ((b * a.S + qp) * a.Hq + h) * (size_t)d;
    if (rsum > 0.0f) {
        const float inv = 1.0f / rsum;
#pragma unroll
        for (int i = 0; i < ATT_DPL; i++) {
            const int dim = lane + 64 * i;
            if (dim < d) ov[dim] = dim < da ? f2h(acc[i] * inv) : (uint16_t)0;
        }
    } else {
        for (int dim = lane; dim < d; dim += 64) ov[dim] = 0;
    }
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                             size_t batch, size_t seq_len, size_t kv_seq_len, size_t num_q_heads,
                             size_t num_kv_heads, size_t head_dim, float scale,
                             const uint16_t* mask, size_t position_offset, size_t window_size,
                             int is_causal, void* stream) {
    if (batch == 0 || seq_len == 0 || num_q_heads == 0 || head_dim == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(q && o && (kv_seq_len == 0 || (k && v)), "attention_f16: null pointer");
    CH_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "attention_f16: num_q_heads must be a multiple of num_kv_heads");
    CH_REQUIRE(head_dim <= (size_t)ATT_MAX_D, "attention_f16: head_dim > 256 not supported");
    CH_REQUIRE(head_dim % 4 == 0, "attention_f16: head_dim must be a multiple of 4");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    AttnArgs a{};
    a.q = q; a.k = k; a.v = v; a.o = o; a.mask = mask;
    a.B = (int)batch; a.S = (int)seq_len; a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads;
    a.d = (int)head_dim; a.Skv = kv_seq_len; a.pos_off = position_offset; a.window = window_size;
    a.causal = is_causal ? 1 : 0; a.scale = scale; a.qgs = 1; a.nqg = 1;
    const size_t items = batch * seq_len * num_q_heads;
    hipLaunchKernelGGL(attention_ref_kernel<false>, dim3(ceil_div(items, 4)), dim3(256), 0,
                       as_stream(stream), a);
    return check_launch("attention_f16");
}

int cactus_hip_attention_hybrid_int8_fp16(const uint16_t* q, const int8_t* k_cached,
                                          const int8_t* v_cached, const float* k_scales,
                                          const float* v_scales, const uint16_t* k_new,
                                          const uint16_t* v_new, uint16_t* o, size_t batch,
                                          size_t seq_len, size_t cache_len, size_t new_len,
                                          size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                          float scale, size_t position_offset, int is_causal,
                                          size_t quant_group_size, void* stream) {
    if (batch == 0 || seq_len == 0 || num_q_heads == 0 || head_dim == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(q && o, "attention_hybrid: null pointer");
    CH_REQUIRE(cache_len == 0 || (k_cached && v_cached && k_scales && v_scales),
               "attention_hybrid: null cache pointer");
    CH_REQUIRE(new_len == 0 || (k_new && v_new), "attention_hybrid: null new K/V pointer");
    CH_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
               "attention_hybrid: num_q_heads must be a multiple of num_kv_heads");
    CH_REQUIRE(head_dim <= (size_t)ATT_MAX_D && head_dim % 8 == 0,
               "attention_hybrid: head_dim must be a multiple of 8 and <= 256");
    CH_REQUIRE(quant_group_size > 0, "attention_hybrid: quant_group_size must be > 0");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    AttnArgs a{};
    a.q = q; a.k = k_new; a.v = v_new; a.kc = k_cached; a.vc = v_cached; a.ks = k_scales;
    a.vs = v_scales; a.o = o;
    a.B = (int)batch; a.S = (int)seq_len; a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads;
    a.d = (int)head_dim; a.Skv = cache_len + new_len; a.cache_len = cache_len; a.new_len = new_len;
    a.pos_off = position_offset; a.causal = is_causal ? 1 : 0; a.scale = scale;
    a.qgs = (int)quant_group_size;
    a.nqg = (int)((head_dim + quant_group_size - 1) / quant_group_size);
    const size_t items = batch * seq_len * num_q_heads;
    hipLaunchKernelGGL(attention_ref_kernel<true>, dim3(ceil_div(items, 4)), dim3(256), 0,
                       as_stream(stream), a);
    return check_launch("attention_hybrid");
}

}  // extern "C"
