// sample.hip -- the FP16 sampler (a14 greedy, and the full sampler of
// kernel_nn.cpp:446-651): temperature, repetition penalty over the last 128
// sampled tokens, top-k, top-p and the draw, in one workgroup; and the FP32
// sampler (kernel_nn.cpp:253-444, the one with the logit bias and min-p).
//
// Phases (one 1024-thread workgroup, vocabulary in a scratch copy):
//   1. f = fp16(logit * fp16(1/T)) (or the raw logits); thread 0 applies the
//      repetition penalty entry by entry in history order (duplicates apply
//      again, as in the reference's loop);
//   2. top-k: the k-th largest value by a two-pass radix select over
//      order-preserving 16-bit keys (high byte, then low byte, LDS
//      histograms); values below it become -inf;
//   3. top-p: the survivors are sorted descending by a bitonic sort in LDS
//      (up to SP_CAND of them; more go through topp_large's global sort)
//      (ties: ascending token, see the oracle), thread 0
//      forms the probabilities and the running sum in that order and every
//      position from the first j > 0 whose sum exceeds top_p is removed;
//   4. the final probabilities over the survivors in token order: parallel
//      expf, an order-preserving compaction, then thread 0 sums, normalises
//      and walks the running sum to the first value >= u, and appends the
//      token to the device-resident history.
// The sequential float sums run by one thread over the survivors only
// (probabilities of removed tokens are exactly 0 and add nothing), so with
// top-k they are short; without any filter they cover the vocabulary.
#include "hip_common.h"

#include <map>
#include <mutex>
#include <random>

namespace cactus_hip {

constexpr int SP_T = 1024;
constexpr int SP_CAND = 16384;         // top-p candidates sorted in LDS; more take the global sort
constexpr int SP_HIST = 128;           // kernel_nn.cpp:517
constexpr uint16_t SP_NEG_INF = 0xFC00u;

// ---------------------------------------------------------------- greedy
// First index of the maximum of (float)logit (kernel_nn.cpp:451-466, and
// :258-273 for FP32 logits): each thread scans an increasing index range
// keeping a strict '>' winner; the combine takes the larger value and, on
// equal values, the smaller index.
__device__ __forceinline__ float logit_f(uint16_t h) { return h2f(h); }
__device__ __forceinline__ float logit_f(float x) { return x; }

template <typename T>
__global__ void __launch_bounds__(1024) argmax_kernel(const T* __restrict__ L, size_t V, uint32_t* out) {
    __shared__ float bv_s[1024];
    __shared__ uint32_t bi_s[1024];
    const int tid = threadIdx.x;
    const size_t per = (V + 1023) / 1024;
    const size_t s0 = tid * per;
    const size_t s1 = (s0 + per < V) ? s0 + per : V;
    float bv = -__builtin_inff();
    uint32_t bi = 0xFFFFFFFFu;
    for (size_t i = s0; i < s1; i++) {
        const float v = logit_f(L[i]);
        if (bi == 0xFFFFFFFFu || v > bv) { bv = v; bi = (uint32_t)i; }
    }
    bv_s[tid] = bv;
    bi_s[tid] = bi;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if (tid < w) {
            const float ov = bv_s[tid + w];
            const uint32_t oi = bi_s[tid + w];
            const float mv = bv_s[tid];
            const uint32_t mi = bi_s[tid];
            bool take;
            if (oi == 0xFFFFFFFFu) take = false;
            else if (mi == 0xFFFFFFFFu) take = true;
            else take = (ov > mv) || (ov == mv && oi < mi);
            if (take) { bv_s[tid] = ov; bi_s[tid] = oi; }
        }
        __syncthreads();
    }
    if (tid == 0) *out = (bi_s[0] == 0xFFFFFFFFu) ? 0u : bi_s[0];
}

// ---------------------------------------------------------------- full sampler
struct SampleArgs {
    const uint16_t* logits;
    uint32_t* out;
    uint16_t* f;        // [V] filtered logits
    float* pv;          // [V] unnormalised probabilities of the survivors
    uint32_t* surv;     // [V] survivor tokens in order
    uint32_t* sk;       // [next_pow2(V)] order keys of a large top-p
    uint32_t* hist;     // [1 + SP_HIST]: count, tokens
    size_t V, top_k;
    float top_p, u;
    uint16_t inv_t;     // fp16(1/T)
    uint16_t pen_inv, pen;
    int scale;          // temperature > 0
};

// order-preserving key of an fp16 value (non-NaN; -0 folded onto +0)
__device__ __forceinline__ uint32_t okey(uint16_t h) {
    if (h == 0x8000u) h = 0;
    return (h & 0x8000u) ? (~(uint32_t)h & 0xFFFFu) : ((uint32_t)h | 0x8000u);
}
__device__ __forceinline__ uint16_t ukey(uint32_t k) {
    return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)(~k & 0xFFFFu);
}
// the same for fp32 values
__device__ __forceinline__ uint32_t okey32(float x) {
    uint32_t u = __float_as_uint(x);
    if (u == 0x80000000u) u = 0;   // -0 == +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ bool is_inf(float x) { return x == __builtin_inff() || x == -__builtin_inff(); }

// ---------------------------------------------------------------- large top-p
// More top-p candidates than the LDS sort holds (top_k 0 or large, a flat
// distribution): their order keys (ascending key = descending value) are
// sorted in a global buffer by a bitonic sort whose strides below one LDS
// chunk run per chunk in LDS; thread 0 sums the probabilities in sorted
// order and walks the running sum to the cut, reading the sorted arrays
// chunk by chunk through LDS; then a token-order pass removes every
// candidate past the cut: all keys beyond the cut key, and the cut key's
// ties past the kept count in ascending token order (the reference's
// std::sort leaves the order of ties unspecified; the oracle's is
// ascending token, as in the LDS path).
constexpr uint32_t TP_CHUNK = SP_CAND * 2;   // 32-bit entries per LDS chunk (the 128 KB candidate buffer)

struct TopPF16 {
    uint16_t* f;
    __device__ bool removed(size_t i) const { return f[i] == SP_NEG_INF; }
    __device__ uint32_t key(size_t i) const { return 0xFFFFu - okey(f[i]); }
    __device__ float value(uint32_t k) const { return h2f(ukey(0xFFFFu - k)); }
    __device__ void remove(size_t i) const { f[i] = SP_NEG_INF; }
};
struct TopPF32 {
    float* f;
    __device__ bool removed(size_t i) const { return is_inf(f[i]); }
    __device__ uint32_t key(size_t i) const { return ~okey32(f[i]); }
    __device__ float value(uint32_t k) const {
        const uint32_t o = ~k;
        return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
    }
    __device__ void remove(size_t i) const { f[i] = -__builtin_inff(); }
};

// compare-exchange of the pair (lo, lo + stride) for pair index p, into
// ascending order where (index & size) == 0
__device__ __forceinline__ void bitonic_pair(uint32_t* x, uint32_t p, uint32_t stride, uint32_t size,
                                             uint32_t base) {
    const uint32_t lo = 2 * p - (p & (stride - 1)), hi = lo + stride;
    const bool up = ((base + lo) & size) == 0;
    const uint32_t u = x[lo], v = x[hi];
    if ((u > v) == up) {
        x[lo] = v;
        x[hi] = u;
    }
}

// ascending sort of sk[0, n2), n2 a power of two (one workgroup)
__device__ void bitonic_sort_global(uint32_t* sk, uint32_t n2, uint32_t* lds) {
    const uint32_t tid = threadIdx.x;
    const uint32_t C = n2 < TP_CHUNK ? n2 : TP_CHUNK;
    auto chunk_stages = [&](uint32_t base, uint32_t size_lo, uint32_t size_hi, uint32_t stride_hi) {
        for (uint32_t i = tid; i < C; i += SP_T) lds[i] = sk[base + i];
        __syncthreads();
        for (uint32_t size = size_lo; size <= size_hi; size <<= 1)
            for (uint32_t stride = min(size >> 1, stride_hi); stride > 0; stride >>= 1) {
                for (uint32_t p = tid; p < C / 2; p += SP_T) bitonic_pair(lds, p, stride, size, base);
                __syncthreads();
            }
        for (uint32_t i = tid; i < C; i += SP_T) sk[base + i] = lds[i];
        __syncthreads();
    };
    for (uint32_t base = 0; base < n2; base += C) chunk_stages(base, 2, C, C);
    for (uint32_t size = 2 * C; size <= n2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride >= C; stride >>= 1) {
            for (uint32_t p = tid; p < n2 / 2; p += SP_T) bitonic_pair(sk, p, stride, size, 0);
            __syncthreads();
        }
        for (uint32_t base = 0; base < n2; base += C) chunk_stages(base, size, size, C >> 1);
    }
}

// top-p over the V entries of ops that are not removed, n of them
// (n > SP_CAND); sk holds next_pow2(V) entries, pv V floats (scratch)
template <class Ops>
__device__ void topp_large(const Ops& ops, size_t V, float top_p, uint32_t* sk, float* pv, uint32_t* lds,
                           uint32_t* scan) {
    __shared__ uint32_t tp[4];
    const uint32_t tid = threadIdx.x;
    if (tid == 0) tp[0] = 0;
    __syncthreads();
    for (size_t i = tid; i < V; i += SP_T)
        if (!ops.removed(i)) sk[atomicAdd(&tp[0], 1u)] = ops.key(i);
    __syncthreads();
    const uint32_t n = tp[0];
    uint32_t n2 = 1;
    while (n2 < n) n2 <<= 1;
    for (uint32_t j = n + tid; j < n2; j += SP_T) sk[j] = 0xFFFFFFFFu;
    __syncthreads();
    bitonic_sort_global(sk, n2, lds);

    // probabilities in sorted order, their sum by thread 0 in that order
    const float mx = ops.value(sk[0]);
    for (uint32_t j = tid; j < n; j += SP_T) pv[j] = cactus_expf(ops.value(sk[j]) - mx);
    __syncthreads();
    float* fl = reinterpret_cast<float*>(lds);
    float sum = 0.0f;
    for (uint32_t c0 = 0; c0 < n; c0 += TP_CHUNK) {
        const uint32_t m = min(TP_CHUNK, n - c0);
        for (uint32_t j = tid; j < m; j += SP_T) fl[j] = pv[c0 + j];
        __syncthreads();
        if (tid == 0)
            for (uint32_t j = 0; j < m; j++) sum += fl[j];
        __syncthreads();
    }
    if (tid == 0) {
        tp[1] = __float_as_uint(sum);
        tp[2] = n;   // the cut: first position removed
    }
    __syncthreads();
    sum = __uint_as_float(tp[1]);
    for (uint32_t j = tid; j < n; j += SP_T) pv[j] = pv[j] / sum;
    __syncthreads();
    // the running sum; the first position j > 0 past top_p is the cut
    float cum = 0.0f;
    for (uint32_t c0 = 0; c0 < n && tp[2] == n; c0 += TP_CHUNK) {
        const uint32_t m = min(TP_CHUNK, n - c0);
        for (uint32_t j = tid; j < m; j += SP_T) fl[j] = pv[c0 + j];
        __syncthreads();
        if (tid == 0)
            for (uint32_t j = 0; j < m; j++) {
                cum += fl[j];
                if (cum > top_p && c0 + j > 0) {
                    tp[2] = c0 + j;
                    break;
                }
            }
        __syncthreads();
    }
    const uint32_t cut = tp[2];
    if (cut >= n) return;
    const uint32_t kc = sk[cut];
    if (tid == 0) {
        uint32_t lo = 0, hi = cut;   // first position of the cut key
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (sk[mid] < kc) lo = mid + 1;
            else hi = mid;
        }
        tp[3] = cut - lo;   // ties of the cut key that stay
    }
    __syncthreads();
    const uint32_t keep = tp[3];
    const size_t per = (V + SP_T - 1) / SP_T;
    const size_t t0 = (size_t)tid * per, t1 = t0 + per < V ? t0 + per : V;
    uint32_t cnt = 0;
    for (size_t i = t0; i < t1; i++) cnt += !ops.removed(i) && ops.key(i) == kc;
    scan[tid] = cnt;
    __syncthreads();
    for (uint32_t o = 1; o < SP_T; o <<= 1) {   // inclusive scan
        const uint32_t v = tid >= o ? scan[tid - o] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t rank = scan[tid] - cnt;
    for (size_t i = t0; i < t1; i++) {
        if (ops.removed(i)) continue;
        const uint32_t k = ops.key(i);
        if (k > kc) {
            ops.remove(i);
        } else if (k == kc) {
            if (rank >= keep) ops.remove(i);
            rank++;
        }
    }
    __syncthreads();
}

__global__ void __launch_bounds__(SP_T) sample_kernel(SampleArgs a) {
    extern __shared__ unsigned long long cand[];   // [SP_CAND], dynamic: 128 KB
    __shared__ uint32_t hbin[256];
    __shared__ uint32_t scan[SP_T];
    __shared__ float red[SP_T / 64];
    __shared__ uint32_t sh_u32[4];
    const int tid = threadIdx.x;
    const size_t V = a.V;

    // 1. temperature, then the repetition penalty (kernel_nn.cpp:501-529)
    for (size_t i = tid; i < V; i += SP_T) a.f[i] = a.scale ? hmul(a.logits[i], a.inv_t) : a.logits[i];
    __syncthreads();
    if (tid == 0) {
        const uint32_t n = a.hist[0];
        for (uint32_t j = 0; j < n; j++) {
            const uint32_t t = a.hist[1 + j];
            if (t < V) a.f[t] = h2f(a.f[t]) > 0.0f ? hmul(a.f[t], a.pen_inv) : hmul(a.f[t], a.pen);
        }
    }
    __syncthreads();

    // 2. top-k (:531-548): the k-th largest value, two radix passes
    if (a.top_k > 0 && a.top_k < V) {
        uint32_t prefix = 0, need = (uint32_t)a.top_k;
        for (int pass = 0; pass < 2; pass++) {
            if (tid < 256) hbin[tid] = 0;
            __syncthreads();
            for (size_t i = tid; i < V; i += SP_T) {
                const uint32_t k = okey(a.f[i]);
                if (pass == 0) atomicAdd(&hbin[k >> 8], 1u);
                else if ((k >> 8) == prefix) atomicAdd(&hbin[k & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t cum = 0;
                int b = 255;
                for (; b > 0; b--) {
                    if (cum + hbin[b] >= need) break;
                    cum += hbin[b];
                }
                sh_u32[0] = (uint32_t)b;
                sh_u32[1] = need - cum;
            }
            __syncthreads();
            prefix = pass == 0 ? sh_u32[0] : ((prefix << 8) | sh_u32[0]);
            need = sh_u32[1];
            __syncthreads();
        }
        const uint32_t kth = prefix;
        for (size_t i = tid; i < V; i += SP_T)
            if (okey(a.f[i]) < kth) a.f[i] = SP_NEG_INF;
        __syncthreads();
    }

    // 3. top-p (:550-590) over the survivors, sorted descending
    if (a.top_p > 0.0f && a.top_p < 1.0f) {
        if (tid == 0) sh_u32[2] = 0;
        __syncthreads();
        for (size_t i = tid; i < V; i += SP_T) {
            if (a.f[i] == SP_NEG_INF) continue;
            const uint32_t slot = atomicAdd(&sh_u32[2], 1u);
            if (slot < (uint32_t)SP_CAND)
                cand[slot] = ((unsigned long long)(0xFFFFu - okey(a.f[i])) << 32) | (unsigned long long)i;
        }
        __syncthreads();
        const uint32_t n = sh_u32[2];
        if (n > (uint32_t)SP_CAND) {
            topp_large(TopPF16{a.f}, V, a.top_p, a.sk, a.pv, reinterpret_cast<uint32_t*>(cand), scan);
        } else {
        uint32_t n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (uint32_t j = n + tid; j < n2; j += SP_T) cand[j] = ~0ull;
        __syncthreads();
        for (uint32_t size = 2; size <= n2; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = tid; i < n2; i += SP_T) {
                    const uint32_t j = i ^ stride;
                    if (j > i) {
                        const bool up = (i & size) == 0;
                        const unsigned long long x = cand[i], y = cand[j];
                        if ((x > y) == up) {
                            cand[i] = y;
                            cand[j] = x;
                        }
                    }
                }
                __syncthreads();
            }
        }
        if (tid == 0) {
            uint32_t cut = n;
            if (n > 0) {
                const float mx = h2f(ukey(0xFFFFu - (uint32_t)(cand[0] >> 32)));
                float sum = 0.0f;
                for (uint32_t j = 0; j < n; j++) sum += cactus_expf(h2f(ukey(0xFFFFu - (uint32_t)(cand[j] >> 32))) - mx);
                float cum = 0.0f;
                for (uint32_t j = 0; j < n; j++) {
                    cum += cactus_expf(h2f(ukey(0xFFFFu - (uint32_t)(cand[j] >> 32))) - mx) / sum;
                    if (cum > a.top_p && j > 0) {
                        cut = j;
                        break;
                    }
                }
            }
            sh_u32[3] = cut;
        }
        __syncthreads();
        for (uint32_t j = sh_u32[3] + tid; j < n; j += SP_T) a.f[(uint32_t)cand[j]] = SP_NEG_INF;
        __syncthreads();
        }
    }

    // 4. the draw over the survivors in token order (:592-651)
    float m = -__builtin_inff();
    for (size_t i = tid; i < V; i += SP_T) m = __builtin_fmaxf(m, h2f(a.f[i]));
    for (int o = 32; o > 0; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < SP_T / 64; w++) mx = __builtin_fmaxf(mx, red[w]);
    if (mx == -__builtin_inff()) {
        if (tid == 0) *a.out = 0;
        return;
    }
    const size_t per = (V + SP_T - 1) / SP_T;
    const size_t c0 = (size_t)tid * per, c1 = c0 + per < V ? c0 + per : V;
    uint32_t cnt = 0;
    for (size_t i = c0; i < c1; i++) cnt += a.f[i] != SP_NEG_INF;
    scan[tid] = cnt;
    __syncthreads();
    for (int o = 1; o < SP_T; o <<= 1) {   // inclusive scan
        const uint32_t v = tid >= o ? scan[tid - o] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t off = scan[tid] - cnt;
    for (size_t i = c0; i < c1; i++) {
        if (a.f[i] == SP_NEG_INF) continue;
        a.surv[off] = (uint32_t)i;
        a.pv[off] = cactus_expf(h2f(a.f[i]) - mx);
        off++;
    }
    __syncthreads();
    if (tid != 0) return;
    const uint32_t S = scan[SP_T - 1];
    float sum = 0.0f;
    for (uint32_t j = 0; j < S; j++) sum += a.pv[j];
    if (sum == 0.0f) {
        *a.out = 0;
        return;
    }
    uint32_t tok = 0;
    bool found = false;
    if (a.u <= 0.0f) {
        found = true;   // the running sum is >= u already at token 0
    } else {
        float cum = 0.0f;
        for (uint32_t j = 0; j < S && !found; j++) {
            cum += a.pv[j] / sum;
            if (cum >= a.u) { tok = a.surv[j]; found = true; }
        }
        for (uint32_t j = S; j > 0 && !found; j--)
            if (a.pv[j - 1] / sum > 0.0f) { tok = a.surv[j - 1]; found = true; }
    }
    // history (:633-650)
    uint32_t n = a.hist[0];
    if (n == (uint32_t)SP_HIST) {
        for (uint32_t j = 1; j < (uint32_t)SP_HIST; j++) a.hist[j] = a.hist[j + 1];
        n = SP_HIST - 1;
    }
    a.hist[1 + n] = tok;
    a.hist[0] = n + 1;
    *a.out = tok;
}

// ---------------------------------------------------------------- FP32 sampler
// cactus_sample_f32 (kernel_nn.cpp:253-444) in one workgroup: the bias
// entries in order, the division by T, top-k by a four-pass radix select over
// order-preserving 32-bit keys, min-p 0.15 (probabilities over the survivors
// in token order: parallel expf, the sum by one thread in token order, the
// division and the threshold in parallel), top-p as in the FP16 sampler and
// the draw.  Both infinities count as removed (std::isinf).  No history.
constexpr int SP_BIAS = 128;           // logit-bias entries carried in the kernel arguments

struct SampleF32Args {
    const float* logits;
    uint32_t* out;
    float* f;           // [V] filtered logits
    float* pv;          // [V] unnormalised probabilities of the survivors
    uint32_t* surv;     // [V] survivor tokens in order
    uint32_t* sk;       // [next_pow2(V)] order keys of a large top-p
    size_t V, top_k;
    float top_p, u, temperature;
    int scale;          // temperature > 0
    int bias_n;
    float bias_v[SP_BIAS];
    uint32_t bias_i[SP_BIAS];
};


// workgroup max of f over [0, V) (every thread gets it)
__device__ float wg_max(const float* f, size_t V, float* red) {
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (size_t i = tid; i < V; i += SP_T) m = __builtin_fmaxf(m, f[i]);
    for (int o = 32; o > 0; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o, 64));
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < SP_T / 64; w++) mx = __builtin_fmaxf(mx, red[w]);
    return mx;
}

// the finite entries of f in token order: surv[j] = token, pv[j] =
// expf(f - mx); returns their count (every thread)
__device__ uint32_t wg_compact(const float* f, size_t V, float mx, uint32_t* surv, float* pv, uint32_t* scan) {
    const int tid = threadIdx.x;
    const size_t per = (V + SP_T - 1) / SP_T;
    const size_t c0 = (size_t)tid * per, c1 = c0 + per < V ? c0 + per : V;
    uint32_t cnt = 0;
    for (size_t i = c0; i < c1; i++) cnt += !is_inf(f[i]);
    __syncthreads();
    scan[tid] = cnt;
    __syncthreads();
    for (int o = 1; o < SP_T; o <<= 1) {   // inclusive scan
        const uint32_t v = tid >= o ? scan[tid - o] : 0u;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    uint32_t off = scan[tid] - cnt;
    for (size_t i = c0; i < c1; i++) {
        if (is_inf(f[i])) continue;
        surv[off] = (uint32_t)i;
        pv[off] = cactus_expf(f[i] - mx);
        off++;
    }
    const uint32_t S = scan[SP_T - 1];
    __syncthreads();
    return S;
}

__global__ void __launch_bounds__(SP_T) sample_f32_kernel(SampleF32Args a) {
    extern __shared__ unsigned long long cand[];   // [SP_CAND], dynamic: 128 KB
    __shared__ uint32_t hbin[256];
    __shared__ uint32_t scan[SP_T];
    __shared__ float red[SP_T / 64];
    __shared__ float shf[2];
    __shared__ uint32_t sh_u32[4];
    const int tid = threadIdx.x;
    const size_t V = a.V;

    // 1. copy, bias (:280-288, in entry order), temperature (:290-294)
    for (size_t i = tid; i < V; i += SP_T) a.f[i] = a.logits[i];
    __syncthreads();
    if (tid == 0)
        for (int j = 0; j < a.bias_n; j++)
            if (a.bias_i[j] < V) a.f[a.bias_i[j]] += a.bias_v[j];
    __syncthreads();
    if (a.scale)
        for (size_t i = tid; i < V; i += SP_T) a.f[i] = a.f[i] / a.temperature;
    __syncthreads();

    // 2. top-k (:296-313): the k-th largest value, four radix passes
    if (a.top_k > 0 && a.top_k < V) {
        uint32_t prefix = 0, need = (uint32_t)a.top_k;
        for (int pass = 0; pass < 4; pass++) {
            const int sh = 24 - 8 * pass;
            if (tid < 256) hbin[tid] = 0;
            __syncthreads();
            for (size_t i = tid; i < V; i += SP_T) {
                const uint32_t k = okey32(a.f[i]);
                if (pass == 0 || (k >> (sh + 8)) == prefix) atomicAdd(&hbin[(k >> sh) & 255u], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t cum = 0;
                int b = 255;
                for (; b > 0; b--) {
                    if (cum + hbin[b] >= need) break;
                    cum += hbin[b];
                }
                sh_u32[0] = (uint32_t)b;
                sh_u32[1] = need - cum;
            }
            __syncthreads();
            prefix = (prefix << 8) | sh_u32[0];
            need = sh_u32[1];
            __syncthreads();
        }
        const uint32_t kth = prefix;
        for (size_t i = tid; i < V; i += SP_T)
            if (okey32(a.f[i]) < kth) a.f[i] = -__builtin_inff();
        __syncthreads();
    }

    // 3. min-p 0.15 (:316-346)
    {
        const float mx = wg_max(a.f, V, red);
        if (!is_inf(mx)) {
            const uint32_t S = wg_compact(a.f, V, mx, a.surv, a.pv, scan);
            if (tid == 0) {
                float sum = 0.0f;
                for (uint32_t j = 0; j < S; j++) sum += a.pv[j];
                shf[0] = sum;
            }
            __syncthreads();
            const float sum = shf[0];
            if (sum > 0.0f) {
                float mp = 0.0f;
                for (uint32_t j = tid; j < S; j += SP_T) mp = __builtin_fmaxf(mp, a.pv[j] / sum);
                for (int o = 32; o > 0; o >>= 1) mp = __builtin_fmaxf(mp, __shfl_xor(mp, o, 64));
                if ((tid & 63) == 0) red[tid >> 6] = mp;
                __syncthreads();
                float maxp = red[0];
                for (int w = 1; w < SP_T / 64; w++) maxp = __builtin_fmaxf(maxp, red[w]);
                const float thr = maxp * 0.15f;
                // removed entries (probability 0) stay -inf; survivors below
                // the threshold join them
                for (uint32_t j = tid; j < S; j += SP_T)
                    if (a.pv[j] / sum < thr) a.f[a.surv[j]] = -__builtin_inff();
            }
            __syncthreads();
        }
    }

    // 4. top-p (:348-392) over the finite entries, sorted descending
    if (a.top_p > 0.0f && a.top_p < 1.0f) {
        if (tid == 0) sh_u32[2] = 0;
        __syncthreads();
        for (size_t i = tid; i < V; i += SP_T) {
            if (is_inf(a.f[i])) continue;
            const uint32_t slot = atomicAdd(&sh_u32[2], 1u);
            if (slot < (uint32_t)SP_CAND)
                cand[slot] = ((unsigned long long)(~okey32(a.f[i])) << 32) | (unsigned long long)i;
        }
        __syncthreads();
        const uint32_t n = sh_u32[2];
        if (n > (uint32_t)SP_CAND) {
            topp_large(TopPF32{a.f}, V, a.top_p, a.sk, a.pv, reinterpret_cast<uint32_t*>(cand), scan);
        } else {
        uint32_t n2 = 1;
        while (n2 < n) n2 <<= 1;
        for (uint32_t j = n + tid; j < n2; j += SP_T) cand[j] = ~0ull;
        __syncthreads();
        for (uint32_t size = 2; size <= n2; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = tid; i < n2; i += SP_T) {
                    const uint32_t j = i ^ stride;
                    if (j > i) {
                        const bool up = (i & size) == 0;
                        const unsigned long long x = cand[i], y = cand[j];
                        if ((x > y) == up) {
                            cand[i] = y;
                            cand[j] = x;
                        }
                    }
                }
                __syncthreads();
            }
        }
        if (tid == 0) {
            uint32_t cut = n;
            if (n > 0) {
                const float mx = a.f[(uint32_t)cand[0]];
                float sum = 0.0f;
                for (uint32_t j = 0; j < n; j++) sum += cactus_expf(a.f[(uint32_t)cand[j]] - mx);
                float cum = 0.0f;
                for (uint32_t j = 0; j < n; j++) {
                    cum += cactus_expf(a.f[(uint32_t)cand[j]] - mx) / sum;
                    if (cum > a.top_p) {
                        cut = j > 0 ? j : 1;   // position 0 always stays (:381-384)
                        break;
                    }
                }
            }
            sh_u32[3] = cut;
        }
        __syncthreads();
        for (uint32_t j = sh_u32[3] + tid; j < n; j += SP_T) a.f[(uint32_t)cand[j]] = -__builtin_inff();
        __syncthreads();
        }
    }

    // 5. the draw over the finite entries in token order (:394-444)
    const float mx = wg_max(a.f, V, red);
    if (is_inf(mx)) {
        if (tid == 0) *a.out = 0;
        return;
    }
    const uint32_t S = wg_compact(a.f, V, mx, a.surv, a.pv, scan);
    if (tid != 0) return;
    float sum = 0.0f;
    for (uint32_t j = 0; j < S; j++) sum += a.pv[j];
    if (sum == 0.0f) {
        *a.out = 0;
        return;
    }
    uint32_t tok = 0;
    bool found = false;
    if (a.u <= 0.0f) {
        found = true;   // the running sum is >= u already at token 0
    } else {
        float cum = 0.0f;
        for (uint32_t j = 0; j < S && !found; j++) {
            cum += a.pv[j] / sum;
            if (cum >= a.u) { tok = a.surv[j]; found = true; }
        }
        for (uint32_t j = S; j > 0 && !found; j--)
            if (a.pv[j - 1] / sum > 0.0f) { tok = a.surv[j - 1]; found = true; }
    }
    *a.out = tok;
}

// ---------------------------------------------------------------- entropy
// Model::decode's out_entropy (engine_model.cpp:255-290): max, then the sum
// of exp in double and the entropy sum in double, each a tree over the
// workgroup (the reference sums sequentially; the double partial sums
// differ in the last bits, far below the float result's precision).
__global__ void __launch_bounds__(1024) entropy_kernel(const uint16_t* __restrict__ L, size_t V, float* out) {
    __shared__ double rd[1024];
    __shared__ float rf[1024];
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (size_t i = tid; i < V; i += 1024) m = __builtin_fmaxf(m, h2f(L[i]));
    rf[tid] = m;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if (tid < w) rf[tid] = __builtin_fmaxf(rf[tid], rf[tid + w]);
        __syncthreads();
    }
    const float mx = rf[0];
    double se = 0.0;
    for (size_t i = tid; i < V; i += 1024) se += exp((double)(h2f(L[i]) - mx));
    rd[tid] = se;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if (tid < w) rd[tid] += rd[tid + w];
        __syncthreads();
    }
    const double lse = (double)mx + log(rd[0]);
    __syncthreads();
    double ent = 0.0;
    for (size_t i = tid; i < V; i += 1024) {
        const double lp = (double)h2f(L[i]) - lse;
        const double p = exp(lp);
        if (p > 1e-10) ent -= p * lp;
    }
    rd[tid] = ent;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if (tid < w) rd[tid] += rd[tid + w];
        __syncthreads();
    }
    if (tid == 0) *out = (float)(rd[0] / log((double)V));
}

// per-device scratch (grown) and token history (zeroed once)
struct SampleState {
    uint16_t* f = nullptr;
    float* f32 = nullptr;
    float* pv = nullptr;
    uint32_t* surv = nullptr;
    uint32_t* sk = nullptr;
    size_t cap = 0;
    uint32_t* hist = nullptr;
};
static std::mutex g_sample_mu;
static std::map<int, SampleState> g_sample;

static int sample_state(size_t V, SampleState** out) {
    int dev = 0;
    CH_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_sample_mu);
    SampleState& s = g_sample[dev];
    if (!s.hist) {
        CH_HIP(hipMalloc(&s.hist, (1 + SP_HIST) * sizeof(uint32_t)));
        CH_HIP(hipMemset(s.hist, 0, (1 + SP_HIST) * sizeof(uint32_t)));
    }
    if (s.cap < V) {
        // buffers of earlier calls may still be read by queued kernels
        CH_HIP(hipDeviceSynchronize());
        if (s.f) CH_HIP(hipFree(s.f));
        if (s.pv) CH_HIP(hipFree(s.pv));
        if (s.surv) CH_HIP(hipFree(s.surv));
        if (s.f32) CH_HIP(hipFree(s.f32));
        if (s.sk) CH_HIP(hipFree(s.sk));
        s.f = nullptr; s.pv = nullptr; s.surv = nullptr; s.f32 = nullptr; s.sk = nullptr; s.cap = 0;
        CH_HIP(hipMalloc(&s.f, V * sizeof(uint16_t)));
        CH_HIP(hipMalloc(&s.pv, V * sizeof(float)));
        CH_HIP(hipMalloc(&s.surv, V * sizeof(uint32_t)));
        CH_HIP(hipMalloc(&s.f32, V * sizeof(float)));
        size_t n2 = 1;
        while (n2 < V) n2 <<= 1;
        CH_HIP(hipMalloc(&s.sk, n2 * sizeof(uint32_t)));
        s.cap = V;
    }
    *out = &s;
    return CACTUS_HIP_OK;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_sample_f16(const uint16_t* logits, uint32_t* out, size_t vocab, float temperature,
                          float top_p, size_t top_k, size_t random_seed, void* stream) {
    CH_REQUIRE(out, "sample: null output");
    CH_REQUIRE(vocab == 0 || logits, "sample: null logits");
    if (vocab == 0) return cactus_hip_memset(out, 0, 4, stream);
    if (temperature == 0.0f && top_p <= 0.0f && top_k == 0) {
        hipLaunchKernelGGL(argmax_kernel<uint16_t>, dim3(1), dim3(1024), 0, as_stream(stream), logits, vocab, out);
        return check_launch("sample");
    }
    CH_REQUIRE(vocab < (1ull << 31), "sample: vocabulary too large");
    CH_REQUIRE(temperature >= 0.0f && temperature == temperature, "sample: temperature must be >= 0");
    SampleState* s = nullptr;
    int rc = sample_state(vocab, &s);
    if (rc) return rc;
    // the reference's draw (kernel_nn.cpp:609-612): mt19937 seeded with the
    // 32-bit seed (a random one for seed 0), first output through libc++'s
    // generate_canonical<float, 24>
    const uint32_t seed = random_seed ? (uint32_t)random_seed : std::random_device{}();
    std::mt19937 gen(seed);
    const uint32_t x = (uint32_t)gen();
    SampleArgs a{};
    a.logits = logits;
    a.out = out;
    a.f = s->f;
    a.pv = s->pv;
    a.surv = s->surv;
    a.sk = s->sk;
    a.hist = s->hist;
    a.V = vocab;
    a.top_k = top_k;
    a.top_p = top_p;
    a.u = (float)x / 4294967296.0f;
    a.scale = temperature > 0.0f;
    a.inv_t = a.scale ? host_f2h(1.0f / temperature) : (uint16_t)0;
    a.pen_inv = host_f2h(1.0f / 1.1f);
    a.pen = host_f2h(1.1f);
    const size_t lds = SP_CAND * sizeof(unsigned long long);
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)sample_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    CH_REQUIRE(attr == hipSuccess, "sample: cannot reserve the candidate LDS");
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(SP_T), lds, as_stream(stream), a);
    return check_launch("sample");
}

int cactus_hip_sample_f32(const float* logits, uint32_t* out, size_t vocab, float temperature, float top_p,
                          size_t top_k, size_t random_seed, const float* bias_values, const uint32_t* bias_indices,
                          size_t bias_count, void* stream) {
    CH_REQUIRE(out, "sample_f32: null output");
    CH_REQUIRE(vocab == 0 || logits, "sample_f32: null logits");
    if (vocab == 0) return cactus_hip_memset(out, 0, 4, stream);
    if (temperature == 0.0f && top_p <= 0.0f && top_k == 0) {
        hipLaunchKernelGGL(argmax_kernel<float>, dim3(1), dim3(1024), 0, as_stream(stream), logits, vocab, out);
        return check_launch("sample_f32");
    }
    CH_REQUIRE(vocab < (1ull << 31), "sample_f32: vocabulary too large");
    CH_REQUIRE(temperature >= 0.0f && temperature == temperature, "sample_f32: temperature must be >= 0");
    const bool biased = bias_values && bias_indices && bias_count > 0;
    if (biased && bias_count > (size_t)SP_BIAS)
        return fail(CACTUS_HIP_EUNSUPPORTED, "sample_f32: at most 128 logit-bias entries");
    SampleState* s = nullptr;
    int rc = sample_state(vocab, &s);
    if (rc) return rc;
    const uint32_t seed = random_seed ? (uint32_t)random_seed : std::random_device{}();
    std::mt19937 gen(seed);
    const uint32_t x = (uint32_t)gen();
    SampleF32Args a{};
    a.logits = logits;
    a.out = out;
    a.f = s->f32;
    a.pv = s->pv;
    a.surv = s->surv;
    a.sk = s->sk;
    a.V = vocab;
    a.top_k = top_k;
    a.top_p = top_p;
    a.u = (float)x / 4294967296.0f;
    a.temperature = temperature;
    a.scale = temperature > 0.0f;
    a.bias_n = biased ? (int)bias_count : 0;
    for (int j = 0; j < a.bias_n; j++) {
        a.bias_v[j] = bias_values[j];
        a.bias_i[j] = bias_indices[j];
    }
    const size_t lds = SP_CAND * sizeof(unsigned long long);
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)sample_f32_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    CH_REQUIRE(attr == hipSuccess, "sample_f32: cannot reserve the candidate LDS");
    hipLaunchKernelGGL(sample_f32_kernel, dim3(1), dim3(SP_T), lds, as_stream(stream), a);
    return check_launch("sample_f32");
}

int cactus_hip_logits_entropy_f16(const uint16_t* logits, size_t vocab, float* out, void* stream) {
    CH_REQUIRE(logits && out && vocab > 0, "logits_entropy: null pointer or empty vocabulary");
    hipLaunchKernelGGL(entropy_kernel, dim3(1), dim3(1024), 0, as_stream(stream), logits, vocab, out);
    return check_launch("logits_entropy");
}

int cactus_hip_sample_history(uint32_t* tokens, size_t* count, void* stream) {
    CH_REQUIRE(tokens && count, "sample_history: null argument");
    SampleState* s = nullptr;
    int rc = sample_state(0, &s);
    if (rc) return rc;
    uint32_t h[1 + SP_HIST];
    CH_HIP(hipMemcpyAsync(h, s->hist, sizeof(h), hipMemcpyDeviceToHost, as_stream(stream)));
    CH_HIP(hipStreamSynchronize(as_stream(stream)));
    *count = h[0];
    for (uint32_t j = 0; j < h[0] && j < (uint32_t)SP_HIST; j++) tokens[j] = h[1 + j];
    return CACTUS_HIP_OK;
}

int cactus_hip_sample_history_reset(void* stream) {
    SampleState* s = nullptr;
    int rc = sample_state(0, &s);
    if (rc) return rc;
    return cactus_hip_memset(s->hist, 0, (1 + SP_HIST) * sizeof(uint32_t), stream);
}

}  // extern "C"
