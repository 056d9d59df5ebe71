// quant.hip -- activation quantization (a1), KV-cache quantization (a7) and
// INT4 unpacking.
#include "decode_device.h"
#include "quant_device.h"

namespace cactus_hip {

// One workgroup computes max|src| over the whole buffer.
__global__ void __launch_bounds__(1024) max_abs_kernel(const uint16_t* __restrict__ src,
                                                       size_t count, float* out) {
    __shared__ float red[16];
    float m = 0.0f;
    for (size_t i = threadIdx.x; i < count; i += blockDim.x)
        m = __builtin_fmaxf(m, __builtin_fabsf(h2f(src[i])));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = red[0];
        for (unsigned i = 1; i < blockDim.x / 64; i++) r = __builtin_fmaxf(r, red[i]);
        *out = r;
    }
}

// cactus_fp16_to_int8 with a host-provided inv = 1.0f / scale.
__global__ void fp16_to_int8_kernel(const uint16_t* __restrict__ src, int8_t* __restrict__ dst,
                                    size_t count, float inv) {
    const size_t body = (count / 8) * 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = quant_code(h2f(src[i]), inv, i >= body);
}

// element e of eight fp16 values held in a uint4
__device__ __forceinline__ uint16_t u4_get(const uint4& v, int e) {
    const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
    return (uint16_t)(e & 1 ? w >> 16 : w & 0xFFFF);
}
__device__ __forceinline__ void u4_set(uint4& v, int e, uint16_t h) {
    uint32_t& w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
    w = e & 1 ? (w & 0xFFFFu) | ((uint32_t)h << 16) : (w & 0xFFFF0000u) | h;
}

// rows of K % 8 == 0 values (K <= 8192) at 16-byte aligned fp16 inputs and
// 8-byte aligned codes: the register path of the row kernels
constexpr int VEC_CPT = 4;   // 8-value chunks per thread
__device__ __forceinline__ bool vec_rows_ok(const uint16_t* x, const uint16_t* w, const int8_t* q, int K) {
    return (K & 7) == 0 && K <= 256 * 8 * VEC_CPT && ((((uintptr_t)x | (uintptr_t)w) & 15) == 0) &&
           (((uintptr_t)q & 7) == 0);
}

// One workgroup per row: scale and codes of quantize_activations_fp16_to_int8.
__global__ void __launch_bounds__(256) quantize_rows_kernel(const uint16_t* __restrict__ x,
                                                            int8_t* __restrict__ q,
                                                            float* __restrict__ scales, int K) {
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const uint16_t* xr = x + row * (size_t)K;
    if (blockDim.x == 256 && vec_rows_ok(x, x, q, K)) {
        // the row in registers: one load, one reduction, codes from registers
        const int tid = threadIdx.x, nch = K >> 3;
        uint4 xv[VEC_CPT];
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++) xv[j] = reinterpret_cast<const uint4*>(xr)[min(tid + 256 * j, nch - 1)];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++)
            if (tid + 256 * j < nch)
#pragma unroll
                for (int e = 0; e < 8; e++) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(u4_get(xv[j], e))));
        m = wave_max(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
        const float s = row_scale_from_max(mx);
        const float inv = 1.0f / s;
        int8_t* qr = q + row * (size_t)K;
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++) {
            const int c = tid + 256 * j;
            if (c < nch) {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo |= (uint32_t)(uint8_t)quant_code(h2f(u4_get(xv[j], e)), inv, false) << (8 * e);
                    hi |= (uint32_t)(uint8_t)quant_code(h2f(u4_get(xv[j], 4 + e)), inv, false) << (8 * e);
                }
                *reinterpret_cast<uint2*>(qr + 8 * c) = make_uint2(lo, hi);
            }
        }
        if (tid == 0) scales[row] = s;
        return;
    }
    const float m = block_max_abs_f16(xr, K, red);
    const float s = row_scale_from_max(m);
    const float inv = 1.0f / s;
    const int body = (K / 8) * 8;
    int8_t* qr = q + row * (size_t)K;
    for (int i = threadIdx.x; i < K; i += blockDim.x) qr[i] = quant_code(h2f(xr[i]), inv, i >= body);
    if (threadIdx.x == 0) scales[row] = s;
}

// RMSNorm (kernel_attention.cpp:484-563) followed by the per-row
// activation quantization of the matmul that consumes it
// (graph_ops_nn.cpp:35-66): the normalized fp16 row stays in LDS, its max
// gives the row scale, the codes are written directly.  The same results as
// cactus_hip_rms_norm_f16 then cactus_hip_quantize_activations, one launch.
__global__ void __launch_bounds__(256) rms_quant_rows_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             int8_t* __restrict__ q, float* __restrict__ scales,
                                                             int K, float eps) {
    extern __shared__ __align__(16) uint16_t xs[];   // the row, then its normalized values
    __shared__ float red[4];
    __shared__ float st[2];
    const int tid = threadIdx.x;
    const size_t row = blockIdx.x;
    const uint16_t* xr = x + row * (size_t)K;
    if (vec_rows_ok(x, w, q, K)) {
        // 16-byte chunks: the row and its weights loaded up front (clamped,
        // branch-free), normalized and quantized in registers
        const int nch = K >> 3;
        uint4 xv[VEC_CPT], wv[VEC_CPT];
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++) {
            const int c = min(tid + 256 * j, nch - 1);
            xv[j] = reinterpret_cast<const uint4*>(xr)[c];
            wv[j] = reinterpret_cast<const uint4*>(w)[c];
        }
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++)
            if (tid + 256 * j < nch) reinterpret_cast<uint4*>(xs)[tid + 256 * j] = xv[j];
        __syncthreads();
        if (tid < 64) {
            float inv;
            uint16_t hinv;
            rms_stats_wave(xs, K, eps, inv, hinv);
            if (tid == 0) {
                st[0] = inv;
                st[1] = __builtin_bit_cast(float, (uint32_t)hinv);
            }
        }
        __syncthreads();
        const float inv = st[0];
        const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, st[1]);
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++) {
            const int c = tid + 256 * j;
            if (c < nch) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint16_t y = rms_apply(u4_get(xv[j], e), u4_get(wv[j], e), 8 * c + e, K, inv, hinv);
                    u4_set(xv[j], e, y);
                    m = __builtin_fmaxf(m, __builtin_fabsf(h2f(y)));
                }
            }
        }
        m = wave_max(m);
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
        const float s = row_scale_from_max(mx);
        const float inv_s = 1.0f / s;
        int8_t* qr = q + row * (size_t)K;
#pragma unroll
        for (int j = 0; j < VEC_CPT; j++) {
            const int c = tid + 256 * j;
            if (c < nch) {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo |= (uint32_t)(uint8_t)quant_code(h2f(u4_get(xv[j], e)), inv_s, false) << (8 * e);
                    hi |= (uint32_t)(uint8_t)quant_code(h2f(u4_get(xv[j], 4 + e)), inv_s, false) << (8 * e);
                }
                *reinterpret_cast<uint2*>(qr + 8 * c) = make_uint2(lo, hi);
            }
        }
        if (tid == 0) scales[row] = s;
        return;
    }
    for (int i = tid; i < K; i += 256) xs[i] = xr[i];
    __syncthreads();
    if (tid < 64) {
        float inv;
        uint16_t hinv;
        rms_stats_wave(xs, K, eps, inv, hinv);
        if (tid == 0) {
            st[0] = inv;
            st[1] = __builtin_bit_cast(float, (uint32_t)hinv);
        }
    }
    __syncthreads();
    const float inv = st[0];
    const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, st[1]);
    const int end8 = (K / 8) * 8;
    float m = 0.0f;
    for (int i = tid; i < K; i += 256) {
        const uint16_t y = rms_apply(xs[i], w[i], i, end8, inv, hinv);
        xs[i] = y;
        m = __builtin_fmaxf(m, __builtin_fabsf(h2f(y)));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float s = row_scale_from_max(mx);
    const float inv_s = 1.0f / s;
    int8_t* qr = q + row * (size_t)K;
    for (int i = tid; i < K; i += 256) qr[i] = quant_code(h2f(xs[i]), inv_s, i >= end8);
    if (tid == 0) scales[row] = s;
}

// SiLU (kernel_nn.cpp:12-44: fast_exp in the vector body, expf in the n % 8
// tail of the whole tensor), the SwiGLU multiply (kernel_blas.cpp:291-316)
// and the row quantization of the down projection that consumes the
// product: one launch, the same codes and scales as the three nodes.
__global__ void __launch_bounds__(256) silu_mul_quant_rows_kernel(const uint16_t* __restrict__ gate,
                                                                  const uint16_t* __restrict__ up,
                                                                  int8_t* __restrict__ q,
                                                                  float* __restrict__ scales, int K,
                                                                  size_t body) {
    extern __shared__ __align__(16) uint16_t ms[];   // the row of silu(gate) * up
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const size_t row = blockIdx.x, base = row * (size_t)K;
    auto value = [&](uint16_t g, uint16_t u, size_t gi) {
        const float x = h2f(g);
        const float e = gi < body ? fast_exp(-x) : cactus_expf(-x);
        const float sig = 1.0f / (1.0f + e);
        return hmul(f2h(x * sig), u);
    };
    float m = 0.0f;
    // 16-byte rows (K % 8 == 0, aligned pointers): each thread's 8-value
    // chunks are loaded up front, four at a time, then computed
    const bool vec = (K & 7) == 0 && (((uintptr_t)gate | (uintptr_t)up | (uintptr_t)q) & 15) == 0;
    if (vec) {
        const int nc = K >> 3;
        for (int c0 = tid; c0 < nc; c0 += 4 * 256) {
            uint4 gv[4], uv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + 256 * j;
                if (c < nc) {
                    gv[j] = *reinterpret_cast<const uint4*>(gate + base + 8 * (size_t)c);
                    uv[j] = *reinterpret_cast<const uint4*>(up + base + 8 * (size_t)c);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + 256 * j;
                if (c < nc) {
                    const uint16_t* g8 = reinterpret_cast<const uint16_t*>(&gv[j]);
                    const uint16_t* u8 = reinterpret_cast<const uint16_t*>(&uv[j]);
                    uint4 ov;
                    uint16_t* o8 = reinterpret_cast<uint16_t*>(&ov);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        o8[e] = value(g8[e], u8[e], base + 8 * (size_t)c + e);
                        m = __builtin_fmaxf(m, __builtin_fabsf(h2f(o8[e])));
                    }
                    *reinterpret_cast<uint4*>(ms + 8 * c) = ov;
                }
            }
        }
    } else {
        for (int i = tid; i < K; i += 256) {
            const size_t gi = base + i;
            const uint16_t v = value(gate[gi], up[gi], gi);
            ms[i] = v;
            m = __builtin_fmaxf(m, __builtin_fabsf(h2f(v)));
        }
    }
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float s = row_scale_from_max(mx);
    const float inv_s = 1.0f / s;
    const int end8 = (K / 8) * 8;
    int8_t* qr = q + base;
    if (vec) {
        // K % 8 == 0: every code is a body code; 8 per thread and store
        for (int c = tid; c < (K >> 3); c += 256) {
            const uint4 v = *reinterpret_cast<const uint4*>(ms + 8 * c);
            const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                lo |= (uint32_t)(uint8_t)quant_code(h2f(h[e]), inv_s, false) << (8 * e);
                hi |= (uint32_t)(uint8_t)quant_code(h2f(h[4 + e]), inv_s, false) << (8 * e);
            }
            *reinterpret_cast<uint2*>(qr + 8 * c) = make_uint2(lo, hi);
        }
    } else {
        for (int i = tid; i < K; i += 256) qr[i] = quant_code(h2f(ms[i]), inv_s, i >= end8);
    }
    if (tid == 0) scales[row] = s;
}

// cactus_quantize_kv_fp16_to_int8: one wave per (token, head, group).
// Body codes: sat8(rne(x * inv)) without a clamp; the count%8 tail of a
// group uses roundf (kernel_quants.cpp:223-264).
__global__ void __launch_bounds__(256) quantize_kv_kernel(const uint16_t* __restrict__ src,
                                                          int8_t* __restrict__ dst,
                                                          float* __restrict__ scales,
                                                          size_t rows, int d, int gs, int ng) {
    const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= rows * (size_t)ng) return;
    const size_t row = wave / ng;
    const int g = (int)(wave % ng);
    const int g0 = g * gs;
    const int cnt = (gs < d - g0) ? gs : d - g0;
    const uint16_t* s = src + row * d + g0;
    int8_t* o = dst + row * d + g0;
    float m = 0.0f;
    for (int i = lane; i < cnt; i += 64) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(s[i])));
    m = wave_max(m);
    const float sc = row_scale_from_max(m);
    const float inv = 1.0f / sc;
    const int body = (cnt / 8) * 8;
    for (int i = lane; i < cnt; i += 64) {
        const float v = h2f(s[i]) * inv;
        int32_t c = (i < body) ? cvt_rne_sat(v) : (int32_t)__builtin_roundf(v);
        o[i] = (int8_t)sat8(c);
    }
    if (lane == 0) scales[row * ng + g] = sc;
}

__global__ void unpack_int4_kernel(const uint8_t* __restrict__ p, int8_t* __restrict__ u,
                                   size_t count) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint8_t b = p[i >> 1];
        int v = (i & 1) ? (b >> 4) : (b & 0x0F);
        u[i] = (int8_t)(v > 7 ? v - 16 : v);
    }
}

static unsigned grid_for(size_t n, unsigned block) {
    size_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > 65535) g = 65535;
    return (unsigned)g;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_fp16_max_abs(const uint16_t* src, size_t count, float* out, void* stream) {
    CH_REQUIRE(out, "fp16_max_abs: null output");
    CH_REQUIRE(count == 0 || src, "fp16_max_abs: null input");
    hipLaunchKernelGGL(max_abs_kernel, dim3(1), dim3(1024), 0, as_stream(stream), src, count, out);
    return check_launch("fp16_max_abs");
}

int cactus_hip_fp16_to_int8(const uint16_t* src, int8_t* dst, size_t count, float scale,
                            void* stream) {
    if (count == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(src && dst, "fp16_to_int8: null pointer");
    const float inv = 1.0f / scale;  // reference computes this once on the host side too
    hipLaunchKernelGGL(fp16_to_int8_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       as_stream(stream), src, dst, count, inv);
    return check_launch("fp16_to_int8");
}

int cactus_hip_quantize_activations(const uint16_t* x, int8_t* q, float* scales, size_t M,
                                    size_t K, void* stream) {
    if (M == 0 || K == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && q && scales, "quantize_activations: null pointer");
    CH_REQUIRE(K < (1u << 30) && M < (1u << 31), "quantize_activations: shape too large");
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)M), dim3(256), 0, as_stream(stream), x,
                       q, scales, (int)K);
    return check_launch("quantize_activations");
}

int cactus_hip_rms_norm_quantize_f16(const uint16_t* x, const uint16_t* weight, int8_t* q, float* scales,
                                     size_t M, size_t K, float eps, void* stream) {
    if (M == 0 || K == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && weight && q && scales, "rms_norm_quantize: null pointer");
    CH_REQUIRE(K <= 32768 && M < (1u << 31), "rms_norm_quantize: rows of at most 32768 values");
    hipLaunchKernelGGL(rms_quant_rows_kernel, dim3((unsigned)M), dim3(256), K * sizeof(uint16_t),
                       as_stream(stream), x, weight, q, scales, (int)K, eps);
    return check_launch("rms_norm_quantize");
}

int cactus_hip_silu_mul_quantize_f16(const uint16_t* gate, const uint16_t* up, int8_t* q, float* scales,
                                     size_t M, size_t K, void* stream) {
    if (M == 0 || K == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(gate && up && q && scales, "silu_mul_quantize: null pointer");
    CH_REQUIRE(K <= 32768 && M < (1u << 31), "silu_mul_quantize: rows of at most 32768 values");
    const size_t body = ((M * K) / 8) * 8;
    hipLaunchKernelGGL(silu_mul_quant_rows_kernel, dim3((unsigned)M), dim3(256), K * sizeof(uint16_t),
                       as_stream(stream), gate, up, q, scales, (int)K, body);
    return check_launch("silu_mul_quantize");
}

int cactus_hip_quantize_kv_fp16_to_int8(const uint16_t* src, int8_t* dst, float* scales,
                                        size_t seq_len, size_t kv_heads, size_t head_dim,
                                        size_t group_size, void* stream) {
    const size_t rows = seq_len * kv_heads;
    if (rows == 0 || head_dim == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(src && dst && scales, "quantize_kv: null pointer");
    CH_REQUIRE(group_size > 0, "quantize_kv: group_size must be > 0");
    CH_REQUIRE(head_dim < (1u << 20), "quantize_kv: head_dim too large");
    const int ng = (int)((head_dim + group_size - 1) / group_size);
    const size_t waves = rows * (size_t)ng;
    hipLaunchKernelGGL(quantize_kv_kernel, dim3(ceil_div(waves, 4)), dim3(256), 0,
                       as_stream(stream), src, dst, scales, rows, (int)head_dim, (int)group_size,
                       ng);
    return check_launch("quantize_kv");
}

int cactus_hip_unpack_int4_to_int8(const uint8_t* packed, int8_t* unpacked, size_t count,
                                   void* stream) {
    if (count == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(packed && unpacked, "unpack_int4: null pointer");
    hipLaunchKernelGGL(unpack_int4_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       as_stream(stream), packed, unpacked, count);
    return check_launch("unpack_int4");
}

}  // extern "C"
