// quant_device.h -- per-row activation quantization shared by the quant
// kernels and the fused matmul prologues.
//
// Reference arithmetic (graph_ops_nn.cpp:35-66 with kernel_quants.cpp:158-221):
//   m   = max |x|                       (order-free)
//   s   = m / 127.0f, floored at 1e-10f
//   inv = 1.0f / s                      (IEEE division)
//   q   = sat8(rne(clamp(x * inv, -128, 127)))   for the first floor(K/8)*8
//   q   = (int8) roundf(clamp(x * inv, -128, 127)) for the K%8 tail
#pragma once
#include "hip_common.h"

namespace cactus_hip {

__device__ __forceinline__ int8_t quant_code(float x, float inv, bool tail) {
    float v = x * inv;
    v = __builtin_fmaxf(__builtin_fminf(v, 127.0f), -128.0f);
    if (!tail) return (int8_t)sat8(cvt_rne_sat(v));
    return (int8_t)(int32_t)__builtin_roundf(v);
}

__device__ __forceinline__ float row_scale_from_max(float m) {
    float s = m / 127.0f;
    if (s < 1e-10f) s = 1e-10f;
    return s;
}

// Block-wide max of |x[0..K)|; every thread returns the result.  `red` must
// hold blockDim.x/64 floats of LDS.
__device__ __forceinline__ float block_max_abs_f16(const uint16_t* __restrict__ x, int K,
                                                   float* red) {
    float m = 0.0f;
    const int tid = threadIdx.x;
    const int nt = blockDim.x;
    // 8 fp16 per 16-byte load when aligned
    if ((((uintptr_t)x) & 15) == 0) {
        const int K8 = K / 8;
        const uint4* x4 = reinterpret_cast<const uint4*>(x);
        for (int i = tid; i < K8; i += nt) {
            uint4 u = x4[i];
            uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                m = __builtin_fmaxf(m, __builtin_fabsf(h2f((uint16_t)(w[j] & 0xFFFF))));
                m = __builtin_fmaxf(m, __builtin_fabsf(h2f((uint16_t)(w[j] >> 16))));
            }
        }
        for (int i = K8 * 8 + tid; i < K; i += nt) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(x[i])));
    } else {
        for (int i = tid; i < K; i += nt) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(x[i])));
    }
    m = wave_max(m);
    const int wid = tid >> 6;
    __syncthreads();
    if ((tid & 63) == 0) red[wid] = m;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (nt >> 6); i++) r = __builtin_fmaxf(r, red[i]);
    return r;
}

}  // namespace cactus_hip
