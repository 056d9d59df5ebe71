// lm_device.h -- FP16-accumulation dot product building blocks of the
// FP16 matmul / LM head (reference kernel_gemm.cpp:8-66).
#pragma once
#include "hip_common.h"

namespace cactus_hip {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

constexpr int LM_THREADS = 256;
constexpr int LM_ROWS_PER_WAVE = 64;
constexpr int LM_KC = 64;                 // k-values staged per step
constexpr int LM_ROW_STRIDE = LM_KC * 2 + 16;  // bytes per staged row (+16 pad)
constexpr int LM_MR = 4;                  // activation rows per pass
constexpr int LM_MAX_K = 8192;

__device__ __forceinline__ h2v as_h2(uint32_t u) { return __builtin_bit_cast(h2v, u); }

// one 8-element step of the eight chains: chains (0,1),(2,3),(4,5),(6,7)
__device__ __forceinline__ void f16_step(h2v acc[4], uint4 av, uint4 bv) {
    acc[0] = __builtin_elementwise_fma(as_h2(av.x), as_h2(bv.x), acc[0]);
    acc[1] = __builtin_elementwise_fma(as_h2(av.y), as_h2(bv.y), acc[1]);
    acc[2] = __builtin_elementwise_fma(as_h2(av.z), as_h2(bv.z), acc[2]);
    acc[3] = __builtin_elementwise_fma(as_h2(av.w), as_h2(bv.w), acc[3]);
}

// hsum_f16x8 (kernel_gemm.cpp:8-15)
__device__ __forceinline__ uint16_t f16_hsum(const h2v acc[4]) {
    const h2v s01 = acc[0] + acc[2];   // (l0+l4, l1+l5)
    const h2v s23 = acc[1] + acc[3];   // (l2+l6, l3+l7)
    const h2v t = s01 + s23;           // ((l0+l4)+(l2+l6), (l1+l5)+(l3+l7))
    const f16 r = t.x + t.y;
    return __builtin_bit_cast(uint16_t, r);
}

}  // namespace cactus_hip
