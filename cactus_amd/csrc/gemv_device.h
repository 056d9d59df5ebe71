// gemv_device.h -- building blocks of the grouped INT8 / packed-INT4 GEMV
// kernels (activation code layout, 16-byte chunk dot products, exact int32
// group sums across lanes).
#pragma once
#include "quant_device.h"

namespace cactus_hip {

constexpr int GEMV_THREADS = 256;

// position of activation element i in LDS; INT4 stores each 8-element run as
// its 4 even elements followed by its 4 odd elements so that one dword pairs
// with the low nibbles and the next with the high nibbles of a weight dword
template <bool INT4>
__device__ __forceinline__ int act_pos(int i) {
    if (!INT4) return i;
    const int j = i & 7;
    return (i & ~7) + ((j & 1) ? 4 : 0) + (j >> 1);
}

// dot product of one 16-byte weight chunk with the matching activation codes
template <bool INT4>
__device__ __forceinline__ int chunk_dot(const int8_t* act, int col, i32x4 w) {
    int s = 0;
    if (!INT4) {
        const i32x4 av = *reinterpret_cast<const i32x4*>(act + col * 16);
        s = __builtin_amdgcn_sdot4(av.x, w.x, s, false);
        s = __builtin_amdgcn_sdot4(av.y, w.y, s, false);
        s = __builtin_amdgcn_sdot4(av.z, w.z, s, false);
        s = __builtin_amdgcn_sdot4(av.w, w.w, s, false);
    } else {
        const i32x4* ap = reinterpret_cast<const i32x4*>(act + col * 32);
        const i32x4 a0 = ap[0], a1 = ap[1];
        const uint32_t wv[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
        const int ae[4] = {a0.x, a0.z, a1.x, a1.z};
        const int ao[4] = {a0.y, a0.w, a1.y, a1.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // nibbles moved to the top of each byte: 16 * code
            const int lo = (int)((wv[j] << 4) & 0xF0F0F0F0u);
            const int hi = (int)(wv[j] & 0xF0F0F0F0u);
            s = __builtin_amdgcn_sdot4(ae[j], lo, s, false);
            s = __builtin_amdgcn_sdot4(ao[j], hi, s, false);
        }
        s >>= 4;  // exact: every product carried a factor 16
    }
    return s;
}

// exact int32 sum over aligned groups of P consecutive lanes (P = 1..64)
__device__ __forceinline__ int group_lane_sum(int v, int P) {
    if (P >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    if (P >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    for (int off = 4; off < P; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace cactus_hip
