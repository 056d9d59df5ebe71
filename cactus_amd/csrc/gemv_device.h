// gemv_device.h -- building blocks of the grouped INT8 / packed-INT4 GEMV
// kernels (activation code layout, 16-byte chunk dot products, exact int32
// group sums across lanes).
#pragma once
#include "quant_device.h"

namespace cactus_hip {

constexpr int GEMV_THREADS = 256;

// INT4 activation layout in LDS: each run of 8 codes c_0..c_7 (INT8 codes,
// |c| <= 127) as two dwords, H with nibble i = c_i >> 4 and L with nibble i
// = (c_i & 15) - 8, both signed 4-bit, so that c_i = 16 h_i + l_i + 8 and a
// weight dword w of 8 signed nibbles dots as
//   sum c_i w_i = 16 dot8(H, w) + dot8(L, w) + 8 dot8(1..1, w)
// with v_dot8_i32_i4 (exact int32, no nibble expansion).  `lo` holds codes
// 0-3 as bytes, `hi` codes 4-7.  A row of K codes keeps its H dwords in
// one plane and its L dwords in another (K/2 bytes each): run r's H at
// byte 4r, its L at K/2 + 4r (nib_store8), so a 32-code weight chunk's four
// H (and four L) dwords are 16 contiguous bytes and the lanes of a wave,
// reading consecutive chunks, read consecutive 16-byte pieces of LDS.
__device__ __forceinline__ uint2 nib_pack8(uint32_t lo, uint32_t hi) {
    // nibbles at bits 8j..8j+3 (j = 0..3) -> bits 4j..4j+3
    auto squeeze = [](uint32_t a) {
        a = (a | (a >> 4)) & 0x00FF00FFu;
        return (a | (a >> 8)) & 0x0000FFFFu;
    };
    const uint32_t h = squeeze((lo >> 4) & 0x0F0F0F0Fu) | (squeeze((hi >> 4) & 0x0F0F0F0Fu) << 16);
    const uint32_t l = squeeze((lo & 0x0F0F0F0Fu) ^ 0x08080808u) | (squeeze((hi & 0x0F0F0F0Fu) ^ 0x08080808u) << 16);
    return make_uint2(h, l);
}

// run r of a row's INT4 codes, nib_pack8'd, into the row's two planes
__device__ __forceinline__ void nib_store8(int8_t* row, int K, int r, uint2 hl) {
    *reinterpret_cast<uint32_t*>(row + 4 * r) = hl.x;
    *reinterpret_cast<uint32_t*>(row + K / 2 + 4 * r) = hl.y;
}

// dot product of one 16-byte weight chunk with the matching activation codes
// (INT8: 16 codes as bytes; INT4: 32 codes, their H and L dwords in the two
// planes of the row, the L plane `lplane` = K/2 bytes after the H plane)
template <bool INT4>
__device__ __forceinline__ int chunk_dot(const int8_t* act, int col, i32x4 w, int lplane = 0) {
    if (!INT4) {
        const i32x4 av = *reinterpret_cast<const i32x4*>(act + col * 16);
        int s = 0;
        s = __builtin_amdgcn_sdot4(av.x, w.x, s, false);
        s = __builtin_amdgcn_sdot4(av.y, w.y, s, false);
        s = __builtin_amdgcn_sdot4(av.z, w.z, s, false);
        s = __builtin_amdgcn_sdot4(av.w, w.w, s, false);
        return s;
    } else {
        const i32x4 hv = *reinterpret_cast<const i32x4*>(act + col * 16);            // {H0, H1, H2, H3}
        const i32x4 lv = *reinterpret_cast<const i32x4*>(act + lplane + col * 16);   // {L0, L1, L2, L3}
        constexpr int ONES = 0x11111111;
        int sh = 0, sl = 0, sw = 0;
        sh = __builtin_amdgcn_sdot8(hv.x, w.x, sh, false);
        sl = __builtin_amdgcn_sdot8(lv.x, w.x, sl, false);
        sw = __builtin_amdgcn_sdot8(ONES, w.x, sw, false);
        sh = __builtin_amdgcn_sdot8(hv.y, w.y, sh, false);
        sl = __builtin_amdgcn_sdot8(lv.y, w.y, sl, false);
        sw = __builtin_amdgcn_sdot8(ONES, w.y, sw, false);
        sh = __builtin_amdgcn_sdot8(hv.z, w.z, sh, false);
        sl = __builtin_amdgcn_sdot8(lv.z, w.z, sl, false);
        sw = __builtin_amdgcn_sdot8(ONES, w.z, sw, false);
        sh = __builtin_amdgcn_sdot8(hv.w, w.w, sh, false);
        sl = __builtin_amdgcn_sdot8(lv.w, w.w, sl, false);
        sw = __builtin_amdgcn_sdot8(ONES, w.w, sw, false);
        return sh * 16 + sl + sw * 8;
    }
}

// exact int32 sum over aligned groups of P consecutive lanes (P = 1..64)
__device__ __forceinline__ int group_lane_sum(int v, int P) {
    if (P >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    if (P >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    for (int off = 4; off < P; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace cactus_hip
