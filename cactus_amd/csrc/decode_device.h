// decode_device.h -- per-row pieces of the Qwen3 decode step shared by the
// fused decode kernels and the decode attention: the reference's RMSNorm
// statistics and scaling, the head RoPE, and the INT8 KV-cache append.
#pragma once
#include "quant_device.h"

namespace cactus_hip {

// ----------------------------------------------------------------- RMSNorm
// lanes 0..3: ((c_l + c_{l+4}) + c_{l+8}) + c_{l+12} of the 16 chain sums
// (row_shl DPP moves within the first 16-lane row)
__device__ __forceinline__ float rms_chain_combine4(float c) {
    const int b = __builtin_bit_cast(int, c);
    const float c4 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x104, 0xF, 0xF, false));
    const float c8 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x108, 0xF, 0xF, false));
    const float c12 = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x10C, 0xF, 0xF, false));
    return ((c + c4) + c8) + c12;
}
__device__ __forceinline__ float lane_value(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// 1/rms of an fp16 row held in LDS, in the reference's order (16 fp32 FMA
// chains, kernel_attention.cpp:500-538).  Called by one whole wave; every
// lane returns inv and fp16(inv).
__device__ __forceinline__ void rms_stats_wave(const uint16_t* xs, int n, float eps, float& inv,
                                               uint16_t& hinv) {
    const int lane = threadIdx.x & 63;
    float chain = 0.0f;
    const int n16 = n / 16, end8 = (n / 8) * 8;
    if (lane < 16) {
        int i = 0;
        // 16 reads in flight per batch, then the chain steps
        for (; i + 16 <= n16; i += 16) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = h2f(xs[(i + j) * 16 + lane]);
#pragma unroll
            for (int j = 0; j < 16; j++) chain = __builtin_fmaf(v[j], v[j], chain);
        }
        for (; i < n16; i++) {
            const float v = h2f(xs[i * 16 + lane]);
            chain = __builtin_fmaf(v, v, chain);
        }
        if (lane < 8 && n16 * 16 + 8 <= n) {
            const float a = h2f(xs[n16 * 16 + lane]);
            chain = __builtin_fmaf(a, a, chain);
        }
    }
    const float t = rms_chain_combine4(chain);
    const float t0 = lane_value(t, 0), t1 = lane_value(t, 1), t2 = lane_value(t, 2), t3 = lane_value(t, 3);
    float ss = (t0 + t1) + (t2 + t3);
    for (int k = end8; k < n; k++) {
        const float a = h2f(xs[k]);
        ss = __builtin_fmaf(a, a, ss);
    }
    const float rms = __builtin_sqrtf(ss / (float)n + eps);
    inv = 1.0f / rms;
    hinv = f2h(inv);
}

// rms_stats_wave for R <= 4 rows of N values each (N % 16 == 0, a head
// row), all at once: 16-lane row r of the wave runs row r's 16 chains, each
// lane's N/16 reads issued before its FMAs, and the per-row combination by
// the same DPP moves within that 16-lane row.  Row r starts at xs + r *
// stride; every lane returns every row's inv and fp16(inv).
template <int N, int R>
__device__ __forceinline__ void rms_stats_rows(const uint16_t* xs, int stride, float eps, float (&inv)[R],
                                               uint16_t (&hinv)[R]) {
    static_assert(N % 16 == 0 && R >= 1 && R <= 4, "head rows");
    const int lane = threadIdx.x & 63;
    const int rr = lane >> 4, l = lane & 15;
    const uint16_t* x = xs + min(rr, R - 1) * stride;
    float v[N / 16];
#pragma unroll
    for (int i = 0; i < N / 16; i++) v[i] = h2f(x[i * 16 + l]);
    float chain = 0.0f;
#pragma unroll
    for (int i = 0; i < N / 16; i++) chain = __builtin_fmaf(v[i], v[i], chain);
    const float t = rms_chain_combine4(chain);
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float ss = (lane_value(t, 16 * r) + lane_value(t, 16 * r + 1)) +
                         (lane_value(t, 16 * r + 2) + lane_value(t, 16 * r + 3));
        const float rms = __builtin_sqrtf(ss / (float)N + eps);
        inv[r] = 1.0f / rms;
        hinv[r] = f2h(inv[r]);
    }
}

// rms_stats_wave over a row stored chain-major in LDS: chain l's values
// x[16 i + l] at xt[l * (n / 16 + 8) + i] (8 elements of padding per chain
// keep the 16 chains' 16-byte reads on distinct banks).  n % 128 == 0.  Each
// chain lane loads 64 values at a time with eight 16-byte reads before its
// FMAs, so the chain waits for LDS once per 64 steps; the same arithmetic
// and order as rms_stats_wave.
constexpr int RMS_T_PAD = 8;
__device__ __forceinline__ int rms_t_index(int k, int n) {
    return (k & 15) * (n / 16 + RMS_T_PAD) + (k >> 4);
}
__device__ __forceinline__ void rms_stats_wave_t(const uint16_t* xt, int n, float eps, float& inv,
                                                 uint16_t& hinv) {
    const int lane = threadIdx.x & 63;
    const int n16 = n / 16, nb = n16 / 8;
    float chain = 0.0f;
    if (lane < 16) {
        const uint4* p = reinterpret_cast<const uint4*>(xt + lane * (n16 + RMS_T_PAD));
        for (int b = 0; b < nb; b += 8) {
            uint4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = p[min(b + j, nb - 1)];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (b + j < nb) {
                    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = h2f((uint16_t)(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xFFFF));
                        chain = __builtin_fmaf(x, x, chain);
                    }
                }
            }
        }
    }
    const float t = rms_chain_combine4(chain);
    const float t0 = lane_value(t, 0), t1 = lane_value(t, 1), t2 = lane_value(t, 2), t3 = lane_value(t, 3);
    const float ss = (t0 + t1) + (t2 + t3);
    const float rms = __builtin_sqrtf(ss / (float)n + eps);
    inv = 1.0f / rms;
    hinv = f2h(inv);
}

__device__ __forceinline__ uint16_t rms_apply(uint16_t x, uint16_t w, int i, int end8, float inv,
                                              uint16_t hinv) {
    return i < end8 ? hmul(hmul(x, hinv), w) : f2h((h2f(x) * inv) * h2f(w));
}

// RoPE of one head row held in LDS (kernel_attention.cpp:640-671) at the
// tables' row for the position: pairs (i, i + d/2); the 8-aligned part of
// the half row in fp16 arithmetic, the tail in fp32.  Writes the rotated
// fp16 values through out(i, value).  One whole wave.
// one rotated pair (i, i + d/2): fp16 arithmetic below vh = 8-aligned half, fp32 above
__device__ __forceinline__ void rope_pair(uint16_t x1, uint16_t x2, uint16_t c, uint16_t s, bool fp16_part,
                                          uint16_t& o1, uint16_t& o2) {
    if (fp16_part) {
        o1 = hfma(x2 ^ 0x8000u, s, hmul(x1, c));
        o2 = hfma(x1, s, hmul(x2, c));
    } else {
        const float fa = h2f(x1), fb = h2f(x2), cf = h2f(c), sf = h2f(s);
        o1 = f2h(fa * cf - fb * sf);
        o2 = f2h(fb * cf + fa * sf);
    }
}

template <class Out>
__device__ __forceinline__ void rope_row(const uint16_t* ys, int d, const uint16_t* ct, const uint16_t* stb,
                                         Out out) {
    const int lane = threadIdx.x & 63;
    const int half = d / 2, vh = (half / 8) * 8;
    for (int i = lane; i < half; i += 64) {
        uint16_t o1, o2;
        rope_pair(ys[i], ys[i + half], ct[i], stb[i], i < vh, o1, o2);
        out(i, o1);
        out(i + half, o2);
    }
}

// quantize_group_fp16_to_int8 per 128-dim group (kernel_quants.cpp:223-264);
// with `sh`, also the row's fp32 products (float)code * scale into the
// product tiles (sh_index layout, key `key`, kv head `h`)
__device__ __forceinline__ void kv_append_row(const uint16_t* src, int8_t* dst, float* scales, int d,
                                              float* sh = nullptr, size_t ntile = 0, size_t key = 0, int h = 0) {
    const int lane = threadIdx.x & 63;
    const int nsl = (d + 63) / 64, da = (d / 8) * 8;
    for (int g0 = 0, g = 0; g0 < d; g0 += 128, g++) {
        const int cnt = min(128, d - g0);
        float m = 0.0f;
        for (int i = lane; i < cnt; i += 64) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(src[g0 + i])));
        m = wave_max(m);
        const float s = row_scale_from_max(m);
        const float inv = 1.0f / s;
        const int body = (cnt / 8) * 8;
        for (int i = lane; i < cnt; i += 64) {
            const float v = h2f(src[g0 + i]) * inv;
            const int32_t c = i < body ? cvt_rne_sat(v) : (int32_t)__builtin_roundf(v);
            const int8_t code = (int8_t)sat8(c);
            dst[g0 + i] = code;
            if (sh) {
                const int dim = g0 + i;
                const float p = dim < da ? (float)code * s : 0.0f;
                sh[sh_index(h, nsl, dim / 64, ntile, key, dim % 64)] = p;
            }
        }
        if (lane == 0) scales[g] = s;
    }
}

}  // namespace cactus_hip
