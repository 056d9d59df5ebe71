// hip_common.h -- shared device helpers and host-side error plumbing for the
// gfx950 kernel library.  Compiled with -ffp-contract=off: every fused
// multiply-add below is written explicitly, matching where the reference
// fuses; every other fp operation rounds on its own.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <cstring>

#include "../../include/cactus_hip.h"

namespace cactus_hip {

// ----------------------------------------------------------------- host side
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define CH_REQUIRE(cond, msg)                                                   \
    do {                                                                        \
        if (!(cond)) return ::cactus_hip::fail(CACTUS_HIP_EINVAL, msg);         \
    } while (0)

#define CH_HIP(call)                                                            \
    do {                                                                        \
        hipError_t e_ = (call);                                                 \
        if (e_ != hipSuccess)                                                   \
            return ::cactus_hip::fail(CACTUS_HIP_ERUNTIME,                      \
                                      std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Value product tiles (kv_shadow.hip): an fp32 mirror of the INT8 value
// cache, per (kv head, 64-dim slice) a run of 64-key tiles laid out
// [key / 4][64 dims][4 keys], so one 16-byte load per lane (lane = dim)
// brings four consecutive keys of a dimension and a wave's load of a key
// quad is one contiguous kilobyte.  ntile = ceil(capacity / 64).
constexpr int SH_TILE_KEYS = 64;
constexpr size_t SH_TILE_FLOATS = (size_t)SH_TILE_KEYS * 64;     // 16 KB per tile
__host__ __device__ inline size_t sh_region_floats(size_t ntile) { return ntile * SH_TILE_FLOATS; }
__host__ __device__ inline size_t sh_index(int kvh, int nsl, int sl, size_t ntile, size_t key, int dl) {
    return ((size_t)(kvh * nsl + sl) * ntile * SH_TILE_KEYS + (key & ~(size_t)3)) * 64 + (size_t)dl * 4 + (key & 3);
}

// Per-(device, stream, kind) scratch buffers of the library (runtime.hip).
// A buffer grows to 1.25x the request when too small.  The buffer it
// replaces is freed once the work queued on the stream before the growth has
// finished (an event, polled on later calls), unless it was handed out
// while the stream was being captured into a graph: a graph may replay it
// at any time, so it is kept until the stream is destroyed
// (cactus_hip_stream_destroy), which frees every buffer of the stream.
// `zero`: a new buffer is zero-filled on the stream (a fill kernel, safe to
// capture) before its first use.
enum ScratchKind {
    SCR_GEMM_ACT = 0,    // matmul activation codes + row scales
    SCR_ATTN,            // exact attention weights, block maxima and sums
    SCR_LM,              // LM head partial maxima + completion counter
    SCR_FAST_PART,       // split-K attention partials
    SCR_FAST_CNT,        // split-K attention completion counters
    SCR_KINDS
};
int stream_scratch(int kind, void* stream, size_t bytes, bool zero, void** out);
// frees every scratch buffer of `stream` (all devices) after synchronizing it
int stream_scratch_release(void* stream);

// Device RoPE tables (fp16 cos/sin [npos][head_dim/2]) built on the host,
// cached per (device, head_dim, theta); grows to at least npos positions.
struct RopeTable {
    uint16_t* cos_d = nullptr;
    uint16_t* sin_d = nullptr;
    size_t npos = 0;
};
// copies the table's pointers and length out under the lock (a concurrent grow
// replaces the map entry)
int rope_table(size_t npos, size_t head_dim, float theta, RopeTable* out);

// fp32 -> fp16 bit pattern on the host: round to nearest even with one
// rounding step (subnormals, overflow to inf, quiet NaN).  Used for tables
// built on the host.
inline uint16_t host_f2h(float f) {
    const double d = (double)f;  // exact
    uint64_t b;
    memcpy(&b, &d, 8);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const uint64_t a = b & 0x7FFFFFFFFFFFFFFFull;
    const int e = (int)(a >> 52);
    if (e == 0x7FF) return sign | ((a & 0xFFFFFFFFFFFFFull) ? 0x7E00 : 0x7C00);
    if (a == 0) return sign;
    const uint64_t mant = (a & 0xFFFFFFFFFFFFFull) | (1ull << 52);  // f is normal as a double
    const int ex = e - 1023;
    if (ex > 15) return sign | 0x7C00;
    const int shift = ex >= -14 ? 42 : 42 + (-14 - ex);
    if (shift > 63) return sign;
    uint64_t q = mant >> shift;
    const uint64_t rem = mant & ((1ull << shift) - 1);
    const uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    const uint32_t r = ex >= -14 ? ((uint32_t)(ex + 15) << 10) + (uint32_t)(q - 1024) : (uint32_t)q;
    if (r >= 0x7C00) return sign | 0x7C00;
    return sign | (uint16_t)r;
}

// --------------------------------------------------------------- device side
typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
// fp32 -> fp16, round to nearest even, applied to an already-rounded fp32
// value.  The empty asm keeps the compiler from folding the producing fp32
// multiply/add into v_fma_mixlo_f16, which would round only once (to fp16)
// where the reference rounds twice (to fp32, then to fp16).
__device__ __forceinline__ float fp32_barrier(float f) {
    asm volatile("" : "+v"(f));
    return f;
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (f16)fp32_barrier(f));
}
__device__ __forceinline__ f16 hbits(uint16_t h) { return __builtin_bit_cast(f16, h); }
__device__ __forceinline__ uint16_t bitsh(f16 h) { return __builtin_bit_cast(uint16_t, h); }
// native fp16 ops: one IEEE rounding each (v_add_f16 / v_mul_f16 / v_fma_f16)
__device__ __forceinline__ uint16_t hadd(uint16_t a, uint16_t b) { return bitsh(hbits(a) + hbits(b)); }
__device__ __forceinline__ uint16_t hmul(uint16_t a, uint16_t b) { return bitsh(hbits(a) * hbits(b)); }
__device__ __forceinline__ uint16_t hfma(uint16_t a, uint16_t b, uint16_t c) {
    return bitsh(__builtin_fmaf16(hbits(a), hbits(b), hbits(c)));
}

__device__ __forceinline__ float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }

// NEON vcvtq_s32_f32: truncate toward zero, saturating, NaN -> 0
__device__ __forceinline__ int32_t cvt_trunc_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}
// NEON vcvtnq_s32_f32: round to nearest even, saturating, NaN -> 0
__device__ __forceinline__ int32_t cvt_rne_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)__builtin_rintf(x);
}
__device__ __forceinline__ int32_t sat8(int32_t v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }
__device__ __forceinline__ float exp2_bits(int32_t zi) {
    return bits_f((uint32_t)((uint32_t)zi + 127u) << 23);
}

// expf used wherever the reference calls libm expf: x = k*ln2 + r (Cody-Waite,
// two-part ln2), e^r by its degree-12 Taylor polynomial in double (Horner,
// fused), one rounding to float.  Relative error of the double result is a
// few 1e-16, so the float result is the correctly rounded e^x except when
// e^x lies within ~1e-15 (relative) of a float rounding boundary.
__device__ __forceinline__ float cactus_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 100.0f) return __builtin_inff();
    if (xf < -110.0f) return 0.0f;
    const double LN2_HI = 6.93147180369123816490e-01;
    const double LN2_LO = 1.90821492927058770002e-10;
    double x = (double)xf;
    double k = __builtin_rint(x * 1.44269504088896338700e+00);
    double r = __builtin_fma(-k, LN2_HI, x);
    r = __builtin_fma(-k, LN2_LO, r);
    double p = 1.0 / 479001600.0;
    p = __builtin_fma(p, r, 1.0 / 39916800.0);
    p = __builtin_fma(p, r, 1.0 / 3628800.0);
    p = __builtin_fma(p, r, 1.0 / 362880.0);
    p = __builtin_fma(p, r, 1.0 / 40320.0);
    p = __builtin_fma(p, r, 1.0 / 5040.0);
    p = __builtin_fma(p, r, 1.0 / 720.0);
    p = __builtin_fma(p, r, 1.0 / 120.0);
    p = __builtin_fma(p, r, 1.0 / 24.0);
    p = __builtin_fma(p, r, 1.0 / 6.0);
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    uint64_t sb = (uint64_t)((int64_t)k + 1023) << 52;
    return (float)(p * __builtin_bit_cast(double, sb));
}

// fast_exp_f32x4 lane (reference kernel_utils.h:108-141)
__device__ __forceinline__ float fast_exp(float x) {
    x = __builtin_fmaxf(x, -87.0f);
    x = __builtin_fminf(x, 87.0f);
    float z = x * 1.4426950408889634f;
    int32_t zi = cvt_trunc_sat(z);
    float zf = z - (float)zi;
    if (zf < 0.0f) { zi -= 1; zf = zf + 1.0f; }
    float u = zf * 0.6931471805599453f;
    float p = 0.009618129842071803f;
    p = __builtin_fmaf(p, u, 0.05550410866482158f);
    p = __builtin_fmaf(p, u, 0.2402265069591007f);
    p = __builtin_fmaf(p, u, 0.6931471805599453f);
    p = __builtin_fmaf(p, u, 1.0f);
    return p * exp2_bits(zi);
}

// second-order 2^x block weight of cactus_attention_f16
// (reference kernel_attention.cpp:174-195); masked scores give 0
__device__ __forceinline__ float poly_exp_weight(float s, float bm) {
    if (s == -__builtin_inff()) return 0.0f;
    float x = s - bm;
    x = x * 1.442695f;
    int32_t xi = cvt_trunc_sat(x);
    float xf = x - (float)xi;
    float y = __builtin_fmaf(xf, 0.6931472f, 1.0f);
    float xf2 = xf * xf;
    y = __builtin_fmaf(xf2, 0.2402265f, y);
    return y * exp2_bits(xi);
}

// --------------------------------------------------------- LDS DMA (gfx950)
// global_load_lds_dword(x4): every active lane moves DW bytes from its own
// global address to LDS at lds_addr + lane * DW.  lds_addr must be uniform over
// the wave.  Completion is counted by vmcnt.
template <int DW>
__device__ __forceinline__ void lds_dma(const void* src, uint32_t lds_addr) {
    // M0 takes a scalar: the destination is uniform over the wave
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr);
    if constexpr (DW == 16)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                     : "memory");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds)
                     : "memory");
}

template <int N>
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// workgroup barrier that orders LDS only (outstanding DMA keeps flying)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Orders one wave's LDS writes before its later LDS reads (and reads before
// later writes).  LDS operations of one wavefront execute in program order,
// so no s_barrier and no counter wait are needed, only compiler ordering.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// acc = fma(w, p, acc) with w taken from lane k of each 16-lane row of wv
// (DPP row_newbcast): a row-replicated operand vector feeds 16 steps without
// an LDS broadcast read per step.  One VALU op per step, the same
// single rounding as fmaf.
template <int K>
__device__ __forceinline__ void fmac_row_bcast(float& acc, float wv, float p) {
    asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                 : "+v"(acc)
                 : "v"(wv), "v"(p), "n"(K));
}

// ---------------------------------------------------------- wave reductions
// Wave-wide max, uniform result; called by whole waves (all 64 lanes
// active).  DPP moves within each 16-lane row (VALU speed, no LDS round
// trips), then the four rows' maxima by readlane.  fmax is exact, so the
// reduction order does not matter.
template <int CTRL>
__device__ __forceinline__ float dpp_move_keep(float v) {
    const int b = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, 0xF, 0xF, false));
}
// Max over the 32-lane half of the wave holding this lane (lanes 0-31 or
// 32-63), every lane of the half gets it; whole waves.  DPP within each
// 16-lane row, then v_permlane16_swap_b32 (lane l and l ^ 16 exchange; the
// instruction as inline assembly: this compiler lowers the builtin's second
// result as a copy of the first).  fmax is exact: the order does not matter.
__device__ __forceinline__ float half_wave_max(float v) {
    v = __builtin_fmaxf(v, dpp_move_keep<0xB1>(v));
    v = __builtin_fmaxf(v, dpp_move_keep<0x4E>(v));
    v = __builtin_fmaxf(v, dpp_move_keep<0x141>(v));
    v = __builtin_fmaxf(v, dpp_move_keep<0x140>(v));
    float x = v, y = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
    return __builtin_fmaxf(x, y);
}
__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, dpp_move_keep<0xB1>(v));    // quad_perm [1,0,3,2]
    v = __builtin_fmaxf(v, dpp_move_keep<0x4E>(v));    // quad_perm [2,3,0,1]
    v = __builtin_fmaxf(v, dpp_move_keep<0x141>(v));   // row_half_mirror
    v = __builtin_fmaxf(v, dpp_move_keep<0x140>(v));   // row_mirror
    auto lane_v = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
    return __builtin_fmaxf(__builtin_fmaxf(lane_v(0), lane_v(16)), __builtin_fmaxf(lane_v(32), lane_v(48)));
}
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace cactus_hip
