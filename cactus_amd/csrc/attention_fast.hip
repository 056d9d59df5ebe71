// attention_fast.hip -- split-K decode attention over the KV cache
// (tolerance mode).
//
// The exact kernels of attention.hip reproduce the reference's value
// accumulation, one fp32 FMA chain per (head, dim) over the keys in order
// (kernel_attention.cpp:206-224, :416-441), which makes a decode step a
// latency-bound walk over the context.  This file computes the same
// function -- causal softmax(q k^T * scale) v with the reference's score
// operands (fp16 q, fp16 or INT8-times-scale k, fp32 sums) -- as an
// HBM-bound split-K ("flash decoding") reduction:
//
//   grid (splits, batch * kv_heads), 512 threads = 8 waves per workgroup;
//   workgroup s owns a split of 256 keys (32 per wave) of one KV head and
//   all the query heads that share it (GQA).  Each wave
//   scores its keys, the workgroup takes its local max M and weights
//   exp(s - M), and each wave accumulates its keys' value rows.  The
//   workgroup writes (M, sum, acc[d]) per query head; the last
//   workgroup of the KV head to finish (an atomic counter, reset by that
//   workgroup) combines the splits:
//       M* = max_s M_s,  L = sum_s e^(M_s - M*) l_s,
//       o  = fp16( sum_s e^(M_s - M*) acc_s / L ).
//
// Only the order of the fp32 sums and the exponential differ from the
// reference, so outputs agree with it to well within fp16 tolerance
// (|gpu - ref| <= 1e-3 + 1e-2 |ref|), not bit for bit.  Positions at or
// beyond cache_len read the FP16 "new" rows, as the hybrid kernel does
// (kernel_attention.cpp:372-388).
#include "hip_common.h"
#include "decode_device.h"

#include <map>
#include <mutex>
#include <utility>

namespace cactus_hip {

constexpr int FA_WAVES = 8;
constexpr int FA_THREADS = 64 * FA_WAVES;
// keys per wave: 32, eight waves: 256-key splits (measured on MI355X at 4096
// INT8 keys, 8 KV heads, 124 rotated caches: 10.6 us against 11.9 with four
// waves (128-key splits, 272 workgroups on 256 CUs), 11.2 with six, 12.3
// with twelve, 11.2 with eight waves of 16 keys); for FP16 rows 32 keys per
// wave also keep each of the reference's 32-key weight blocks inside one wave
template <bool HYBRID> constexpr int fa_kpw() { return 32; }
template <bool HYBRID> constexpr int fa_kpb() { return fa_kpw<HYBRID>() * FA_WAVES; }
constexpr int FA_MAX_SPLITS = 512;               // the combine keeps every split's (M, sum) in LDS
constexpr int FA_MAX_GQ = 4;

struct FastArgs {
    const uint16_t* q;        // prepared queries [B][Hq][d] (null with prep)
    const uint16_t* k;        // FP16 keys: [B][Skv][Hkv][d] (FP16 form) or new rows [B][new][Hkv][d]
    const uint16_t* v;
    const int8_t* kc;         // INT8 cache [B][cache][Hkv][d] (hybrid form)
    const int8_t* vc;
    const float* ks;          // [B][cache][Hkv][nqg]
    const float* vs;
    uint16_t* o;              // [B][Hq][d]
    float* part;              // [B*Hkv][nsplit][GQ][d + 4]: acc[d], M, sum, pad
    uint32_t* cnt;            // [B*Hkv], zero between launches
    int B, Hq, Hkv, nsplit, nqg;
    size_t Skv;               // FP16 form: keys; hybrid: cache_len + new_len
    size_t cache_len, new_len, pos_off, window;
    float scale;
    const uint32_t* dyn;      // decode step state {token, position, cache length, step} or null
    // fused head preparation (decode step): raw rows, norm weights, RoPE
    // tables and the cache the step's key and value are appended to
    const uint16_t* q_raw; const uint16_t* k_raw; const uint16_t* v_raw;
    const uint16_t* q_norm; const uint16_t* k_norm;
    const uint16_t* cos_t; const uint16_t* sin_t;
    float eps;
    uint32_t table_pos;
    int8_t* kc_w; int8_t* vc_w; float* ks_w; float* vs_w; float* vsh;
    size_t sh_ntile, max_cache;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane moves within 16-lane rows (no LDS traffic)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane j <- 7 - j within 8 lanes
constexpr int DPP_MIRROR = 0x140;      // lane j <- 15 - j within 16 lanes
constexpr int DPP_ROR4 = 0x124;        // row_ror:4
constexpr int DPP_ROR8 = 0x128;        // row_ror:8

// sum over aligned groups of N lanes (N = 4, 8 or 16), in every lane of the group
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<DPP_XOR1>(v);
    v += dpp_f<DPP_XOR2>(v);
    if (N >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if (N >= 16) v += dpp_f<DPP_MIRROR>(v);
    return v;
}
template <int N>
__device__ __forceinline__ float group_max(float v) {
    v = __builtin_fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = __builtin_fmaxf(v, dpp_f<DPP_XOR2>(v));
    if (N >= 8) v = __builtin_fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    if (N >= 16) v = __builtin_fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return v;
}
__device__ __forceinline__ float lane_bcast(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// wave-wide max / sum, uniform result
__device__ __forceinline__ float wave_max_u(float v) {
    v = group_max<16>(v);
    return __builtin_fmaxf(__builtin_fmaxf(lane_bcast(v, 0), lane_bcast(v, 16)),
                           __builtin_fmaxf(lane_bcast(v, 32), lane_bcast(v, 48)));
}
__device__ __forceinline__ float wave_sum_u(float v) {
    v = group_sum<16>(v);
    return (lane_bcast(v, 0) + lane_bcast(v, 16)) + (lane_bcast(v, 32) + lane_bcast(v, 48));
}
__device__ __forceinline__ float agent_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes as two 8-byte agent-scope loads (the widest lock-free atomic)
__device__ __forceinline__ f32x4 agent_load4(const float* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (f32x4){__builtin_bit_cast(float, (uint32_t)lo), __builtin_bit_cast(float, (uint32_t)(lo >> 32)),
                   __builtin_bit_cast(float, (uint32_t)hi), __builtin_bit_cast(float, (uint32_t)(hi >> 32))};
}
__device__ __forceinline__ void agent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS written by some lanes of a wave, then read by others: the wave's LDS
// operations execute in order, so only the compiler must not move them
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// HYBRID: INT8 cache + FP16 new rows; otherwise FP16 keys and values.
// PREP: q and the step's k come raw (head RMSNorm + RoPE here); one extra
// workgroup per KV head (blockIdx.x == nsplit) only prepares the step's k
// and appends it and v to the cache, off the splits' critical path.
//
// Lane layout: a key row is CPL 16-byte chunks; CPL consecutive lanes read
// one row (so each load instruction moves 64/CPL whole rows, coalesced) and
// a lane owns the DPL dims of its chunk for its NI keys (one per load
// instruction).  Scores are partial dots reduced over the CPL lanes of a
// row; value sums stay per lane and are reduced over the rows at the end.
template <bool HYBRID, bool PREP, int D, int GQ>
__global__ void __launch_bounds__(FA_THREADS) attn_splitk_kernel(FastArgs a) {
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static_assert(GQ >= 1 && GQ <= FA_MAX_GQ, "query heads per KV head");
    constexpr int ESZ = HYBRID ? 1 : 2;            // bytes per cached element
    constexpr int CPL = D * ESZ / 16;              // lanes (16-byte chunks) per row
    constexpr int DPL = 16 / ESZ;                  // dims per lane
    constexpr int R = 64 / CPL;                    // rows per load instruction
    constexpr int FA_KPW = fa_kpw<HYBRID>(), FA_KPB = fa_kpb<HYBRID>();
    constexpr int NI = FA_KPW / R;                 // load instructions (keys) per lane
    static_assert(NI >= 1, "keys per wave");
    static_assert(CPL >= 4 && CPL <= 16 && 64 % CPL == 0, "row layout");
    __shared__ __align__(16) uint16_t qs[GQ][D];   // prepared queries, fp16
    __shared__ __align__(16) uint16_t kn[D];       // prepared new key (PREP)
    __shared__ __align__(16) uint16_t tmp[FA_WAVES][D];
    __shared__ float redm[GQ][FA_WAVES], reds[GQ][FA_WAVES];
    __shared__ __align__(16) float vsum[FA_WAVES * 4 * GQ * D];   // value sums per 16-lane row
    __shared__ float ms[GQ * FA_MAX_SPLITS];       // combine: split maxima, then weights
    __shared__ float ls[GQ * FA_MAX_SPLITS];       // combine: split sums
    __shared__ float Ltot[GQ];
    __shared__ bool last;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cl = lane % CPL, rl = lane / CPL;
    const int bg = blockIdx.y;                    // b * Hkv + g
    const int b = bg / a.Hkv, g = bg % a.Hkv;
    const int s = blockIdx.x;

    size_t cache_len = a.cache_len, pos = a.pos_off, Skv = a.Skv;
    if (a.dyn) {
        cache_len = a.dyn[2];
        pos = a.dyn[1];
        Skv = cache_len + a.new_len;
    }
    // causal key range of the query (kernel_attention.cpp:78-96, :328-337)
    size_t kv_start = 0, kv_end = Skv;
    if (!HYBRID && a.window > 0 && a.window < Skv && pos > a.window) kv_start = pos - a.window;
    if (pos + 1 < kv_end) kv_end = pos + 1;
    const size_t k0 = kv_start + (size_t)s * FA_KPB;
    const size_t k1 = k0 + FA_KPB < kv_end ? k0 + FA_KPB : kv_end;
    const bool has_keys = k0 < kv_end;
    const bool has_new = HYBRID && has_keys && k1 > cache_len;
    const bool appends = PREP && s == a.nsplit;
    const bool prep_ok = !PREP || pos < a.table_pos;   // the host keeps positions inside the tables
    const size_t wk0 = k0 + (size_t)wid * FA_KPW;      // this wave's first key

    // ---- 0. (fused step) the head preparation's inputs, loaded first and
    // branch-free (clamped rows and table position; values unused where no
    // preparation runs), so preparing them waits for these only and the key
    // and value rows below stay in flight meanwhile
    constexpr int EPL = D / 64;                        // elements per lane of a row
    const bool do_q = PREP && prep_ok && wid < GQ && !appends;
    const bool do_k = PREP && prep_ok && (has_new || appends) && wid == GQ % FA_WAVES;
    uint16_t pq[EPL], pqn[EPL], pk[EPL], pkn[EPL];
    uint16_t pcv = 0, psv = 0;
    if constexpr (PREP) {
        const uint16_t* qsrc = a.q_raw + ((size_t)b * a.Hq + g * GQ + min(wid, GQ - 1)) * D;
        const uint16_t* ksrc = a.k_raw + ((size_t)b * a.Hkv + g) * D;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            pq[j] = qsrc[lane + 64 * j];
            pqn[j] = a.q_norm[lane + 64 * j];
            pk[j] = ksrc[lane + 64 * j];
            pkn[j] = a.k_norm[lane + 64 * j];
        }
        const size_t tpos = prep_ok ? pos : 0;
        const int hl = min(lane, D / 2 - 1);
        pcv = a.cos_t[tpos * (D / 2) + hl];
        psv = a.sin_t[tpos * (D / 2) + hl];
    }

    // ---- 1. key and value chunks, in flight first (key of instruction i:
    // wk0 + i*R + rl)
    // Branch-free: a lane without a cached key of its own reads row 0 (or a
    // stand-in when there is no cache) and its data are never used -- a
    // branch around the loads made the compiler wait for each instruction's
    // rows before issuing the next.
    i32x4 kch[NI], vch[NI];
    float ksc[NI], vsc[NI];
    const void* stand_in = PREP ? (const void*)a.q_raw : (const void*)a.q;
    const bool has_rows = HYBRID ? cache_len > 0 : Skv > 0;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const size_t kp = wk0 + (size_t)i * R + rl;
        const bool own = has_keys && kp < k1 && (!HYBRID || kp < cache_len);   // FP16 new rows: read below
        const size_t kr = own ? kp : 0;
        const char* kb = reinterpret_cast<const char*>(stand_in);
        const char* vb = kb;
        const float* ksp = reinterpret_cast<const float*>(stand_in);
        const float* vsp = ksp;
        if (has_rows) {
            if (HYBRID) {
                const size_t row = ((size_t)b * cache_len + kr) * a.Hkv + g;
                kb = reinterpret_cast<const char*>(a.kc + row * D);
                vb = reinterpret_cast<const char*>(a.vc + row * D);
                // scales carry no batch offset (kernel_attention.cpp:353, :424)
                ksp = a.ks + (kr * a.Hkv + g) * a.nqg;
                vsp = a.vs + (kr * a.Hkv + g) * a.nqg;
            } else {
                const size_t row = ((size_t)b * Skv + kr) * a.Hkv + g;
                kb = reinterpret_cast<const char*>(a.k + row * D);
                vb = reinterpret_cast<const char*>(a.v + row * D);
            }
        }
        kch[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(kb) + cl);
        vch[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(vb) + cl);
        ksc[i] = HYBRID ? *ksp : 1.0f;
        vsc[i] = HYBRID ? *vsp : 1.0f;
    }

    // ---- 2. queries (and the step's new key) into LDS
    if (PREP) {
        const int half = D / 2, end8 = (D / 8) * 8, vh = (half / 8) * 8;
        // q/k head RMSNorm then RoPE at the step's position, one wave per row
        // (rope_row's arithmetic, with this lane's table entries in registers)
        auto prep_row = [&](const uint16_t (&xr)[EPL], const uint16_t (&nr)[EPL], uint16_t* dst) {
            uint16_t* xs = tmp[wid];
#pragma unroll
            for (int j = 0; j < EPL; j++) xs[lane + 64 * j] = xr[j];
            wave_lds_sync();
            float inv1[1];
            uint16_t hinv1[1];
            rms_stats_rows<D, 1>(xs, D, a.eps, inv1, hinv1);
            const float inv = inv1[0];
            const uint16_t hinv = hinv1[0];
            uint16_t yv[EPL];
#pragma unroll
            for (int j = 0; j < EPL; j++) yv[j] = rms_apply(xr[j], nr[j], lane + 64 * j, end8, inv, hinv);
            wave_lds_sync();
#pragma unroll
            for (int j = 0; j < EPL; j++) xs[lane + 64 * j] = yv[j];
            wave_lds_sync();
            if (lane < half) {
                const uint16_t x1 = xs[lane], x2 = xs[lane + half];
                uint16_t o1, o2;
                if (lane < vh) {
                    o1 = hfma(x2 ^ 0x8000u, psv, hmul(x1, pcv));
                    o2 = hfma(x1, psv, hmul(x2, pcv));
                } else {
                    const float fa = h2f(x1), fb = h2f(x2), cf = h2f(pcv), sf = h2f(psv);
                    o1 = f2h(fa * cf - fb * sf);
                    o2 = f2h(fb * cf + fa * sf);
                }
                dst[lane] = o1;
                dst[lane + half] = o2;
            }
        };
        if (do_q) prep_row(pq, pqn, qs[wid]);
        // the new key: wave GQ, or wave 0 after its query head when GQ == 4
        if (do_k) prep_row(pk, pkn, kn);
    } else {
        for (int i = tid; i < GQ * D; i += FA_THREADS)
            qs[i / D][i % D] = a.q[((size_t)b * a.Hq + g * GQ + i / D) * D + i % D];
    }
    __syncthreads();
    if (appends && prep_ok && cache_len < a.max_cache && wid == GQ % FA_WAVES) {
        // the step's key (prepared) and value to slot cache_len
        // (engine_cache.cpp:234-267), with the exact mode's product tiles
        const int ng = (D + 127) / 128;
        const size_t row = (size_t)cache_len * a.Hkv + g;
        kv_append_row(kn, a.kc_w + row * D, a.ks_w + row * ng, D);
        kv_append_row(a.v_raw + ((size_t)b * a.Hkv + g) * D, a.vc_w + row * D, a.vs_w + row * ng, D, a.vsh,
                      a.sh_ntile, cache_len, g);
    }
    if (appends) return;   // the appending workgroup holds no split
    // this lane's query dims, fp32, and (INT8) their sum
    float qv[GQ][DPL], qsum[GQ];
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        qsum[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            qv[h][e] = h2f(qs[h][cl * DPL + e]);
            qsum[h] += qv[h][e];
        }
    }

    // ---- 3. scores of the lane's NI keys
    float sc[NI][GQ];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const size_t kp = wk0 + (size_t)i * R + rl;
        const bool valid = has_keys && kp < k1;
        float acc[GQ];
#pragma unroll
        for (int h = 0; h < GQ; h++) acc[h] = 0.0f;
        if (HYBRID && valid && kp >= cache_len) {
            // an FP16 new row (kernel_attention.cpp:372-388)
            const uint16_t* kr = PREP ? kn : a.k + (((size_t)b * a.new_len + (kp - cache_len)) * a.Hkv + g) * D;
#pragma unroll
            for (int e = 0; e < DPL; e++) {
                const float kv = h2f(kr[cl * DPL + e]);
#pragma unroll
                for (int h = 0; h < GQ; h++) acc[h] = __builtin_fmaf(qv[h][e], kv, acc[h]);
            }
        } else {
            const uint32_t w4[4] = {(uint32_t)kch[i].x, (uint32_t)kch[i].y, (uint32_t)kch[i].z, (uint32_t)kch[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (HYBRID) {
                    // code + 128 as an unsigned byte; 128 * sum(q) comes off below
                    const uint32_t u = w4[j] ^ 0x80808080u;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float kv = (float)((u >> (8 * e)) & 0xFFu);
#pragma unroll
                        for (int h = 0; h < GQ; h++) acc[h] = __builtin_fmaf(qv[h][j * 4 + e], kv, acc[h]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const float kv = h2f((uint16_t)(w4[j] >> (16 * e)));
#pragma unroll
                        for (int h = 0; h < GQ; h++) acc[h] = __builtin_fmaf(qv[h][j * 2 + e], kv, acc[h]);
                    }
                }
            }
            if (HYBRID)
#pragma unroll
                for (int h = 0; h < GQ; h++) acc[h] = __builtin_fmaf(-128.0f, qsum[h], acc[h]);
        }
        // the row's CPL partial dots
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            acc[h] = group_sum<CPL>(acc[h]);
            const bool cached = HYBRID && kp < cache_len;
            sc[i][h] = valid ? acc[h] * (cached ? ksc[i] : 1.0f) * a.scale : -__builtin_inff();
        }
    }

    // ---- 4. weights relative to this wave's max: no barrier, so a wave
    // whose keys arrived goes on to its values while others still wait.
    // The workgroup max M and each wave's factor e^(m_w - M) enter once, in
    // the sum of the waves' rows below.
    constexpr float LOG2E = 1.4426950408889634f;
    float wm[GQ];
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        float m = sc[0][h];
#pragma unroll
        for (int i = 1; i < NI; i++) m = __builtin_fmaxf(m, sc[i][h]);
        wm[h] = wave_max_u(m);
        if (lane == 0) redm[h][wid] = wm[h];
    }
    float p[NI][GQ];
    if (HYBRID) {
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int h = 0; h < GQ; h++)
                p[i][h] = sc[i][h] > -__builtin_inff() ? fast_exp2((sc[i][h] - wm[h]) * LOG2E) : 0.0f;
    } else {
        // the reference weighs the first floor(n/4)*4 keys of each 32-key
        // block (blocks from kv_start, n = min(32, Skv - block start)) by its
        // second-order 2^x polynomial relative to the block max, the rest by
        // exp (kernel_attention.cpp:160-204).  A wave holds exactly one
        // block here (32 keys from a block boundary), so the block max is the
        // wave max and the block's factor is the wave's.
        static_assert(HYBRID || FA_KPW == 32, "one 32-key block per wave");
        const int bpoly = (int)(min((size_t)32, Skv > wk0 ? Skv - wk0 : (size_t)0) / 4) * 4;
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            const float bm = wm[h];
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int in_blk = i * R + rl;
                const float sv = sc[i][h];
                float w = 0.0f;
                if (sv > -__builtin_inff())
                    w = in_blk < bpoly ? poly_exp_weight(sv, bm) : fast_exp2((sv - bm) * LOG2E);
                p[i][h] = w;
            }
        }
    }
    // block sum of the weights: every key counted once (by its cl == 0 lane)
#pragma unroll
    for (int h = 0; h < GQ; h++) {
        float t = 0.0f;
        if (cl == 0)
#pragma unroll
            for (int i = 0; i < NI; i++) t += p[i][h];
        t = wave_sum_u(t);
        if (lane == 0) reds[h][wid] = t;
    }

    // ---- 5. values: av[h][e] over the lane's keys; the rows of every wave
    // are summed through LDS
    float av[GQ][DPL];
#pragma unroll
    for (int h = 0; h < GQ; h++)
#pragma unroll
        for (int e = 0; e < DPL; e++) av[h][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const size_t kp = wk0 + (size_t)i * R + rl;
        float vv[DPL];
        float f = 1.0f;
        if (HYBRID && has_keys && kp < k1 && kp >= cache_len) {
            const uint16_t* vr = PREP ? a.v_raw + ((size_t)b * a.Hkv + g) * D
                                      : a.v + (((size_t)b * a.new_len + (kp - cache_len)) * a.Hkv + g) * D;
#pragma unroll
            for (int e = 0; e < DPL; e++) vv[e] = h2f(vr[cl * DPL + e]);
        } else {
            const uint32_t w4[4] = {(uint32_t)vch[i].x, (uint32_t)vch[i].y, (uint32_t)vch[i].z, (uint32_t)vch[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (HYBRID) {
#pragma unroll
                    for (int e = 0; e < 4; e++) vv[j * 4 + e] = (float)(int8_t)(w4[j] >> (8 * e));
                } else {
#pragma unroll
                    for (int e = 0; e < 2; e++) vv[j * 2 + e] = h2f((uint16_t)(w4[j] >> (16 * e)));
                }
            }
            if (HYBRID) f = vsc[i];
            if (!(has_keys && kp < k1)) {
                // a key outside the split: its (unused) data contribute nothing
                f = 0.0f;
#pragma unroll
                for (int e = 0; e < DPL; e++) vv[e] = 0.0f;
            }
        }
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            const float w = p[i][h] * f;
#pragma unroll
            for (int e = 0; e < DPL; e++) av[h][e] = __builtin_fmaf(w, vv[e], av[h][e]);
        }
    }
    // rows of one 16-lane group first (DPP rotations keep the dims aligned:
    // lanes i, i + CPL, ... of a row share their dims), then
    // vsum[wave][row16][h][d] from the first CPL lanes of each 16-lane row
#pragma unroll
    for (int h = 0; h < GQ; h++)
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            float v = av[h][e];
            if (CPL == 4) v += dpp_f<DPP_ROR4>(v);
            if (CPL <= 8) v += dpp_f<DPP_ROR8>(v);
            av[h][e] = v;
        }
    if ((lane & 15) < CPL)
#pragma unroll
        for (int h = 0; h < GQ; h++) {
            float* dst = &vsum[((wid * 4 + (lane >> 4)) * GQ + h) * D + cl * DPL];
#pragma unroll
            for (int e = 0; e < DPL; e += 4)
                *reinterpret_cast<f32x4*>(dst + e) = (f32x4){av[h][e], av[h][e + 1], av[h][e + 2], av[h][e + 3]};
        }
    __syncthreads();

    // ---- 6. this split's partial: (M, sum, acc[d]) per query head, M the
    // workgroup max, each wave's rows and weight sum scaled by e^(m_w - M);
    // written with agent-scope stores (visible to the combining workgroup on
    // any XCD without a cache writeback)
    constexpr int PS = D + 4;                     // floats per (split, head): acc[D], M, sum, 2 pad
    float* part = a.part + ((size_t)bg * a.nsplit + s) * GQ * PS;
    auto wave_factors = [&](int h, float (&ew)[FA_WAVES]) -> float {
        float mx = redm[h][0];
#pragma unroll
        for (int w = 1; w < FA_WAVES; w++) mx = __builtin_fmaxf(mx, redm[h][w]);
#pragma unroll
        for (int w = 0; w < FA_WAVES; w++) {
            const float m = redm[h][w];
            ew[w] = m > -__builtin_inff() ? fast_exp2((m - mx) * LOG2E) : 0.0f;
        }
        return mx;
    };
    for (int i = tid; i < GQ * D; i += FA_THREADS) {
        const int h = i / D, dm = i % D;
        float ew[FA_WAVES];
        wave_factors(h, ew);
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < FA_WAVES; w++) {
            const float* r = &vsum[(w * 4 * GQ + h) * D + dm];
            t = __builtin_fmaf(ew[w], (r[0] + r[GQ * D]) + (r[2 * GQ * D] + r[3 * GQ * D]), t);
        }
        agent_store(part + h * PS + dm, t);
    }
    if (tid < GQ) {
        float ew[FA_WAVES];
        const float mx = wave_factors(tid, ew);
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < FA_WAVES; w++) l = __builtin_fmaf(ew[w], reds[tid][w], l);
        agent_store(part + tid * PS + D, has_keys ? mx : -__builtin_inff());
        agent_store(part + tid * PS + D + 1, l);
    }
    // every store of the workgroup has completed before the count goes up.
    // The count is relaxed: the partials are agent-scope atomic stores whose
    // acknowledgements come from the coherence point, so they are visible
    // there before the increment issues; an acquire-release increment (an
    // L2 writeback before it and an invalidate after, per workgroup) cost
    // 0.45-0.55 us more per launch for the same results.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.cnt + bg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(a.nsplit - 1);
    __syncthreads();
    if (!last) return;

    // ---- 7. the last workgroup of this KV head combines the splits that
    // hold keys (nact <= FA_MAX_SPLITS, checked on the host), with agent-scope
    // loads.  Thread t owns four consecutive outputs (group t % NG) and the
    // splits t / NG, t / NG + TPG, ...: all of its 16-byte column loads and
    // the splits' (M, sum) pairs are issued together; one wave per query head
    // then forms M* and the weights e^(M_s - M*); the TPG partial sums of a
    // group meet in LDS.
    const int nact = kv_end > kv_start ? (int)((kv_end - kv_start + FA_KPB - 1) / FA_KPB) : 0;
    const float* pb = a.part + (size_t)bg * a.nsplit * GQ * PS;
    constexpr int NG = GQ * D / 4;                // float4 output groups
    constexpr int TPG = FA_THREADS / NG;          // threads (split lanes) per group
    // Up to NR splits per thread (decode at a few thousand keys): the TPG
    // consecutive lanes of one output group hold splits sj, sj + TPG, ...
    // with their (M, sum) in registers; M*, the weights' sum and the
    // weighted partial rows meet by DPP within the lane group, with no LDS
    // and no barrier.
    constexpr int NR = 4;
    if constexpr (TPG >= 4 && TPG <= 16) {
        if (nact <= TPG * NR) {
            const int gi = tid / TPG, sj = tid % TPG;
            const int gh = (gi * 4) / D, gd = (gi * 4) % D;
            f32x4 cr[NR];
            float mr[NR], lr[NR];
#pragma unroll
            for (int u = 0; u < NR; u++) {
                const int t = sj + u * TPG;
                cr[u] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                mr[u] = -__builtin_inff();
                lr[u] = 0.0f;
                if (t < nact) {
                    const float* pt = pb + ((size_t)t * GQ + gh) * PS;
                    cr[u] = agent_load4(pt + gd);
                    mr[u] = agent_load(pt + D);
                    lr[u] = agent_load(pt + D + 1);
                }
            }
            float mx = mr[0];
#pragma unroll
            for (int u = 1; u < NR; u++) mx = __builtin_fmaxf(mx, mr[u]);
            mx = group_max<TPG>(mx);
            float L = 0.0f;
            f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int u = 0; u < NR; u++) {
                const float e = mr[u] > -__builtin_inff() ? fast_exp2((mr[u] - mx) * LOG2E) : 0.0f;
                L = __builtin_fmaf(e, lr[u], L);
                acc.x = __builtin_fmaf(e, cr[u].x, acc.x);
                acc.y = __builtin_fmaf(e, cr[u].y, acc.y);
                acc.z = __builtin_fmaf(e, cr[u].z, acc.z);
                acc.w = __builtin_fmaf(e, cr[u].w, acc.w);
            }
            L = group_sum<TPG>(L);
            acc.x = group_sum<TPG>(acc.x);
            acc.y = group_sum<TPG>(acc.y);
            acc.z = group_sum<TPG>(acc.z);
            acc.w = group_sum<TPG>(acc.w);
            if (sj == 0) {
                uint16_t* out = a.o + ((size_t)b * a.Hq + g * GQ + gh) * D + gd;
                const uint32_t lo = (uint32_t)f2h(L > 0.0f ? acc.x / L : 0.0f) |
                                    ((uint32_t)f2h(L > 0.0f ? acc.y / L : 0.0f) << 16);
                const uint32_t hi = (uint32_t)f2h(L > 0.0f ? acc.z / L : 0.0f) |
                                    ((uint32_t)f2h(L > 0.0f ? acc.w / L : 0.0f) << 16);
                *reinterpret_cast<uint2*>(out) = make_uint2(lo, hi);
            }
            if (tid == 0) __hip_atomic_store(a.cnt + bg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    constexpr int NCH = 96 / TPG > 0 ? (96 / TPG < 24 ? 96 / TPG : 24) : 1;   // loads in flight per thread
    static_assert(FA_THREADS % NG == 0, "output groups");
    const int gi = tid % NG, sj = tid / NG;
    const int gh = (gi * 4) / D, gd = (gi * 4) % D;
    f32x4 cv[NCH];
#pragma unroll
    for (int u = 0; u < NCH; u++) {
        const int t = sj + u * TPG;
        cv[u] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        if (t < nact)
            cv[u] = agent_load4(pb + ((size_t)t * GQ + gh) * PS + gd);
    }
    for (int i = tid; i < nact * GQ; i += FA_THREADS) {
        const float* pt = pb + (size_t)i * PS + D;
        ms[i] = agent_load(pt);
        ls[i] = agent_load(pt + 1);
    }
    __syncthreads();
    if (wid < GQ) {
        float mx = -__builtin_inff();
        for (int t = lane; t < nact; t += 64) mx = __builtin_fmaxf(mx, ms[t * GQ + wid]);
        mx = wave_max_u(mx);
        float L = 0.0f;
        for (int t = lane; t < nact; t += 64) {
            const float m = ms[t * GQ + wid];
            const float e = m > -__builtin_inff() ? fast_exp2((m - mx) * LOG2E) : 0.0f;
            ms[t * GQ + wid] = e;
            L = __builtin_fmaf(e, ls[t * GQ + wid], L);
        }
        L = wave_sum_u(L);
        if (lane == 0) Ltot[wid] = L;
    }
    __syncthreads();
    f32x4 acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < NCH; u++) {
        const int t = sj + u * TPG;
        if (t < nact) {
            const float e = ms[t * GQ + gh];
            acc.x = __builtin_fmaf(e, cv[u].x, acc.x);
            acc.y = __builtin_fmaf(e, cv[u].y, acc.y);
            acc.z = __builtin_fmaf(e, cv[u].z, acc.z);
            acc.w = __builtin_fmaf(e, cv[u].w, acc.w);
        }
    }
    for (int t = sj + NCH * TPG; t < nact; t += TPG) {
        const f32x4 v = agent_load4(pb + ((size_t)t * GQ + gh) * PS + gd);
        const float e = ms[t * GQ + gh];
        acc.x = __builtin_fmaf(e, v.x, acc.x);
        acc.y = __builtin_fmaf(e, v.y, acc.y);
        acc.z = __builtin_fmaf(e, v.z, acc.z);
        acc.w = __builtin_fmaf(e, v.w, acc.w);
    }
    f32x4* red4 = reinterpret_cast<f32x4*>(vsum);   // [TPG][NG]
    red4[sj * NG + gi] = acc;
    __syncthreads();
    if (tid < NG) {
        f32x4 t4 = red4[tid];
        for (int j2 = 1; j2 < TPG; j2++) {
            const f32x4 v = red4[j2 * NG + tid];
            t4.x += v.x; t4.y += v.y; t4.z += v.z; t4.w += v.w;
        }
        const float L = Ltot[gh];
        uint16_t* out = a.o + ((size_t)b * a.Hq + g * GQ + gh) * D + gd;
        const uint32_t lo = (uint32_t)f2h(L > 0.0f ? t4.x / L : 0.0f) | ((uint32_t)f2h(L > 0.0f ? t4.y / L : 0.0f) << 16);
        const uint32_t hi = (uint32_t)f2h(L > 0.0f ? t4.z / L : 0.0f) | ((uint32_t)f2h(L > 0.0f ? t4.w / L : 0.0f) << 16);
        *reinterpret_cast<uint2*>(out) = make_uint2(lo, hi);
    }
    if (tid == 0) __hip_atomic_store(a.cnt + bg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------ prefill (many query rows)
// Causal hybrid attention of a prefill chunk -- S query rows against the
// INT8 cache and the chunk's own FP16 rows (kernel_attention.cpp:257-482)
// -- as flash attention on FP16 MFMA (v_mfma_f32_16x16x32_f16), tolerance
// mode.  A workgroup owns 16 * W query vectors of one KV head (vector m:
// row m / GQ, head m % GQ; 16 per wave) and walks the keys in 32-key tiles
// staged in LDS as FP16.  Key codes are exact in fp16 and their per-key
// scale multiplies the score (s = scale_k (q . code) scale); value rows are
// staged as fp16(code * scale_v) (normal-range fp16, relative error 2^-12),
// so the weights enter the P V product as fp16(p) without a scale that
// could push them into fp16's subnormal range.  FP16 rows carry scale 1.  Each wave computes the tile's
// transposed scores S^T = K Q^T, so that a lane's scores are already the A
// operand of the P V product for the same keys (lane l holds vector l % 16
// and keys {4g + i, 16 + 4g + i}, g = l / 16); the V operand reads the
// tile transposed in LDS in that key order.  The online softmax state
// (running max, sum) stays in fp32 per vector, the output accumulates in
// fp32 and is divided once at the end.
constexpr int PF_T = 32;    // keys per tile

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
    const uint16_t* q;        // [B][S][Hq][D]
    const int8_t* kc;         // [B][cache][Hkv][D]
    const int8_t* vc;
    const float* ks;          // [cache][Hkv][nqg] (no batch offset, kernel_attention.cpp:353, :424)
    const float* vs;
    const uint16_t* kn;       // [B][new][Hkv][D]
    const uint16_t* vn;
    uint16_t* o;              // [B][S][Hq][D]
    float* part;              // split partials [B*Hkv][nqb][nsplit][16 W][D + 4]: acc[D], max, sum
    int B, S, Hq, Hkv, nqg;
    int nsplit, tps;          // key splits per query block (1: no partials), tiles per split
    size_t cache_len, new_len, pos_off;
    float scale;
};

// tiles (32 keys) a query block reads: keys up to its last row's position
__device__ __forceinline__ int pf_block_tiles(const PrefillArgs& a, int gm0, int nv, int gq) {
    const int last_row = min(a.S - 1, (gm0 + nv - 1) / gq);
    size_t kv_end = a.pos_off + (size_t)last_row + 1;
    const size_t Skv = a.cache_len + a.new_len;
    if (kv_end > Skv) kv_end = Skv;
    return (int)((kv_end + PF_T - 1) / PF_T);
}

// max / sum over the four lanes l % 16 == c of a wave (lanes c, c + 16,
// c + 32, c + 48), same bits in all four: v_permlane16_swap_b32 /
// v_permlane32_swap_b32 on a value and its copy leave the lane's own value
// in one register and its partner's (lane l ^ 16, l ^ 32) in the other.
// Issued as inline assembly: the builtins' second result is lowered as a
// copy of the first by this compiler.
__device__ __forceinline__ void swap_pair16(float v, float& x, float& y) {
    x = v;
    y = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ void swap_pair32(float v, float& x, float& y) {
    x = v;
    y = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
}
__device__ __forceinline__ float xrow_max(float v) {
    float x, y;
    swap_pair16(v, x, y);
    swap_pair32(__builtin_fmaxf(x, y), x, y);
    return __builtin_fmaxf(x, y);
}
__device__ __forceinline__ float xrow_sum(float v) {
    float x, y;
    swap_pair16(v, x, y);
    swap_pair32(x + y, x, y);
    return x + y;
}

template <int D, int GQ, int W, int NB, int VB>
__global__ void __launch_bounds__(64 * W) attn_prefill_mfma_kernel(PrefillArgs a) {
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static_assert(64 * W >= 2 * D, "staging threads: 32 keys x D/16 pieces");
    constexpr int NV = 16 * W * VB;            // query vectors per workgroup (16 VB per wave)
    constexpr int KS = D + 8;                  // LDS row of a key tile, halves
    constexpr int VS = PF_T + 8;               // LDS row of a transposed value tile, halves
    constexpr int CPR = D / 16;                // 16-dim pieces per key row
    constexpr int NC = D / 32;                 // 32-dim MFMA steps of a score
    constexpr int ND = D / 16;                 // 16-dim output blocks
    __shared__ __align__(16) _Float16 ksh[2][PF_T][KS];
    __shared__ __align__(16) _Float16 vt[2][D][VS];
    __shared__ __align__(16) float ksc[2][PF_T];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane >> 4, lr = lane & 15;
    const int bg = blockIdx.y, b = bg / a.Hkv, g = bg % a.Hkv;
    const int qb = blockIdx.x / a.nsplit, sp_ = blockIdx.x % a.nsplit;
    const int gm0 = qb * NV;
    const size_t Skv = a.cache_len + a.new_len;
    const int last_row = min(a.S - 1, (gm0 + NV - 1) / GQ);
    size_t kv_end = a.pos_off + (size_t)last_row + 1;
    if (kv_end > Skv) kv_end = Skv;
    const int ntile_all = (int)((kv_end + PF_T - 1) / PF_T);
    // this workgroup's split of the tiles
    const int t_begin = sp_ * a.tps;
    const int nt = min(ntile_all - t_begin, a.tps);
    if (nt <= 0) return;   // no keys here; the combine counts only splits that hold some

    // ---- this lane's query vectors: lr of each of the wave's VB blocks of
    // 16 (B operands of S^T = K Q^T; every key and value fragment read from
    // LDS feeds VB MFMAs, and the blocks' softmax chains interleave)
    int vm[VB], vrow[VB];
    bool vok[VB];
    size_t vpos[VB];
#pragma unroll
    for (int vb = 0; vb < VB; vb++) {
        vm[vb] = gm0 + (wid * VB + vb) * 16 + lr;
        vrow[vb] = vm[vb] / GQ;
        vok[vb] = vrow[vb] < a.S;
        vpos[vb] = a.pos_off + (size_t)vrow[vb];
    }
    // the wave's first row (its smallest position) and whether all its rows exist
    const int wrow0 = (gm0 + wid * 16 * VB) / GQ, wrow1 = (gm0 + wid * 16 * VB + 16 * VB - 1) / GQ;
    const bool wave_all_rows = wrow1 < a.S;
    const size_t wave_min_pos = a.pos_off + (size_t)wrow0;
    h16x8 qv[VB][NC];
#pragma unroll
    for (int vb = 0; vb < VB; vb++) {
        const uint16_t* qp =
            a.q + (((size_t)b * a.S + (vok[vb] ? vrow[vb] : 0)) * a.Hq + (size_t)g * GQ + vm[vb] % GQ) * D;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint4 u = vok[vb] ? *reinterpret_cast<const uint4*>(qp + 32 * c + 8 * lg) : make_uint4(0, 0, 0, 0);
            qv[vb][c] = __builtin_bit_cast(h16x8, u);
        }
    }

    // ---- tile staging: thread -> (key sj, 16-dim piece sp), lanes of a
    // wave on 32 different keys so the transposed value writes spread over
    // the LDS banks.  Every tile issues the same loads -- the key's INT8
    // cache piece and its FP16 new-row piece, each from a clamped in-bounds
    // row -- and picks one when staging, so the loads take no branch and
    // the compiler keeps NB tiles in flight (slot t % NB).
    const int sj = tid % PF_T, sp = tid / PF_T;
    const bool stager = sp < CPR;
    const size_t rstride = (size_t)a.Hkv * D;   // elements between consecutive keys
    const int8_t* kcb = nullptr;
    const int8_t* vcb = nullptr;
    const float* ksb = nullptr;
    const float* vsb = nullptr;
    const uint16_t* knb = nullptr;
    const uint16_t* vnb = nullptr;
    {
        // a valid stand-in for a missing part (its values are never used)
        const uint16_t* any16 = a.q;
        if (a.cache_len > 0) {
            kcb = a.kc + ((size_t)b * a.cache_len * a.Hkv + g) * D + 16 * sp;
            vcb = a.vc + ((size_t)b * a.cache_len * a.Hkv + g) * D + 16 * sp;
            ksb = a.ks + (size_t)g * a.nqg;
            vsb = a.vs + (size_t)g * a.nqg;
        } else {
            kcb = vcb = reinterpret_cast<const int8_t*>(any16);
            ksb = vsb = reinterpret_cast<const float*>(any16);
        }
        if (a.new_len > 0) {
            knb = a.kn + ((size_t)b * a.new_len * a.Hkv + g) * D + 16 * sp;
            vnb = a.vn + ((size_t)b * a.new_len * a.Hkv + g) * D + 16 * sp;
        } else {
            knb = vnb = any16;
        }
    }
    const int clen = (int)a.cache_len, nlen = (int)a.new_len;
    const size_t cstride = a.cache_len > 0 ? rstride : 0;   // stand-ins do not move
    const size_t nstride = a.new_len > 0 ? rstride : 0;
    const size_t sstride = a.cache_len > 0 ? (size_t)a.Hkv * a.nqg : 0;
    struct Raw {
        uint4 kc, vc;            // 16 INT8 codes
        uint4 kn[2], vn[2];      // 16 FP16 values
        float ks, vs;
    };
    Raw raw[NB];
    auto fetch = [&](int t, Raw& r) {
        const int kp = t * PF_T + sj;
        const int ci = min(kp, max(clen - 1, 0)), ni = min(max(kp - clen, 0), max(nlen - 1, 0));
        r.kc = *reinterpret_cast<const uint4*>(kcb + (size_t)ci * cstride);
        r.vc = *reinterpret_cast<const uint4*>(vcb + (size_t)ci * cstride);
        const uint4* k4 = reinterpret_cast<const uint4*>(knb + (size_t)ni * nstride);
        const uint4* v4 = reinterpret_cast<const uint4*>(vnb + (size_t)ni * nstride);
        r.kn[0] = k4[0];
        r.kn[1] = k4[1];
        r.vn[0] = v4[0];
        r.vn[1] = v4[1];
        r.ks = ksb[(size_t)ci * sstride];
        r.vs = vsb[(size_t)ci * sstride];
    };
    auto stage = [&](int t, int buf, const Raw& r) {
        if (!stager) return;
        const int kp = t * PF_T + sj;
        const bool live = kp < (int)kv_end, cached = kp < clen;
        h16x8 k0, k1;
        _Float16 vh[16];
        if (cached) {
            // key codes to exact fp16: the biased byte b ^ 0x80 = b + 128
            // under the exponent byte 0x64 reads as 1024 + b + 128, and 1152
            // comes off in packed fp16 (integers below 2048 are exact)
            const uint32_t kx[4] = {r.kc.x ^ 0x80808080u, r.kc.y ^ 0x80808080u, r.kc.z ^ 0x80808080u,
                                    r.kc.w ^ 0x80808080u};
            typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
            const h16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const h16x2 lo = __builtin_bit_cast(h16x2, __builtin_amdgcn_perm(0x64646464u, kx[j], 0x04010400u)) - bias;
                const h16x2 hi = __builtin_bit_cast(h16x2, __builtin_amdgcn_perm(0x64646464u, kx[j], 0x04030402u)) - bias;
                h16x8& kd = j < 2 ? k0 : k1;
                const int e0 = 4 * (j & 1);
                kd[e0] = lo[0];
                kd[e0 + 1] = lo[1];
                kd[e0 + 2] = hi[0];
                kd[e0 + 3] = hi[1];
            }
            // values fp16(fp32(code * scale)): with u = code + 128 (an unsigned
            // byte), fma(u, scale, -128 scale) is that fp32 product exactly
            // (one rounding of u scale - 128 scale = code scale; -128 scale is exact)
            const float ms = -128.0f * r.vs;
            const uint32_t vx[4] = {r.vc.x ^ 0x80808080u, r.vc.y ^ 0x80808080u, r.vc.z ^ 0x80808080u,
                                    r.vc.w ^ 0x80808080u};
#pragma unroll
            for (int e = 0; e < 16; e++)
                vh[e] = (_Float16)fp32_barrier(__builtin_fmaf((float)((vx[e >> 2] >> (8 * (e & 3))) & 0xFFu), r.vs, ms));
        } else {
            k0 = __builtin_bit_cast(h16x8, r.kn[0]);
            k1 = __builtin_bit_cast(h16x8, r.kn[1]);
            const h16x8 v0 = __builtin_bit_cast(h16x8, r.vn[0]), v1 = __builtin_bit_cast(h16x8, r.vn[1]);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                vh[e] = v0[e];
                vh[8 + e] = v1[e];
            }
        }
        if (!live) {
            // keys past the block's causal end: zero values (their weights are 0)
#pragma unroll
            for (int e = 0; e < 16; e++) vh[e] = (_Float16)0.0f;
        }
        *reinterpret_cast<h16x8*>(&ksh[buf][sj][16 * sp]) = k0;
        *reinterpret_cast<h16x8*>(&ksh[buf][sj][16 * sp + 8]) = k1;
#pragma unroll
        for (int e = 0; e < 16; e++) vt[buf][16 * sp + e][sj] = vh[e];
        if (sp == 0) ksc[buf][sj] = (cached ? r.ks : 1.0f) * a.scale;
    };

    constexpr float LOG2E = 1.4426950408889634f;
    const float NEG_INF = -__builtin_inff();
    float m_run[VB], l_run[VB];
    f32x4 acc[VB][ND];   // O^T: lane l holds dims 16 db + 4 lg + i of vector lr of each block
#pragma unroll
    for (int vb = 0; vb < VB; vb++) {
        m_run[vb] = NEG_INF;
        l_run[vb] = 0.0f;
#pragma unroll
        for (int db = 0; db < ND; db++) acc[vb][db] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }

#pragma unroll
    for (int u = 0; u < NB; u++) fetch(t_begin + u, raw[u]);   // clamped rows: in bounds past the split too
    stage(t_begin, 0, raw[0]);
    __syncthreads();
    for (int l0 = 0; l0 < nt; l0 += NB)
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const int tl = l0 + u;
        if (tl >= nt) break;
        const int t = t_begin + tl;
        const int buf = tl & 1;
        // scores S^T for keys 16h + 4lg + i of the tile, vector lr of each block
        f32x4 st[VB][2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int vb = 0; vb < VB; vb++) st[vb][h] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const h16x8 kv = *reinterpret_cast<const h16x8*>(&ksh[buf][16 * h + lr][32 * c + 8 * lg]);
#pragma unroll
                for (int vb = 0; vb < VB; vb++)
                    st[vb][h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qv[vb][c], st[vb][h], 0, 0, 0);
            }
        }
        // a tile below every row's causal end and the key range needs no
        // mask (wave-uniform test); the others mask key by key
        const size_t tile_last = (size_t)t * PF_T + PF_T - 1;
        const bool interior = wave_all_rows && tile_last < kv_end && tile_last <= wave_min_pos;
        const f32x4 ksv0 = *reinterpret_cast<const f32x4*>(&ksc[buf][4 * lg]);
        const f32x4 ksv1 = *reinterpret_cast<const f32x4*>(&ksc[buf][16 + 4 * lg]);
        float corr[VB];
        h16x8 pa[VB];   // P^T operands: keys {4 lg + j, 16 + 4 lg + j} of vector lr
#pragma unroll
        for (int vb = 0; vb < VB; vb++) {
            float s[8];
            float mx = NEG_INF;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const f32x4 ksv = h ? ksv1 : ksv0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (interior) {
                        s[4 * h + i] = st[vb][h][i] * ksv[i];
                    } else {
                        const size_t kp = (size_t)t * PF_T + 16 * h + 4 * lg + i;
                        const bool ok = vok[vb] && kp < kv_end && kp <= vpos[vb];
                        s[4 * h + i] = ok ? st[vb][h][i] * ksv[i] : NEG_INF;
                    }
                    mx = __builtin_fmaxf(mx, s[4 * h + i]);
                }
            }
            mx = xrow_max(mx);
            const float m_new = __builtin_fmaxf(m_run[vb], mx);
            const bool live = m_new > NEG_INF;
            corr[vb] = live ? fast_exp2((m_run[vb] - m_new) * LOG2E) : 1.0f;
            float psum = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float pv = (live && s[j] > NEG_INF) ? fast_exp2((s[j] - m_new) * LOG2E) : 0.0f;
                psum += pv;
                pa[vb][j] = (_Float16)pv;
            }
            l_run[vb] = l_run[vb] * corr[vb] + xrow_sum(psum);
            m_run[vb] = m_new;
        }
        // O^T += V^T P^T: A = V^T (dims 16 db + lr, the same 8 keys)
#pragma unroll
        for (int db = 0; db < ND; db++) {
            const h16x4 v0 = *reinterpret_cast<const h16x4*>(&vt[buf][16 * db + lr][4 * lg]);
            const h16x4 v1 = *reinterpret_cast<const h16x4*>(&vt[buf][16 * db + lr][16 + 4 * lg]);
            const h16x8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
            for (int vb = 0; vb < VB; vb++)
                acc[vb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pa[vb], acc[vb][db] * corr[vb], 0, 0, 0);
        }
        // the next tile into the other LDS buffer (its last readers finished
        // before the previous barrier), then tile t + NB into this slot
        if (tl + 1 < nt) stage(t + 1, buf ^ 1, raw[(u + 1) % NB]);
        if (tl + NB < nt) fetch(t + NB, raw[u]);
        __syncthreads();
    }

    // ---- output: vector lr of each block, dims 16 db + 4 lg + i
#pragma unroll
    for (int vb = 0; vb < VB; vb++) {
        if (a.nsplit > 1) {
            // this split's partial (acc, running max, sum) of the vector
            const int nqb = (int)gridDim.x / a.nsplit;
            float* pp = a.part +
                        ((((size_t)bg * nqb + qb) * a.nsplit + sp_) * NV + (wid * VB + vb) * 16 + lr) * (D + 4);
#pragma unroll
            for (int db = 0; db < ND; db++) *reinterpret_cast<f32x4*>(pp + 16 * db + 4 * lg) = acc[vb][db];
            if (lg == 0) {
                pp[D] = m_run[vb];
                pp[D + 1] = l_run[vb];
            }
            continue;
        }
        if (!vok[vb]) continue;
        uint16_t* op = a.o + (((size_t)b * a.S + vrow[vb]) * a.Hq + (size_t)g * GQ + vm[vb] % GQ) * D;
        const float inv = l_run[vb] > 0.0f ? 1.0f / l_run[vb] : 0.0f;
#pragma unroll
        for (int db = 0; db < ND; db++) {
            const uint32_t lo = (uint32_t)f2h(acc[vb][db][0] * inv) | ((uint32_t)f2h(acc[vb][db][1] * inv) << 16);
            const uint32_t hi = (uint32_t)f2h(acc[vb][db][2] * inv) | ((uint32_t)f2h(acc[vb][db][3] * inv) << 16);
            *reinterpret_cast<uint2*>(op + 16 * db + 4 * lg) = make_uint2(lo, hi);
        }
    }
}

// Combine of the key splits: grid (query blocks x NV / 16, B * Hkv), 256
// threads; a workgroup takes 16 query vectors, 16 threads per vector with
// D/16 dims each.  M = max_s M_s, L = sum_s e^(M_s - M) l_s,
// o = sum_s e^(M_s - M) acc_s / L.  Loads are branch-free (clamped splits,
// weight 0 past the block's split count) and issued per batch of splits.
constexpr int PF_MAX_SPLITS = 16;

template <int D, int GQ, int NV>
__global__ void __launch_bounds__(256) attn_prefill_combine_kernel(PrefillArgs a) {
    constexpr int VPW = 16, DS = D / 16, SB = 4;
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x, vl = tid / 16, dq = (tid % 16) * DS;
    const int qb = blockIdx.x / (NV / VPW), v = (blockIdx.x % (NV / VPW)) * VPW + vl;
    const int bg = blockIdx.y, b = bg / a.Hkv, g = bg % a.Hkv;
    const int nqb = (int)gridDim.x / (NV / VPW);
    const int gm0 = qb * NV;
    const int ns = min(a.nsplit, (pf_block_tiles(a, gm0, NV, GQ) + a.tps - 1) / a.tps);
    const int vm = gm0 + v, row = vm / GQ;
    if (row >= a.S) return;
    uint16_t* op = a.o + (((size_t)b * a.S + row) * a.Hq + (size_t)g * GQ + vm % GQ) * D + dq;
    if (ns <= 0) {   // no key tile reaches this block: zero rows, as with L = 0
#pragma unroll
        for (int e = 0; e < DS; e += 2) *reinterpret_cast<uint32_t*>(op + e) = 0u;
        return;
    }
    const float* pb = a.part + (((size_t)bg * nqb + qb) * a.nsplit * NV + v) * (D + 4);
    const size_t sstep = (size_t)NV * (D + 4);
    float ms[PF_MAX_SPLITS], ls[PF_MAX_SPLITS];
#pragma unroll
    for (int s = 0; s < PF_MAX_SPLITS; s++) {
        const float* ps = pb + (size_t)min(s, ns - 1) * sstep;
        ms[s] = ps[D];
        ls[s] = ps[D + 1];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < PF_MAX_SPLITS; s++)
        if (s < ns) M = __builtin_fmaxf(M, ms[s]);
    float L = 0.0f;
#pragma unroll
    for (int s = 0; s < PF_MAX_SPLITS; s++) {
        ms[s] = (s < ns && ms[s] > -__builtin_inff()) ? fast_exp2((ms[s] - M) * LOG2E) : 0.0f;   // weights
        L = __builtin_fmaf(ms[s], ls[s], L);
    }
    float out[DS];
#pragma unroll
    for (int e = 0; e < DS; e++) out[e] = 0.0f;
#pragma unroll
    for (int s0 = 0; s0 < PF_MAX_SPLITS; s0 += SB) {
        if (s0 >= ns) break;
        f32x4 x[SB][DS / 4];
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const float* ps = pb + (size_t)min(s0 + u, ns - 1) * sstep + dq;
#pragma unroll
            for (int e = 0; e < DS / 4; e++) x[u][e] = *reinterpret_cast<const f32x4*>(ps + 4 * e);
        }
#pragma unroll
        for (int u = 0; u < SB; u++) {
            const float w = ms[s0 + u];
#pragma unroll
            for (int e = 0; e < DS / 4; e++) {
                out[4 * e] = __builtin_fmaf(w, x[u][e][0], out[4 * e]);
                out[4 * e + 1] = __builtin_fmaf(w, x[u][e][1], out[4 * e + 1]);
                out[4 * e + 2] = __builtin_fmaf(w, x[u][e][2], out[4 * e + 2]);
                out[4 * e + 3] = __builtin_fmaf(w, x[u][e][3], out[4 * e + 3]);
            }
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int e = 0; e < DS; e += 2)
        *reinterpret_cast<uint32_t*>(op + e) = (uint32_t)f2h(out[e] * inv) | ((uint32_t)f2h(out[e + 1] * inv) << 16);
}

// ------------------------------------------------ per-(device, stream) workspace
// split partials, and the per-KV-head completion counters (zeroed when made;
// the combining workgroup leaves its counter at zero)
struct FastWs {
    float* part = nullptr;
    uint32_t* cnt = nullptr;
};

static int fast_ws(void* stream, size_t part_floats, size_t ncnt, FastWs* out) {
    void* p = nullptr;
    int rc = stream_scratch(SCR_FAST_PART, stream, part_floats * sizeof(float), false, &p);
    if (rc) return rc;
    out->part = static_cast<float*>(p);
    out->cnt = nullptr;
    if (ncnt) {
        rc = stream_scratch(SCR_FAST_CNT, stream, ncnt * sizeof(uint32_t), true, &p);
        if (rc) return rc;
        out->cnt = static_cast<uint32_t*>(p);
    }
    return CACTUS_HIP_OK;
}

size_t fast_attention_splits(size_t keys, bool hybrid) {
    const size_t kpb = hybrid ? fa_kpb<true>() : fa_kpb<false>();
    return keys == 0 ? 1 : (keys + kpb - 1) / kpb;
}

template <bool HYBRID, bool PREP>
static int launch_fast(const FastArgs& a, int d, int gq, hipStream_t st) {
    const dim3 grid((unsigned)(a.nsplit + (PREP ? 1 : 0)), (unsigned)(a.B * a.Hkv));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(FA_THREADS), 0, st, a);
        return check_launch("attention (split-K)");
    };
#define FA_CASE(D_, G_) if (d == D_ && gq == G_) return go(attn_splitk_kernel<HYBRID, PREP, D_, G_>);
    FA_CASE(128, 2) FA_CASE(128, 1) FA_CASE(128, 4) FA_CASE(64, 2) FA_CASE(64, 1) FA_CASE(64, 4)
#undef FA_CASE
    return fail(CACTUS_HIP_EUNSUPPORTED, "attention (split-K): head_dim 64/128 with 1, 2 or 4 query heads per KV head");
}

bool fast_attention_supported(size_t seq_len, size_t d, size_t gq, const void* mask) {
    return seq_len == 1 && !mask && (d == 64 || d == 128) && (gq == 1 || gq == 2 || gq == 4);
}

// the combine holds every split's (M, sum) in LDS: at most FA_MAX_SPLITS splits
constexpr size_t FA_MAX_KEYS_F16 = (size_t)FA_MAX_SPLITS * fa_kpb<false>();    // 131072
constexpr size_t FA_MAX_KEYS_HYBRID = (size_t)FA_MAX_SPLITS * fa_kpb<true>();  // 131072

int attention_fast_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, size_t B,
                       size_t Skv, size_t Hq, size_t Hkv, size_t d, float scale, size_t pos_off, size_t window,
                       void* stream) {
    FastArgs a{};
    a.q = q; a.k = k; a.v = v; a.o = o;
    a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.nqg = 1;
    a.Skv = Skv; a.cache_len = 0; a.new_len = 0; a.pos_off = pos_off; a.window = window; a.scale = scale;
    size_t start = 0, end = Skv;
    if (window > 0 && window < Skv && pos_off > window) start = pos_off - window;
    if (pos_off + 1 < end) end = pos_off + 1;
    a.nsplit = (int)fast_attention_splits(end > start ? end - start : 0, false);
    FastWs w;
    int rc = fast_ws(stream, B * Hkv * (size_t)a.nsplit * (Hq / Hkv) * (d + 4), B * Hkv, &w);
    if (rc) return rc;
    a.part = w.part; a.cnt = w.cnt;
    return launch_fast<false, false>(a, (int)d, (int)(Hq / Hkv), as_stream(stream));
}

int attention_fast_hybrid(const uint16_t* q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
                          const uint16_t* k_new, const uint16_t* v_new, uint16_t* o, size_t B, size_t cache_len,
                          size_t new_len, size_t Hq, size_t Hkv, size_t d, float scale, size_t pos_off, size_t qgs,
                          void* stream) {
    FastArgs a{};
    a.q = q; a.k = k_new; a.v = v_new; a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs; a.o = o;
    a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.nqg = (int)((d + qgs - 1) / qgs);
    a.Skv = cache_len + new_len; a.cache_len = cache_len; a.new_len = new_len; a.pos_off = pos_off;
    a.scale = scale;
    size_t end = a.Skv;
    if (pos_off + 1 < end) end = pos_off + 1;
    a.nsplit = (int)fast_attention_splits(end, true);
    FastWs w;
    int rc = fast_ws(stream, B * Hkv * (size_t)a.nsplit * (Hq / Hkv) * (d + 4), B * Hkv, &w);
    if (rc) return rc;
    a.part = w.part; a.cnt = w.cnt;
    return launch_fast<true, false>(a, (int)d, (int)(Hq / Hkv), as_stream(stream));
}

bool fast_prefill_supported(size_t d, size_t gq) {
    return (d == 64 || d == 128) && (gq == 1 || gq == 2 || gq == 4);
}

int attention_prefill_fast(const uint16_t* q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
                           const uint16_t* k_new, const uint16_t* v_new, uint16_t* o, size_t B, size_t S,
                           size_t cache_len, size_t new_len, size_t Hq, size_t Hkv, size_t d, float scale,
                           size_t pos_off, size_t qgs, void* stream) {
    constexpr int W = 4, NB = 2, VB = 2, NV = 16 * W * VB;
    PrefillArgs a{};
    a.q = q; a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs; a.kn = k_new; a.vn = v_new; a.o = o;
    a.B = (int)B; a.S = (int)S; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.nqg = (int)((d + qgs - 1) / qgs);
    a.cache_len = cache_len; a.new_len = new_len; a.pos_off = pos_off; a.scale = scale;
    const int gq = (int)(Hq / Hkv);
    const size_t nqb = (S * gq + NV - 1) / NV;
    // key splits: enough workgroups to cover the CUs, at least 4 tiles each
    size_t kv_last = pos_off + S;
    if (kv_last > cache_len + new_len) kv_last = cache_len + new_len;
    const size_t tiles = (kv_last + PF_T - 1) / PF_T;
    size_t nsplit = (512 + nqb * B * Hkv - 1) / (nqb * B * Hkv);
    const size_t max_split = (tiles + 3) / 4;
    if (nsplit > max_split) nsplit = max_split;
    if (nsplit > PF_MAX_SPLITS) nsplit = PF_MAX_SPLITS;
    if (nsplit < 1) nsplit = 1;
    a.tps = (int)((tiles + nsplit - 1) / nsplit);
    a.nsplit = (int)((tiles + a.tps - 1) / a.tps);
    if (a.nsplit < 1) a.nsplit = 1;
    if (a.nsplit > 1) {
        FastWs w;
        const int rc = fast_ws(stream, B * Hkv * nqb * (size_t)a.nsplit * NV * (d + 4), 0, &w);
        if (rc) return rc;
        a.part = w.part;
    }
    const dim3 grid((unsigned)(nqb * a.nsplit), (unsigned)(B * Hkv));
    const dim3 cgrid((unsigned)(nqb * (NV / 16)), (unsigned)(B * Hkv));
    auto go = [&](auto kern, auto comb) {
        hipLaunchKernelGGL(kern, grid, dim3(64 * W), 0, as_stream(stream), a);
        int rc = check_launch("attention (prefill, MFMA)");
        if (rc || a.nsplit == 1) return rc;
        hipLaunchKernelGGL(comb, cgrid, dim3(256), 0, as_stream(stream), a);
        return check_launch("attention (prefill, split combine)");
    };
#define PF_CASE(D_, G_) \
    if (d == D_ && gq == G_) \
        return go(attn_prefill_mfma_kernel<D_, G_, W, NB, VB>, attn_prefill_combine_kernel<D_, G_, NV>);
    PF_CASE(128, 2) PF_CASE(128, 1) PF_CASE(128, 4) PF_CASE(64, 2) PF_CASE(64, 1) PF_CASE(64, 4)
#undef PF_CASE
    return fail(CACTUS_HIP_EUNSUPPORTED, "attention (prefill, MFMA): head_dim 64/128 with 1, 2 or 4 query heads per KV head");
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_attention_f16_fast(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                  size_t batch, size_t seq_len, size_t kv_seq_len, size_t num_q_heads,
                                  size_t num_kv_heads, size_t head_dim, float scale, const uint16_t* mask,
                                  size_t position_offset, size_t window_size, int is_causal, void* stream) {
    if (batch == 0 || seq_len == 0 || num_q_heads == 0 || head_dim == 0) return CACTUS_HIP_OK;
    const bool fast = num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && is_causal &&
                      fast_attention_supported(seq_len, head_dim, num_q_heads / num_kv_heads, mask) &&
                      batch * num_kv_heads < 65536 && kv_seq_len <= FA_MAX_KEYS_F16 && ((uintptr_t)k & 15) == 0;
    if (!fast)
        return cactus_hip_attention_f16(q, k, v, o, batch, seq_len, kv_seq_len, num_q_heads, num_kv_heads,
                                        head_dim, scale, mask, position_offset, window_size, is_causal, stream);
    CH_REQUIRE(q && o && (kv_seq_len == 0 || (k && v)), "attention_f16_fast: null pointer");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    return attention_fast_f16(q, k, v, o, batch, kv_seq_len, num_q_heads, num_kv_heads, head_dim, scale,
                              position_offset, window_size, stream);
}

int cactus_hip_attention_hybrid_int8_fp16_fast(const uint16_t* q, const int8_t* k_cached, const int8_t* v_cached,
                                               const float* k_scales, const float* v_scales, const uint16_t* k_new,
                                               const uint16_t* v_new, uint16_t* o, size_t batch, size_t seq_len,
                                               size_t cache_len, size_t new_len, size_t num_q_heads,
                                               size_t num_kv_heads, size_t head_dim, float scale,
                                               size_t position_offset, int is_causal, size_t quant_group_size,
                                               void* stream) {
    if (batch == 0 || seq_len == 0 || num_q_heads == 0 || head_dim == 0) return CACTUS_HIP_OK;
    const bool aligned16 = ((uintptr_t)k_cached & 15) == 0 && ((uintptr_t)v_cached & 15) == 0;
    // prefill rows: flash attention on FP16 MFMA
    const bool prefill = seq_len > 1 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && is_causal &&
                         fast_prefill_supported(head_dim, num_q_heads / num_kv_heads) &&
                         quant_group_size >= head_dim && batch * num_kv_heads < 65536 && aligned16 &&
                         ((uintptr_t)q & 15) == 0 && ((uintptr_t)k_new & 15) == 0 && ((uintptr_t)v_new & 15) == 0 &&
                         seq_len * (num_q_heads / num_kv_heads) < (1ull << 31);
    if (prefill) {
        CH_REQUIRE(q && o, "attention_hybrid_fast: null pointer");
        CH_REQUIRE(cache_len == 0 || (k_cached && v_cached && k_scales && v_scales),
                   "attention_hybrid_fast: null cache pointer");
        CH_REQUIRE(new_len == 0 || (k_new && v_new), "attention_hybrid_fast: null new K/V pointer");
        if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
        return attention_prefill_fast(q, k_cached, v_cached, k_scales, v_scales, k_new, v_new, o, batch, seq_len,
                                      cache_len, new_len, num_q_heads, num_kv_heads, head_dim, scale,
                                      position_offset, quant_group_size, stream);
    }
    const bool fast = num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && is_causal &&
                      fast_attention_supported(seq_len, head_dim, num_q_heads / num_kv_heads, nullptr) &&
                      quant_group_size >= head_dim && batch * num_kv_heads < 65536 &&
                      cache_len + new_len <= FA_MAX_KEYS_HYBRID && aligned16;
    if (!fast)
        return cactus_hip_attention_hybrid_int8_fp16(q, k_cached, v_cached, k_scales, v_scales, k_new, v_new, o,
                                                     batch, seq_len, cache_len, new_len, num_q_heads,
                                                     num_kv_heads, head_dim, scale, position_offset, is_causal,
                                                     quant_group_size, stream);
    CH_REQUIRE(q && o, "attention_hybrid_fast: null pointer");
    CH_REQUIRE(cache_len == 0 || (k_cached && v_cached && k_scales && v_scales),
               "attention_hybrid_fast: null cache pointer");
    CH_REQUIRE(new_len == 0 || (k_new && v_new), "attention_hybrid_fast: null new K/V pointer");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    return attention_fast_hybrid(q, k_cached, v_cached, k_scales, v_scales, k_new, v_new, o, batch, cache_len,
                                 new_len, num_q_heads, num_kv_heads, head_dim, scale, position_offset,
                                 quant_group_size, stream);
}

size_t cactus_hip_decode_attention_fast_workspace(size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                                  size_t max_cache) {
    if (num_kv_heads == 0) return 0;
    const size_t nsplit = fast_attention_splits(max_cache + 1, true);
    return 256 + num_kv_heads * nsplit * (num_q_heads / num_kv_heads) * (head_dim + 4) * sizeof(float);
}

int cactus_hip_decode_prep_attention_fast(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                          const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                          size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float theta,
                                          const uint32_t* state, int8_t* k_cache, int8_t* v_cache,
                                          float* k_scales, float* v_scales, size_t max_cache, float* v_shadow,
                                          float scale, uint16_t* o, void* workspace, size_t workspace_bytes,
                                          void* stream) {
    CH_REQUIRE(q_raw && k_raw && v_raw && q_norm && k_norm && state && k_cache && v_cache && k_scales &&
               v_scales && o && workspace, "decode_prep_attention_fast: null pointer");
    CH_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && num_kv_heads <= 64,
               "decode_prep_attention_fast: bad head counts");
    CH_REQUIRE(fast_attention_supported(1, head_dim, num_q_heads / num_kv_heads, nullptr),
               "decode_prep_attention_fast: head_dim 64 or 128 with 1, 2 or 4 query heads per KV head");
    CH_REQUIRE(max_cache + 1 <= FA_MAX_KEYS_HYBRID, "decode_prep_attention_fast: cache longer than 131071 tokens");
    CH_REQUIRE(((uintptr_t)k_cache & 15) == 0 && ((uintptr_t)v_cache & 15) == 0 && ((uintptr_t)workspace & 255) == 0,
               "decode_prep_attention_fast: misaligned cache or workspace");
    CH_REQUIRE(workspace_bytes >= cactus_hip_decode_attention_fast_workspace(num_q_heads, num_kv_heads, head_dim,
                                                                             max_cache),
               "decode_prep_attention_fast: workspace too small");
    RopeTable t;
    int rc = rope_table(max_cache + 1, head_dim, theta, &t);
    if (rc) return rc;
    FastArgs a{};
    a.o = o;
    a.B = 1; a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads; a.nqg = 1;
    a.kc = k_cache; a.vc = v_cache; a.ks = k_scales; a.vs = v_scales;
    a.cache_len = max_cache; a.new_len = 1; a.Skv = max_cache + 1; a.pos_off = max_cache;
    a.scale = scale; a.dyn = state;
    a.q_raw = q_raw; a.k_raw = k_raw; a.v_raw = v_raw; a.q_norm = q_norm; a.k_norm = k_norm;
    a.cos_t = t.cos_d; a.sin_t = t.sin_d; a.eps = eps; a.table_pos = (uint32_t)t.npos;
    a.kc_w = k_cache; a.vc_w = v_cache; a.ks_w = k_scales; a.vs_w = v_scales; a.vsh = v_shadow;
    a.sh_ntile = (max_cache + 63) / 64; a.max_cache = max_cache;
    a.nsplit = (int)fast_attention_splits(max_cache + 1, true);
    a.cnt = static_cast<uint32_t*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
    return launch_fast<true, true>(a, (int)head_dim, (int)(num_q_heads / num_kv_heads), as_stream(stream));
}

}  // extern "C"
