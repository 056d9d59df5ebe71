// attention.hip -- KV-cache attention (a5 FP16 KV, a6 INT8 cache + FP16 new)
// with the reference's exact order of operations (kernel_attention.cpp:10-482).
//
// The reference walks each (query, head) serially through 32-key blocks.  Only
// two of its steps carry a dependence from one key to the next: the running
// sum and the weighted-value accumulators.  Everything else is independent
// per key or per block, so it runs here in two kernels:
//
//  A. scores  -- one lane per key, a wave per 64 keys (two reference blocks)
//     and per query/KV-head group.  Each lane computes the score exactly as
//     the reference does: fp32 FMA chains on dims 8c+j, combined as
//     ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)), times `scale`, masked to -inf.
//     The block max, the weights (second-order 2^x polynomial on the first
//     floor(n/4)*4 keys of a FP16 block and expf elsewhere; expf everywhere
//     for the INT8 hybrid) and the block sum in the reference's order are
//     written to scratch.
//  B. values  -- one lane per output dim.  The rescale factors
//     expf(previous_max - block_max) are computed in parallel, the running
//     sum is chained once per (query, head), and every lane then applies
//     acc = acc * corr at each block start and acc = fma(v, w, acc) key by
//     key, in increasing position, exactly as the reference.  The output is
//     fp16(acc * (1/sum)) on the 8-aligned prefix of head_dim.
#include "hip_common.h"
#include "attention_args.h"
#include "decode_device.h"

#include <map>
#include <utility>
#include <mutex>

namespace cactus_hip {

// ----------------------------------------------------------------- kernel A
// grid.x: 64-key chunks (4 per workgroup), grid.y: (b, qp, kv head).  A lane
// owns one key: its whole key row is loaded up front (DMAX >= head_dim), so a
// score costs one memory round trip.
template <bool HYBRID, int DMAX>
__global__ void __launch_bounds__(256) attn_scores_kernel(AttnArgs a_in) {
    const AttnArgs a = resolve(a_in);
    __shared__ float qsh[ATT_MAX_GQ][ATT_MAX_D];
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t row = blockIdx.y;                    // (b, qp, kvh)
    const int kvh = (int)(row % a.Hkv);
    const size_t qp = (row / a.Hkv) % a.S;
    const size_t b = row / ((size_t)a.Hkv * a.S);
    const int d = a.d, da = (d / 8) * 8, gq = a.gq;
    const int h0 = kvh * gq;
    for (int i = threadIdx.x; i < gq * d; i += 256) {
        const int hh = i / d, dim = i % d;
        qsh[hh][dim] = h2f(a.q[((b * a.S + qp) * a.Hq + h0 + hh) * (size_t)d + dim]);
    }
    __syncthreads();

    size_t kv_start, kv_end, blk_limit;
    kv_range<HYBRID>(a, qp, kv_start, kv_end, blk_limit);
    const size_t chunk = (size_t)blockIdx.x * 4 + wid;
    const size_t bs0 = kv_start + chunk * 64 + (lane & 32);   // this lane's block start
    if (kv_start + chunk * 64 >= kv_end) return;              // wave-uniform
    const int jl = lane & 31;
    const bool block_live = bs0 < kv_end;
    const size_t be = block_live ? ((bs0 + ATT_BLOCK < blk_limit) ? bs0 + ATT_BLOCK : blk_limit) : bs0;
    const int bsz = (int)(be - bs0);
    const size_t kp = bs0 + jl;
    const size_t aq = a.pos_off + qp;
    const bool is_decode = (!HYBRID) && (qp == (size_t)a.S - 1) && a.S > 1;
    const float NEG_INF = -__builtin_inff();
    // FP16: a block wholly in the future of a non-last query is skipped by the
    // reference (kernel_attention.cpp:100-105): it contributes nothing
    const bool block_skipped = !HYBRID && !is_decode && a.causal && bs0 > aq;
    const bool in_block = block_live && jl < bsz && !block_skipped;
    bool computed = in_block;
    if (computed && a.causal && kp > aq && (HYBRID || !is_decode)) computed = false;

    float score[ATT_MAX_GQ];
#pragma unroll
    for (int hh = 0; hh < ATT_MAX_GQ; hh++) score[hh] = NEG_INF;
    if (computed) {
        constexpr int NC = DMAX / 8;   // 8-dim chunks of a key row
        const int nca = da / 8;
        // per chunk: 8 key values as float (INT8 code * scale, or fp16)
        auto dot_heads = [&](auto chunk_vals) {
#pragma unroll
            for (int hh = 0; hh < ATT_MAX_GQ; hh++) {
                if (hh >= gq) break;
                float ch[8];
#pragma unroll
                for (int c = 0; c < 8; c++) ch[c] = 0.0f;
#pragma unroll
                for (int cc = 0; cc < NC; cc++) {
                    if (cc >= nca) break;
                    float kk[8];
                    chunk_vals(cc, kk);
#pragma unroll
                    for (int c = 0; c < 8; c++) ch[c] = __builtin_fmaf(qsh[hh][cc * 8 + c], kk[c], ch[c]);
                }
                const float t0 = ch[0] + ch[4], t1 = ch[1] + ch[5];
                const float t2 = ch[2] + ch[6], t3 = ch[3] + ch[7];
                score[hh] = (t0 + t1) + (t2 + t3);
            }
        };
        if (HYBRID && kp < a.cache_len) {
            const int8_t* kr = a.kc + ((b * a.cache_len + kp) * a.Hkv + kvh) * (size_t)d;
            // scales carry no batch offset (kernel_attention.cpp:353)
            const float* sr = a.ks + (kp * a.Hkv + kvh) * (size_t)a.nqg;
            uint2 kw[NC];
            float ksc[NC];
#pragma unroll
            for (int cc = 0; cc < NC; cc++) {
                const int cb = cc < nca ? cc * 8 : 0;   // chunks past the row reload chunk 0
                kw[cc] = *reinterpret_cast<const uint2*>(kr + cb);
                ksc[cc] = sr[cb / a.qgs];
            }
            dot_heads([&](int cc, float* kk) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    kk[c] = (float)(int8_t)((kw[cc].x >> (8 * c)) & 0xFF) * ksc[cc];
                    kk[4 + c] = (float)(int8_t)((kw[cc].y >> (8 * c)) & 0xFF) * ksc[cc];
                }
            });
        } else if (nca > 0) {
            const size_t kpos = HYBRID ? kp - a.cache_len : kp;
            const size_t klen = HYBRID ? a.new_len : a.Skv;
            const uint16_t* kr = a.k + ((b * klen + kpos) * a.Hkv + kvh) * (size_t)d;
            uint32_t kw[NC][4];
#pragma unroll
            for (int cc = 0; cc < NC; cc++) {
                const int cb = cc < nca ? cc * 8 : 0;
                if ((d & 7) == 0) {
                    const uint4 w = *reinterpret_cast<const uint4*>(kr + cb);
                    kw[cc][0] = w.x; kw[cc][1] = w.y; kw[cc][2] = w.z; kw[cc][3] = w.w;
                } else {
                    const uint2 w0 = *reinterpret_cast<const uint2*>(kr + cb);
                    const uint2 w1 = *reinterpret_cast<const uint2*>(kr + cb + 4);
                    kw[cc][0] = w0.x; kw[cc][1] = w0.y; kw[cc][2] = w1.x; kw[cc][3] = w1.y;
                }
            }
            dot_heads([&](int cc, float* kk) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    kk[2 * c] = h2f((uint16_t)(kw[cc][c] & 0xFFFF));
                    kk[2 * c + 1] = h2f((uint16_t)(kw[cc][c] >> 16));
                }
            });
        } else {
#pragma unroll
            for (int hh = 0; hh < ATT_MAX_GQ; hh++) score[hh] = 0.0f;
        }
#pragma unroll
        for (int hh = 0; hh < ATT_MAX_GQ; hh++) {
            if (hh >= gq) break;
            float sc = score[hh];
            if (!HYBRID) {
                const uint16_t* kr = a.k + ((b * a.Skv + kp) * a.Hkv + kvh) * (size_t)d;
                for (int i = da; i < d; i++) sc = __builtin_fmaf(qsh[hh][i], h2f(kr[i]), sc);
            }
            sc = sc * a.scale;
            if (!HYBRID) {
                if (a.causal && kp > aq) sc = NEG_INF;
                else if (a.window > 0 && kp < aq && (aq - kp) > a.window) sc = NEG_INF;
                else if (a.mask && h2f(a.mask[(b * a.S + qp) * a.Skv + kp]) == 0.0f) sc = NEG_INF;
            }
            score[hh] = sc;
        }
    }

    // per head of the group: block max, weights, block sum, stores
    const int blk = (int)((bs0 - kv_start) / ATT_BLOCK);
    const int vs4 = HYBRID ? 0 : (bsz / 4) * 4;
    const int half = lane & 32;
    for (int hh = 0; hh < gq; hh++) {
        float s = score[hh];
        // max over the 32 lanes of this block (half-wave reduction)
        const float m = half_wave_max(s);
        float w = 0.0f;
        if (in_block) {
            if (jl < vs4) w = poly_exp_weight(s, m);
            else w = (s != NEG_INF) ? cactus_expf(s - m) : 0.0f;
        }
        // block sum in the reference's order, for both half-wave blocks
        float sumA = 0.0f, sumB = 0.0f;
        const int bszA = __builtin_amdgcn_readlane(bsz, 0);
        const int bszB = __builtin_amdgcn_readlane(bsz, 32);
        {
            // the two half-wave blocks' chains interleave; every lane index is
            // a constant (v_readlane), every bound a uniform branch
            const int v4A = HYBRID ? 0 : (bszA / 4) * 4;
            const int v4B = HYBRID ? 0 : (bszB / 4) * 4;
#pragma unroll
            for (int j = 0; j < ATT_BLOCK; j += 4) {
                float xa[4], xb[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    xa[e] = lane_f(w, j + e);
                    xb[e] = lane_f(w, 32 + j + e);
                }
                if (j < v4A) {
                    sumA = sumA + ((xa[0] + xa[1]) + (xa[2] + xa[3]));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (j + e < bszA) sumA = sumA + xa[e];
                }
                if (j < v4B) {
                    sumB = sumB + ((xb[0] + xb[1]) + (xb[2] + xb[3]));
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (j + e < bszB) sumB = sumB + xb[e];
                }
            }
        }
        const size_t r = (b * a.S + qp) * a.Hq + h0 + hh;
        // every key of a live block gets its weight (0 when not computed);
        // a block holding a zero weight is flagged by the sign of its sum
        const bool wlane = block_live && jl < bsz;
        const uint64_t zb = __ballot(wlane && !(w != 0.0f));
        const bool has_zero = ((zb >> half) & 0xFFFFFFFFull) != 0;
        if (wlane) a.w[r * a.wstride + (kp - kv_start)] = w;
        if (block_live && jl == 0) {
            a.bmax[r * a.nbstride + blk] = block_skipped ? NEG_INF : m;
            const float bs = block_skipped ? 0.0f : (half ? sumB : sumA);
            a.bsum[r * a.nbstride + blk] = has_zero ? set_sign(bs) : bs;
        }
    }
}

// ------------------------------------------------ kernel A, many query rows
// Prefill form of the scores.  A lane still owns one key, but a wave scores
// it against SQ_NQ query vectors (SQ_NQ/gq consecutive query rows times the
// gq heads of the kv head): the key row is loaded and converted once per 16
// dims for all of them.  A query vector enters the FMA through DPP
// row_newbcast from a register that holds 16 of its dims replicated over the
// four 16-lane rows, so a score step is one VALU op.  The reference's
// per-score order is kept: accumulator c of query q takes dims 8i+c in
// increasing i, then ((c0+c4)+(c1+c5)) + ((c2+c6)+(c3+c7)), times scale.
// The INT8 key value (float)code * scale is formed as
// fma((float)(code + 128), scale, -128 * scale): the exact product rounded
// once, the same float as the reference's rounded multiply.  Block sums run
// in the reference's sequential order in one lane per (query, block), from
// the wave's weights in LDS.
constexpr int SQ_NQ = 8;

template <int NQ, int K>
__device__ __forceinline__ void sq_step(float (&acc)[NQ][8], const float (&qv)[NQ], float k) {
#pragma unroll
    for (int q = 0; q < NQ; q++) fmac_row_bcast<K>(acc[q][K & 7], qv[q], k);
}
template <int NQ, int... K>
__device__ __forceinline__ void sq_group16(float (&acc)[NQ][8], const float (&qv)[NQ], const float* kk,
                                           std::integer_sequence<int, K...>) {
    asm volatile("s_nop 1");   // DPP source read after a possible VALU write of qv
    (sq_step<NQ, K>(acc, qv, kk[K]), ...);
}

// NQ query vectors per wave, NW waves (64-key chunks) per workgroup.  The
// prefill form is NQ = 8, NW = 4; the decode form (one query row) is
// NQ = 1, NW = 1, the gq heads of a kv head in gq workgroups per chunk
// (hsplit), with the lane's whole INT8 key row loaded before the query, so
// the two memory round trips overlap.
template <bool HYBRID, int D, int NQ, int NW>
__global__ void __launch_bounds__(64 * NW) attn_scores_rows_kernel(AttnArgs a_in) {
    constexpr bool PRE = NQ <= 2;                      // key row preloaded
    const AttnArgs a = resolve(a_in);
    __shared__ float qsh[NQ][D];
    __shared__ __align__(16) float wsh[NW][NQ][64];
    __shared__ float msh[NW][NQ][2];
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    // gq: the query heads of the kv head this workgroup takes (all of them,
    // or 1 / hsplit of them in the decode form)
    const int hsp = a.hsplit > 1 ? a.hsplit : 1;
    const int gq = a.gq / hsp, qr = NQ / gq;
    const int ngrp = (a.S + qr - 1) / qr;
    size_t gy = blockIdx.y;                            // (b, row group, kv head)
    unsigned bx = blockIdx.x, nbx = gridDim.x;         // chunk, chunks (+ appender)
    int hs = 0;                                        // head share of the split
    if (a.xcd_chunks) {
        const int L = blockIdx.x;
        int j = L >> 3;
        nbx = (unsigned)(a.xcd_chunks / hsp);
        bx = (unsigned)(j % a.xcd_chunks);
        hs = (int)(bx % (unsigned)hsp);
        bx /= (unsigned)hsp;
        j /= a.xcd_chunks;
        const int kvx = (L & 7) + 8 * (j / a.xcd_rest);
        if (kvx >= a.Hkv) return;                      // whole workgroup, before any barrier
        gy = (size_t)(j % a.xcd_rest) * a.Hkv + kvx;
    }
    const int kvh = (int)(gy % a.Hkv);
    gy /= a.Hkv;
    const int qp0 = (int)(gy % ngrp) * qr;
    const size_t b = gy / ngrp;
    const int d = a.d;
    const int h0 = kvh * a.gq + hs * gq;
    // per query vector: its row's key range (kv_start is 0 on this path)
    const float NEG_INF = -__builtin_inff();
    size_t kv_end_max = 0;
    for (int r = 0; r < qr; r++) {
        if (qp0 + r >= a.S) break;
        size_t s0, e, bl;
        kv_range<HYBRID>(a, (size_t)(qp0 + r), s0, e, bl);
        if (e > kv_end_max) kv_end_max = e;
    }
    const size_t chunk = (size_t)bx * NW + wid;
    const size_t wbase = chunk * 64;                   // first key of the wave
    const int jl = lane & 31;
    const size_t bs0 = wbase + (lane & 32);
    const size_t kp = wbase + lane;
    const bool kload = kp < kv_end_max;
    const bool kint8 = HYBRID && kp < a.cache_len;
    const int8_t* krow8 = nullptr;
    const uint16_t* krow16 = nullptr;
    const float* ksr = nullptr;
    if (kint8) {
        krow8 = a.kc + ((b * a.cache_len + kp) * a.Hkv + kvh) * (size_t)d;
        ksr = a.ks + (kp * a.Hkv + kvh) * (size_t)a.nqg;   // no batch offset (kernel_attention.cpp:353)
    } else {
        const size_t kpos = HYBRID ? kp - a.cache_len : kp;
        const size_t klen = HYBRID ? a.new_len : a.Skv;
        krow16 = a.k + ((b * klen + kpos) * a.Hkv + kvh) * (size_t)d;
    }
    // decode form: the lane's INT8 key row, loaded branch-free (a lane
    // without a cached key reads a stand-in row, its values unused) so no
    // wait is forced at the load; issued after the head preparation's own
    // loads when that runs here
    uint4 pre[PRE ? D / 16 : 1];
    float pres = 0.0f;
    auto preload = [&]() {
        if constexpr (PRE) {
            const bool own = kload && kint8;
            const void* stand_in = a.prep.q_raw ? (const void*)a.prep.q_raw : (const void*)a.q;
            const int8_t* src = own ? krow8 : reinterpret_cast<const int8_t*>(stand_in);
            const float* ssrc = own ? ksr : reinterpret_cast<const float*>(stand_in);
#pragma unroll
            for (int m = 0; m < D / 16; m++) pre[m] = *reinterpret_cast<const uint4*>(src + 16 * m);
            pres = ssrc[0];
        }
    };
    // decode form with the head preparation fused in (one wave, one row):
    // q of the group's heads and, in the chunk holding it, the new key row
    // get the reference's head RMSNorm and RoPE here (the step's attn_prep
    // arithmetic, kernel_attention.cpp:484-676); that chunk also appends the
    // new key and value to the INT8 cache (and the value's product tiles)
    __shared__ uint16_t prow[PRE ? NQ + 1 : 1][PRE ? D : 1];
    __shared__ uint16_t pys[PRE ? NQ + 1 : 1][PRE ? D : 1];
    __shared__ uint16_t krot[PRE ? D : 1];
    __shared__ __align__(16) float nk_acc[PRE ? NQ : 1][8];
    bool nk_lane = false;                               // the new key's accumulators come from nk_acc
    if constexpr (PRE && NW == 1) {
        if (a.prep.q_raw) {
            const bool appender = bx == nbx - 1;
            if (appender && hs != 0) return;               // one appender per kv head
            if (!appender && wbase >= kv_end_max) return;   // one wave: no barrier waits for it
            const int end8 = (d / 8) * 8, half = d / 2, vh = (half / 8) * 8;
            const uint32_t pos = (uint32_t)a.pos_off;
            const bool tab_ok = pos < a.prep.table_pos;
            const bool has_k = appender || (wbase <= a.cache_len && a.cache_len < wbase + 64);
            const int nq = appender ? 0 : NQ;            // q rows of this workgroup
            // every operand of the rows' RMSNorm and RoPE is loaded up front
            constexpr int EPL = D / 64;                   // elements per lane of a row
            uint16_t raw[NQ + 1][EPL], nwq[EPL], nwk[EPL];
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const int i = lane + 64 * e;
#pragma unroll
                for (int r = 0; r < NQ; r++) raw[r][e] = nq ? a.prep.q_raw[(size_t)(h0 + r) * d + i] : (uint16_t)0;
                raw[NQ][e] = has_k ? a.prep.k_raw[(size_t)kvh * d + i] : (uint16_t)0;
                nwq[e] = a.prep.q_norm[i];
                nwk[e] = a.prep.k_norm[i];
            }
            const size_t trow = (size_t)(tab_ok ? pos : 0) * half;
            const uint16_t cv = lane < half ? a.prep.cos_t[trow + lane] : (uint16_t)0;
            const uint16_t sv = lane < half ? a.prep.sin_t[trow + lane] : (uint16_t)0;
            preload();   // (the appender too: no branch around loads)
            // rows r < nq: q heads h0 + r; row NQ: the new key
#pragma unroll
            for (int r = 0; r <= NQ; r++)
#pragma unroll
                for (int e = 0; e < EPL; e++) prow[r][lane + 64 * e] = raw[r][e];
            wave_lds_order();
            // the NQ + 1 rows' statistics at once, one 16-lane row each (a
            // row that is not prepared gets values that are never used)
            float inv[NQ + 1];
            uint16_t hinv[NQ + 1];
            rms_stats_rows<D, NQ + 1>(&prow[0][0], D, a.prep.eps, inv, hinv);
#pragma unroll
            for (int r = 0; r <= NQ; r++)
#pragma unroll
                for (int e = 0; e < EPL; e++) {
                    const int i = lane + 64 * e;
                    pys[r][i] = rms_apply(raw[r][e], r < NQ ? nwq[e] : nwk[e], i, end8, inv[r], hinv[r]);
                }
            wave_lds_order();
            // RoPE (kernel_attention.cpp:640-671): pair (i, i + d/2), lane i
#pragma unroll
            for (int r = 0; r <= NQ; r++) {
                if (lane < half && ((r < nq) || (r == NQ && has_k))) {
                    const uint16_t x1 = pys[r][lane], x2 = pys[r][lane + half];
                    uint16_t o1, o2;
                    if (lane < vh) {
                        o1 = hfma(x2 ^ 0x8000u, sv, hmul(x1, cv));
                        o2 = hfma(x1, sv, hmul(x2, cv));
                    } else {
                        const float fa = h2f(x1), fb = h2f(x2), cf = h2f(cv), sf = h2f(sv);
                        o1 = f2h(fa * cf - fb * sf);
                        o2 = f2h(fb * cf + fa * sf);
                    }
                    if (r < NQ) {
                        qsh[r][lane] = tab_ok ? h2f(o1) : 0.0f;
                        qsh[r][lane + half] = tab_ok ? h2f(o2) : 0.0f;
                    } else {
                        krot[lane] = o1;
                        krot[lane + half] = o2;
                    }
                }
            }
            wave_lds_order();
            if (appender) {
                // the extra workgroup of the kv head appends the step's key
                // and value to the cache (read by later steps only)
                if (tab_ok && a.cache_len < a.max_cache) {
                    const int ng = (d + 127) / 128;
                    const size_t crow = (size_t)a.cache_len * a.Hkv + kvh;
                    kv_append_row(krot, a.prep.kc + crow * d, a.prep.ks + crow * ng, d);
                    kv_append_row(a.prep.v_raw + (size_t)kvh * d, a.prep.vc + crow * d, a.prep.vs + crow * ng, d,
                                  a.prep.vsh, a.sh_ntile, a.cache_len, kvh);
                }
                return;
            }
            // the new key's eight accumulators per query vector, lane
            // 8 q + c running accumulator c of query q over dims 8 i + c in
            // increasing i: the main loop's operands and order, one
            // D/8-step chain per lane instead of the key lane's fp16 row read
            // from LDS at every step of that loop
            if (has_k) {
                if (lane < 8 * NQ) {
                    const int q = lane >> 3, c = lane & 7;
                    float s = 0.0f;
#pragma unroll
                    for (int i = 0; i < D / 8; i++) s = __builtin_fmaf(qsh[q][8 * i + c], h2f(krot[8 * i + c]), s);
                    nk_acc[q][c] = s;
                }
                wave_lds_order();
                nk_lane = kp == a.cache_len;
            }
        }
    }
    if (!(PRE && NW == 1) || !a.prep.q_raw) {
        preload();
        for (int i = threadIdx.x; i < NQ * D; i += 64 * NW) {
            const int v = i / D, dim = i % D;
            const int qp = qp0 + v / gq;
            qsh[v][dim] = qp < a.S ? h2f(a.q[((b * a.S + qp) * a.Hq + h0 + v % gq) * (size_t)d + dim]) : 0.0f;
        }
    }
    __syncthreads();
    if (wbase >= kv_end_max) return;                   // wave-uniform; no barrier follows

    // ---- dot products of this lane's key with every query vector
    float acc[NQ][8];
#pragma unroll
    for (int q = 0; q < NQ; q++)
#pragma unroll
        for (int c = 0; c < 8; c++) acc[q][c] = 0.0f;
    const int lr = lane & 15;
    // prefill form: the next 16 dims of the key (codes and scale, or fp16
    // values) are loaded while the current 16 feed the FMAs, so a step's
    // global round trip overlaps the previous step's 128 FMAs
    // The loads take no branch: a lane past the last key reads the row of
    // the wave's last live key instead (its values are never used), an INT8
    // row is read through both pointers, an fp16 row as two halves.
    uint4 nx0[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    uint4 nx1[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    float nxs[2] = {0.0f, 0.0f};   // two buffers, alternating by step
    const bool one_scale = a.qgs >= D;
    float s_row = 0.0f;
    const uint8_t* ld0 = nullptr;
    const uint8_t* ld1 = nullptr;
    int ldstep = 0;
    if constexpr (!PRE) {
        if (kload && kint8 && one_scale) s_row = ksr[0];
        const size_t kpl = kload ? kp : kv_end_max - 1;   // kv_end_max > wbase here
        if (HYBRID && kpl < a.cache_len) {
            ld0 = reinterpret_cast<const uint8_t*>(a.kc + ((b * a.cache_len + kpl) * a.Hkv + kvh) * (size_t)d);
            ld1 = ld0;
            ldstep = 16;
        } else {
            const size_t kpos = HYBRID ? kpl - a.cache_len : kpl;
            const size_t klen = HYBRID ? a.new_len : a.Skv;
            ld0 = reinterpret_cast<const uint8_t*>(a.k + ((b * klen + kpos) * a.Hkv + kvh) * (size_t)d);
            ld1 = ld0 + 16;
            ldstep = 32;
        }
    }
    auto fetch = [&](int m) {
        if constexpr (!PRE) {
            nx0[m & 1] = *reinterpret_cast<const uint4*>(ld0 + (size_t)ldstep * m);
            nx1[m & 1] = *reinterpret_cast<const uint4*>(ld1 + (size_t)ldstep * m);
            if (!one_scale) nxs[m & 1] = (kload && kint8) ? ksr[(16 * m) / a.qgs] : 0.0f;
        }
    };
    // decode form: every step's query values in registers before the loop
    // (a read from LDS right before its step's FMAs would wait out the LDS
    // latency at each of the D/16 steps)
    float qall[PRE ? D / 16 : 1][NQ];
    if constexpr (PRE) {
#pragma unroll
        for (int m = 0; m < D / 16; m++)
#pragma unroll
            for (int q = 0; q < NQ; q++) qall[m][q] = qsh[q][16 * m + lr];
    }
    auto conv_i8 = [](float (&kk)[16], const uint4 raw, const float s) {
        const float ns = -128.0f * s;
        const uint32_t w4[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                                raw.w ^ 0x80808080u};
#pragma unroll
        for (int e = 0; e < 16; e++)
            kk[e] = __builtin_fmaf((float)((w4[e >> 2] >> (8 * (e & 3))) & 0xFFu), s, ns);
    };
    auto conv_f16 = [](float (&kk)[16], const uint4 r0, const uint4 r1) {
        const uint32_t h[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kk[2 * e] = h2f((uint16_t)(h[e] & 0xFFFF));
            kk[2 * e + 1] = h2f((uint16_t)(h[e] >> 16));
        }
    };
    // one 16-dim step; ALL_I8: the fused decode form with one scale per key
    // row, where every lane converts its preloaded INT8 row without a branch
    // (a lane past the last key converts its stand-in row and the new key's
    // lane its own, unused: their scores are not computed, or replaced below)
    auto step = [&](int m, auto all_i8) {
        float kk[16];
        if constexpr (PRE && decltype(all_i8)::value) {
            conv_i8(kk, pre[m], pres);
        } else if constexpr (PRE) {
            if (kload && kint8) {
                conv_i8(kk, pre[m], (a.qgs >= D) ? pres : ksr[(16 * m) / a.qgs]);
            } else if (kload && !nk_lane) {
                conv_f16(kk, *reinterpret_cast<const uint4*>(krow16 + 16 * m),
                         *reinterpret_cast<const uint4*>(krow16 + 16 * m + 8));
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++) kk[e] = 0.0f;
            }
        } else {
            if (m + 1 < D / 16) fetch(m + 1);
            // a lane past the last key converts the row it loaded; its
            // scores are never used (not computed, or masked to -inf)
            if (ldstep == 16) conv_i8(kk, nx0[m & 1], one_scale ? s_row : nxs[m & 1]);
            else conv_f16(kk, nx0[m & 1], nx1[m & 1]);
        }
        float qv[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) qv[q] = PRE ? qall[m][q] : qsh[q][16 * m + lr];
        sq_group16<NQ>(acc, qv, kk, std::make_integer_sequence<int, 16>{});
    };
    fetch(0);
    bool all_i8 = false;
    if constexpr (PRE && NW == 1 && HYBRID) all_i8 = a.prep.q_raw != nullptr && a.qgs >= D;
    if (all_i8) {
#pragma unroll
        for (int m = 0; m < D / 16; m++) step(m, std::true_type{});
    } else {
#pragma unroll
        for (int m = 0; m < D / 16; m++) step(m, std::false_type{});
    }
    if constexpr (PRE && NW == 1) {
        if (__builtin_amdgcn_readfirstlane(__ballot(nk_lane) != 0ull ? 1 : 0)) {   // the new key's chunk only
            typedef float f4v __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                const f4v lo = *reinterpret_cast<const f4v*>(&nk_acc[q][0]);
                const f4v hi = *reinterpret_cast<const f4v*>(&nk_acc[q][4]);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    acc[q][c] = nk_lane ? lo[c] : acc[q][c];
                    acc[q][c + 4] = nk_lane ? hi[c] : acc[q][c + 4];
                }
            }
        }
    }

    // ---- per query vector: mask, block max, weight, stores
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int qp = qp0 + q / gq;
        const bool row_ok = qp < a.S;
        const size_t aq = a.pos_off + qp;
        size_t s0 = 0, kv_end = 0, blk_limit = 0;
        if (row_ok) kv_range<HYBRID>(a, (size_t)qp, s0, kv_end, blk_limit);
        const bool block_live = row_ok && bs0 < kv_end;
        const size_t be = block_live ? ((bs0 + ATT_BLOCK < blk_limit) ? bs0 + ATT_BLOCK : blk_limit) : bs0;
        const int bsz = (int)(be - bs0);
        const bool is_decode = (!HYBRID) && (qp == a.S - 1) && a.S > 1;
        const bool block_skipped = !HYBRID && !is_decode && a.causal && bs0 > aq;
        const bool in_block = block_live && jl < bsz && !block_skipped;
        bool computed = in_block;
        if (computed && a.causal && kp > aq && (HYBRID || !is_decode)) computed = false;
        float sc = NEG_INF;
        if (computed) {
            const float t0 = acc[q][0] + acc[q][4], t1 = acc[q][1] + acc[q][5];
            const float t2 = acc[q][2] + acc[q][6], t3 = acc[q][3] + acc[q][7];
            sc = ((t0 + t1) + (t2 + t3)) * a.scale;
            if (!HYBRID) {
                if (a.causal && kp > aq) sc = NEG_INF;
                else if (a.mask && h2f(a.mask[(b * a.S + qp) * a.Skv + kp]) == 0.0f) sc = NEG_INF;
            }
        }
        const float mx = half_wave_max(sc);
        const int vs4 = HYBRID ? 0 : (bsz / 4) * 4;
        float w = 0.0f;
        if (in_block) {
            if (jl < vs4) w = poly_exp_weight(sc, mx);
            else w = (sc != NEG_INF) ? cactus_expf(sc - mx) : 0.0f;
        }
        const bool wlane = block_live && jl < bsz;
        const size_t row = (b * a.S + (row_ok ? qp : 0)) * a.Hq + h0 + q % gq;
        if (wlane) a.w[row * a.wstride + kp] = w;
        wsh[wid][q][lane] = w;
        if (jl == 0) msh[wid][q][lane >> 5] = mx;
    }
    wave_lds_order();
    // ---- block sums, one lane per (query vector, block), reference order
    if (lane < 2 * NQ) {
        const int q = lane >> 1, half = lane & 1;
        const int qp = qp0 + q / gq;
        const size_t bs = wbase + 32 * half;
        if (qp < a.S) {
            const size_t aq = a.pos_off + qp;
            size_t s0, kv_end, blk_limit;
            kv_range<HYBRID>(a, (size_t)qp, s0, kv_end, blk_limit);
            if (bs < kv_end) {
                const size_t be = (bs + ATT_BLOCK < blk_limit) ? bs + ATT_BLOCK : blk_limit;
                const int bsz = (int)(be - bs);
                const bool is_decode = (!HYBRID) && (qp == a.S - 1) && a.S > 1;
                const bool block_skipped = !HYBRID && !is_decode && a.causal && bs > aq;
                // the block's 32 weights by eight 16-byte reads first (the slots
                // past bsz hold other keys' weights or stale values; they are
                // selected out), then the fold in the reference's order
                typedef float f4v __attribute__((ext_vector_type(4)));
                const f4v* x4 = reinterpret_cast<const f4v*>(&wsh[wid][q][32 * half]);
                float x[32];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const f4v v = x4[t];
                    x[4 * t] = v.x; x[4 * t + 1] = v.y; x[4 * t + 2] = v.z; x[4 * t + 3] = v.w;
                }
                const int v4 = HYBRID ? 0 : (bsz / 4) * 4;
                float sum = 0.0f;
                bool has_zero = false;
#pragma unroll
                for (int j = 0; j < 32; j += 4) {
                    if (!HYBRID && j < v4) {
                        sum = sum + ((x[j] + x[j + 1]) + (x[j + 2] + x[j + 3]));
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; u++) sum = j + u < bsz ? sum + x[j + u] : sum;
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) has_zero |= j + u < bsz && !(x[j + u] != 0.0f);
                }
                const size_t row = (b * a.S + qp) * a.Hq + h0 + q % gq;
                const int blk = (int)(bs / ATT_BLOCK);
                a.bmax[row * a.nbstride + blk] = block_skipped ? NEG_INF : msh[wid][q][half];
                const float bsv = block_skipped ? 0.0f : sum;
                a.bsum[row * a.nbstride + blk] = has_zero ? set_sign(bsv) : bsv;
            }
        }
    }
}

// ----------------------------------------------------------------- kernel B
// The value accumulation is one fp32 FMA chain per (query, head, dimension)
// over the keys in order, rescaled at every block whose max is finite
// (kernel_attention.cpp:160-169 and :199-217 for FP16, :396-455 for the
// hybrid), so it is latency-bound: the chains must run at FMA cadence.
//
// One workgroup per (b, group of `qpg` query positions, kv head, 64-dim
// slice).  Waves 0..nc-1 (nc = qpg * gq) are chain waves: wave c owns query
// position qp0 + c / gq and head kvh * gq + c % gq, each lane one output
// dimension.  The CH_NP stage waves convert value rows into the reference's
// fp32 operands (INT8 code * per-key group scale, or fp16 -> fp32) and stage
// them, with the chain waves' weights, in LDS one CH_T-key tile ahead of the
// chains, so a chain step is one broadcast LDS read and one FMA.
constexpr int CH_T = 128;              // keys per staged tile
constexpr int CH_NP = 2;               // stage waves
constexpr int CH_PS = CH_T + 4;        // floats per staged dimension row (bank skew)
constexpr int CH_MAX_THREADS = 64 * (ATT_MAX_GQ + CH_NP);

template <bool HYBRID>
__global__ void __launch_bounds__(CH_MAX_THREADS) attn_chain_kernel(AttnArgs a_in, int qpg, int nbmax,
                                                                     int vec_ok) {
    const AttnArgs a = resolve(a_in);
    extern __shared__ __align__(16) unsigned char smem[];
    const int gq = a.gq, nc = qpg * gq;
    float* prod = reinterpret_cast<float*>(smem);            // [2][64][CH_PS]
    float* wts = prod + 2 * 64 * CH_PS;                      // [2][nc][CH_T]
    float* corr_s = wts + 2 * nc * CH_T;                     // [nc][nbmax]
    float* bsum_s = corr_s + (size_t)nc * nbmax;             // [nc][nbmax]
    const float NEG_INF = -__builtin_inff();

    const int d = a.d, da = (d / 8) * 8;
    const int nsl = (d + 63) / 64;
    size_t g = blockIdx.x;
    const int sl = (int)(g % nsl);
    g /= nsl;
    const int kvh = (int)(g % a.Hkv);
    g /= a.Hkv;
    const int ngrp = (a.S + qpg - 1) / qpg;
    const int qp0 = (int)(g % ngrp) * qpg;
    const size_t b = g / ngrp;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;

    // keys of the group: every row starts at the same kv_start (the host
    // uses qpg = 1 for a sliding window); the last position reaches furthest
    size_t ks, ke_first, bl_first;
    kv_range<HYBRID>(a, (size_t)qp0, ks, ke_first, bl_first);
    const int qlast = min(qp0 + qpg, a.S) - 1;
    size_t ks_l, ke_l, bl_l;
    kv_range<HYBRID>(a, (size_t)qlast, ks_l, ke_l, bl_l);
    size_t kneed = ks;
    if (ke_l > ks) {
        kneed = ks + ((ke_l - ks + ATT_BLOCK - 1) / ATT_BLOCK) * ATT_BLOCK;
        if (kneed > bl_l) kneed = bl_l;
    }
    const int nst = (int)((kneed - ks + CH_T - 1) / CH_T);

    // ---- stage waves: tile t -> buffer t & 1
    auto stage = [&](int t) {
        const int pl = (int)threadIdx.x - nc * 64;
        const size_t tb = ks + (size_t)t * CH_T;
        float* pbuf = prod + (t & 1) * 64 * CH_PS;
        for (int item = pl; item < (CH_T / 4) * 16; item += CH_NP * 64) {
            const int dq = item & 15, kq = item >> 4;
            const int dim0 = sl * 64 + dq * 4;
            float pr[4][4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const size_t kp = tb + kq * 4 + e;
#pragma unroll
                for (int c = 0; c < 4; c++) pr[e][c] = 0.0f;
                if (kp >= kneed || dim0 >= da) continue;
                if (HYBRID && kp < a.cache_len) {
                    const size_t off = (b * a.cache_len + kp) * a.Hkv + kvh;
                    const int8_t* src = a.vc + off * d + dim0;
                    // value scales carry no batch offset (kernel_attention.cpp:424)
                    const float sc = a.vs[(kp * a.Hkv + kvh) * a.nqg + dim0 / a.qgs];
                    int8_t cd[4];
                    if (vec_ok) {
                        const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
#pragma unroll
                        for (int c = 0; c < 4; c++) cd[c] = (int8_t)((w >> (8 * c)) & 0xFF);
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; c++) cd[c] = src[c];
                    }
#pragma unroll
                    for (int c = 0; c < 4; c++) pr[e][c] = (float)cd[c] * sc;
                } else {
                    const size_t vpos = HYBRID ? kp - a.cache_len : kp;
                    const size_t vlen = HYBRID ? a.new_len : a.Skv;
                    const uint16_t* src = a.v + ((b * vlen + vpos) * a.Hkv + kvh) * (size_t)d + dim0;
                    if (vec_ok) {
                        const uint2 w = *reinterpret_cast<const uint2*>(src);
                        pr[e][0] = h2f((uint16_t)(w.x & 0xFFFF));
                        pr[e][1] = h2f((uint16_t)(w.x >> 16));
                        pr[e][2] = h2f((uint16_t)(w.y & 0xFFFF));
                        pr[e][3] = h2f((uint16_t)(w.y >> 16));
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; c++) pr[e][c] = h2f(src[c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                *reinterpret_cast<float4*>(pbuf + (dq * 4 + c) * CH_PS + kq * 4) =
                    make_float4(pr[0][c], pr[1][c], pr[2][c], pr[3][c]);
        }
        // weights of the chain rows for this tile (columns beyond a row's
        // keys are never read by its chain)
        float* wbuf = wts + (t & 1) * nc * CH_T;
        for (int i = pl; i < nc * (CH_T / 4); i += CH_NP * 64) {
            const int c = i / (CH_T / 4), j4 = (i % (CH_T / 4)) * 4;
            const int qp = qp0 + c / gq;
            float4 w4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const size_t col = (size_t)t * CH_T + j4;
            if (qp < a.S && col + 4 <= a.wstride) {
                const size_t row = (b * a.S + qp) * a.Hq + kvh * gq + (c % gq);
                w4 = *reinterpret_cast<const float4*>(a.w + row * a.wstride + col);
            }
            *reinterpret_cast<float4*>(wbuf + c * CH_T + j4) = w4;
        }
    };

    // ---- chain waves: block rescale factors of the row
    const bool is_chain = wv < nc;
    const int qp = qp0 + (is_chain ? wv / gq : 0);
    const bool row_ok = is_chain && qp < a.S;
    const size_t row = (b * a.S + (size_t)(row_ok ? qp : 0)) * a.Hq + kvh * gq + (is_chain ? wv % gq : 0);
    size_t rks = 0, rke = 0, rbl = 0;
    int nb = 0;
    if (row_ok) {
        kv_range<HYBRID>(a, (size_t)qp, rks, rke, rbl);
        nb = rke > rks ? (int)((rke - rks + ATT_BLOCK - 1) / ATT_BLOCK) : 0;
    }
    if (row_ok) {
        // corr[blk] = expf(running max before blk - block max) when the block
        // max is finite (the running max is the last finite block max), else
        // NEG_INF: the block leaves the accumulators unscaled
        const float* bm = a.bmax + row * a.nbstride;
        const float* bsm = a.bsum + row * a.nbstride;
        float carry = NEG_INF;
        for (int c0 = 0; c0 < nb; c0 += 64) {
            const int i = c0 + lane;
            const float m = i < nb ? bm[i] : NEG_INF;
            const float bs = i < nb ? bsm[i] : 0.0f;
            const bool fin = m > NEG_INF;
            int idx = fin ? lane : -1;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int o = __shfl_up(idx, off, 64);
                if (lane >= off) idx = max(idx, o);
            }
            int ex = __shfl_up(idx, 1, 64);
            if (lane == 0) ex = -1;
            const float pm = __shfl(m, ex < 0 ? 0 : ex, 64);
            const float prev = ex >= 0 ? pm : carry;
            if (i < nb) {
                corr_s[wv * nbmax + i] = fin ? cactus_expf(prev - m) : NEG_INF;
                bsum_s[wv * nbmax + i] = bs;
            }
            const int last = __shfl(idx, 63, 64);
            if (last >= 0) carry = __shfl(m, last, 64);
        }
    }
    if (!is_chain && nst > 0) stage(0);

    float acc = 0.0f, rs = 0.0f;
    const int dim = sl * 64 + lane;
    for (int t = 0; t < nst; t++) {
        __syncthreads();
        if (!is_chain) {
            if (t + 1 < nst) stage(t + 1);
            continue;
        }
        if (!row_ok) continue;
        const float* pt = prod + (t & 1) * 64 * CH_PS + lane * CH_PS;
        const float* wt = wts + ((t & 1) * nc + wv) * CH_T;
        const int b0 = t * (CH_T / ATT_BLOCK);
        const int b1 = min(nb, b0 + CH_T / ATT_BLOCK);
        for (int blk = b0; blk < b1; blk++) {
            const float c = corr_s[wv * nbmax + blk];
            const float bse = bsum_s[wv * nbmax + blk];
            if (c != NEG_INF) {
                acc = acc * c;
                rs = rs * c;
            }
            const size_t bs0 = rks + (size_t)blk * ATT_BLOCK;
            const size_t be = bs0 + ATT_BLOCK < rbl ? bs0 + ATT_BLOCK : rbl;
            const int bsz = (int)(be - bs0);
            const int jo = (blk - b0) * ATT_BLOCK;
            if (bsz == ATT_BLOCK && !__builtin_signbit(bse)) {
                float4 pv[8], wv4[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    pv[j] = *reinterpret_cast<const float4*>(pt + jo + 4 * j);
                    wv4[j] = *reinterpret_cast<const float4*>(wt + jo + 4 * j);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    acc = __builtin_fmaf(pv[j].x, wv4[j].x, acc);
                    acc = __builtin_fmaf(pv[j].y, wv4[j].y, acc);
                    acc = __builtin_fmaf(pv[j].z, wv4[j].z, acc);
                    acc = __builtin_fmaf(pv[j].w, wv4[j].w, acc);
                }
            } else {
                // a zero weight is skipped (kernel_attention.cpp:200-201): an
                // FMA with it could turn an accumulator of -0 into +0
                for (int j = 0; j < bsz; j++) {
                    const float w = wt[jo + j];
                    if (w != 0.0f) acc = __builtin_fmaf(pt[jo + j], w, acc);
                }
            }
            rs = rs + __builtin_fabsf(bse);
        }
    }
    if (row_ok && dim < d) {
        uint16_t* ov = a.o + row * (size_t)d;
        if (!(rs > 0.0f) || dim >= da) ov[dim] = 0;
        else ov[dim] = f2h(acc * (1.0f / rs));
    }
}

// ------------------------------------------------ kernel B, LDS-DMA form
// The same chains as attn_chain_kernel with the value tiles fetched by
// gfx950 LDS DMA (global_load_lds_dword[x4]): the stage waves keep
// CdCfg::D - 1 tiles of raw value rows, scales and weights in flight in an
// LDS ring without holding them in registers, convert one tile per step and
// never wait for more than the oldest tile.  Keys outside the tiles (the
// hybrid's new fp16 rows) are read by the chains directly.
//
// The DMA is issued from inline assembly so that the compiler does not make
// every LDS read wait for every outstanding DMA; the waits are explicit
// (s_waitcnt vmcnt) and the step barrier waits for LDS only.  M0 carries
// the LDS destination; nothing else in these kernels uses M0.
constexpr int CD_T = 64;               // keys per tile
constexpr int CD_PS = CD_T + 4;        // floats per product row (bank skew)
constexpr int CD_NP = 4;               // stage waves
constexpr int CD_KPW = CD_T / CD_NP;   // keys of a tile per stage wave
constexpr int CD_WR = ATT_MAX_GQ / CD_NP;  // weight rows per stage wave

template <bool HYBRID, int DW>
struct CdCfg {
    static constexpr int D = DW == 16 ? 8 : 5;                  // ring depth (tiles)
    static constexpr int ROW_B = HYBRID ? 64 : 128;             // bytes of a 64-dim key row
    static constexpr int ROWS_LPT = CD_KPW * ROW_B / (64 * DW); // DMA per stage wave per tile
    static constexpr int SC_LPT = HYBRID ? 1 : 0;
    static constexpr int W_LPT = (CD_WR * 256 + 64 * DW - 1) / (64 * DW);
    static constexpr int LPT = ROWS_LPT + SC_LPT + W_LPT;
    static constexpr int VM_WAIT = (D - 2) * LPT;               // DMA younger than the next tile
    static constexpr int ROWS_OFF = 0;
    static constexpr int SC_OFF = CD_T * ROW_B;
    static constexpr int W_OFF = SC_OFF + (HYBRID ? CD_T * 4 : 0);
    static constexpr int SLOT = W_OFF + ATT_MAX_GQ * CD_T * 4;
    static_assert(VM_WAIT <= 63, "vmcnt range");
    static_assert(ROWS_LPT * 64 * DW == CD_KPW * ROW_B, "row chunks");
};

// Block rescale factors of one chain row, into LDS: corr[blk] =
// expf(running max before blk - block max) when the block max is finite
// (the running max is the last finite block max), else NEG_INF (the block
// leaves the accumulators unscaled); bsum[blk] is the block's flagged sum.
// One whole wave.
__device__ __forceinline__ void chain_corr_scan(int nb, float* corr);
__device__ __forceinline__ void chain_corr(const AttnArgs& a, size_t row, int nb, float* corr, float* bsum) {
    const int lane = threadIdx.x & 63;
    const float* bm = a.bmax + row * a.nbstride;
    const float* bsm = a.bsum + row * a.nbstride;
#pragma unroll 4
    for (int i = lane; i < nb; i += 64) {
        corr[i] = bm[i];
        bsum[i] = bsm[i];
    }
    chain_corr_scan(nb, corr);
}
// block maxima in corr[0, nb) -> the corrections, in place (one wave)
__device__ __forceinline__ void chain_corr_scan(int nb, float* corr) {
    const int lane = threadIdx.x & 63;
    const float NEG_INF = -__builtin_inff();
    float carry = NEG_INF;
    for (int c0 = 0; c0 < nb; c0 += 64) {
        const int i = c0 + lane;
        const float m = i < nb ? corr[i] : NEG_INF;
        const bool fin = m > NEG_INF;
        int idx = fin ? lane : -1;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(idx, off, 64);
            if (lane >= off) idx = max(idx, o);
        }
        int ex = __shfl_up(idx, 1, 64);
        if (lane == 0) ex = -1;
        const float pm = __shfl(m, ex < 0 ? 0 : ex, 64);
        const float prev = ex >= 0 ? pm : carry;
        if (i < nb) corr[i] = fin ? cactus_expf(prev - m) : NEG_INF;
        const int last = __shfl(idx, 63, 64);
        if (last >= 0) carry = __shfl(m, last, 64);
    }
}

// 16 chain steps: keys k = 0..15 with products p[k], weights in lanes k of wv
template <int... K>
__device__ __forceinline__ void chain16(float& acc, const float* p, float wv, std::integer_sequence<int, K...>) {
    asm volatile("s_nop 1");   // DPP source read after a possible VALU write of wv
    (fmac_row_bcast<K>(acc, wv, p[K]), ...);
}

// One tile of a chain row: blocks [b0, b1), all keys inside the tile; pt
// is this lane's product row of the tile, wt the row's weights.
__device__ __forceinline__ void chain_tile(const float* pt, const float* wt, int b0, int b1, size_t rks,
                                           size_t rbl, const float* cw, const float* cb, float& acc,
                                           float& rs, const float* meta = nullptr) {
    const float NEG_INF = -__builtin_inff();
    // both blocks of the tile full: every LDS read of the tile at once;
    // weights row-replicated into 4 VGPRs (16 keys each) for the DPP steps.
    // meta: the blocks' {corr, corr, sum, sum} read ahead by the caller
    if (b1 - b0 == 2 && rks + (size_t)(b0 + 2) * ATT_BLOCK <= rbl) {
        const float c0 = meta ? meta[0] : cw[b0], c1 = meta ? meta[1] : cw[b0 + 1];
        const float s0 = meta ? meta[2] : cb[b0], s1 = meta ? meta[3] : cb[b0 + 1];
        if (!__builtin_signbit(s0) && !__builtin_signbit(s1)) {
            const int lr = threadIdx.x & 15;
            float pv[64];
            float wv[4];
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const float4 v = *reinterpret_cast<const float4*>(pt + 4 * q);
                pv[4 * q] = v.x;
                pv[4 * q + 1] = v.y;
                pv[4 * q + 2] = v.z;
                pv[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int q = 0; q < 4; q++) wv[q] = wt[16 * q + lr];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float c = h ? c1 : c0;
                if (c != NEG_INF) {
                    acc = acc * c;
                    rs = rs * c;
                }
                chain16(acc, pv + 32 * h, wv[2 * h], std::make_integer_sequence<int, 16>{});
                chain16(acc, pv + 32 * h + 16, wv[2 * h + 1], std::make_integer_sequence<int, 16>{});
                rs = rs + (h ? s1 : s0);
            }
            return;
        }
    }
    for (int blk = b0; blk < b1; blk++) {
        const float c = cw[blk];
        const float bse = cb[blk];
        if (c != NEG_INF) {
            acc = acc * c;
            rs = rs * c;
        }
        const size_t bs0 = rks + (size_t)blk * ATT_BLOCK;
        const size_t be = bs0 + ATT_BLOCK < rbl ? bs0 + ATT_BLOCK : rbl;
        const int bsz = (int)(be - bs0);
        const int jo = (blk - b0) * ATT_BLOCK;
        if (bsz == ATT_BLOCK && !__builtin_signbit(bse)) {
            float4 pv[8], wq[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                pv[j] = *reinterpret_cast<const float4*>(pt + jo + 4 * j);
                wq[j] = *reinterpret_cast<const float4*>(wt + jo + 4 * j);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                acc = __builtin_fmaf(pv[j].x, wq[j].x, acc);
                acc = __builtin_fmaf(pv[j].y, wq[j].y, acc);
                acc = __builtin_fmaf(pv[j].z, wq[j].z, acc);
                acc = __builtin_fmaf(pv[j].w, wq[j].w, acc);
            }
        } else {
            // a zero weight is skipped (kernel_attention.cpp:200-201): an
            // FMA with it could turn an accumulator of -0 into +0
            for (int j = 0; j < bsz; j++) {
                const float w = wt[jo + j];
                if (w != 0.0f) acc = __builtin_fmaf(pt[jo + j], w, acc);
            }
        }
        rs = rs + __builtin_fabsf(bse);
    }
}

// Blocks of a chain row reaching past the tiles: tile keys from the last
// tile (tbase: its first key; pt, wt as in chain_tile), the hybrid's new
// rows read directly (pf: the first new row, loaded early).
template <bool HYBRID>
__device__ __forceinline__ void chain_tail(const AttnArgs& a, size_t b, int kvh, int dim, size_t row, int nb_tile,
                                           int nb, size_t rks, size_t rbl, size_t kt_end, size_t tbase,
                                           const float* pt, const float* wt, bool pf, float pf_p, float pf_w,
                                           const float* cw, const float* cb, float& acc, float& rs) {
    const float NEG_INF = -__builtin_inff();
    const int d = a.d;
    for (int blk = nb_tile; blk < nb; blk++) {
        const float c = cw[blk];
        const float bse = cb[blk];
        if (c != NEG_INF) {
            acc = acc * c;
            rs = rs * c;
        }
        const size_t bs0 = rks + (size_t)blk * ATT_BLOCK;
        const size_t be = bs0 + ATT_BLOCK < rbl ? bs0 + ATT_BLOCK : rbl;
        const int bsz = (int)(be - bs0);
        // new rows past the prefetched one: one batch of loads per block
        float gp[ATT_BLOCK], gw[ATT_BLOCK];
#pragma unroll
        for (int j = 0; j < ATT_BLOCK; j++) {
            gp[j] = 0.0f;
            gw[j] = 0.0f;
        }
        if constexpr (HYBRID) {
            const size_t covered = pf ? (size_t)a.cache_len + 1 : kt_end;
            if (be > (covered > kt_end ? covered : kt_end)) {
                const int dimc = dim < d ? dim : d - 1;
#pragma unroll
                for (int j = 0; j < ATT_BLOCK; j++) {
                    size_t kp = bs0 + j;
                    if (kp >= be) kp = be - 1;
                    if (kp < a.cache_len) kp = a.cache_len;
                    gw[j] = a.w[row * a.wstride + (kp - rks)];
                    gp[j] = h2f(a.v[((b * a.new_len + (kp - a.cache_len)) * a.Hkv + kvh) * (size_t)d + dimc]);
                }
            }
        }
        float pv[ATT_BLOCK], wq[ATT_BLOCK];
#pragma unroll
        for (int j = 0; j < ATT_BLOCK; j++) {
            pv[j] = 0.0f;
            wq[j] = 0.0f;
            const size_t kp = bs0 + j;
            if (j < bsz) {
                if (kp < kt_end) {
                    pv[j] = pt[kp - tbase];
                    wq[j] = wt[kp - tbase];
                } else if (pf && kp == a.cache_len) {
                    pv[j] = pf_p;
                    wq[j] = pf_w;
                } else {
                    pv[j] = gp[j];
                    wq[j] = gw[j];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < ATT_BLOCK; j++)
            if (j < bsz && wq[j] != 0.0f) acc = __builtin_fmaf(pv[j], wq[j], acc);
        rs = rs + __builtin_fabsf(bse);
    }
}

template <bool HYBRID, int DW>
__global__ void __launch_bounds__(64 * (ATT_MAX_GQ + CD_NP)) attn_chain_dma_kernel(AttnArgs a_in, int qpg,
                                                                                    int nbmax) {
    using C = CdCfg<HYBRID, DW>;
    const AttnArgs a = resolve(a_in);
    extern __shared__ __align__(16) unsigned char smem[];
    const int gq = a.gq, nc = qpg * gq;
    unsigned char* ring = smem;                                            // [D][SLOT]
    float* prod = reinterpret_cast<float*>(smem + C::D * C::SLOT);         // [2][64][CD_PS]
    float* corr_s = prod + 2 * 64 * CD_PS;                                 // [nc][nbmax]
    float* bsum_s = corr_s + (size_t)nc * nbmax;                           // [nc][nbmax]
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)ring;

    const int d = a.d, da = (d / 8) * 8;
    const int nsl = (d + 63) / 64;
    size_t g = blockIdx.x;
    const int sl = (int)(g % nsl);
    g /= nsl;
    const int kvh = (int)(g % a.Hkv);
    g /= a.Hkv;
    const int ngrp = (a.S + qpg - 1) / qpg;
    const int qp0 = (int)(g % ngrp) * qpg;
    const size_t b = g / ngrp;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;

    size_t ks, ke_f, bl_f;
    kv_range<HYBRID>(a, (size_t)qp0, ks, ke_f, bl_f);
    const int qlast = min(qp0 + qpg, a.S) - 1;
    size_t ks_l, ke_l, bl_l;
    kv_range<HYBRID>(a, (size_t)qlast, ks_l, ke_l, bl_l);
    size_t kneed = ks;
    if (ke_l > ks) {
        kneed = ks + ((ke_l - ks + ATT_BLOCK - 1) / ATT_BLOCK) * ATT_BLOCK;
        if (kneed > bl_l) kneed = bl_l;
    }
    // keys served by tiles: the INT8 cache for the hybrid, all for FP16
    const size_t kt_end = HYBRID ? (kneed < a.cache_len ? kneed : (size_t)a.cache_len) : kneed;
    const int nst = kt_end > ks ? (int)((kt_end - ks + CD_T - 1) / CD_T) : 0;
    const bool is_chain = wv < nc;
    const int pw = wv - nc;

    // DMA sources of tile 0 per lane; a tile further is a fixed stride on
    // (the last tile clamps keys to the tile range instead)
    const size_t krow = (size_t)a.Hkv * d;                     // elements between keys
    const size_t vlen = HYBRID ? a.cache_len : a.Skv;
    const char* vbase = HYBRID ? reinterpret_cast<const char*>(a.vc) : reinterpret_cast<const char*>(a.v);
    constexpr int ESZ = HYBRID ? 1 : 2;
    auto row_src = [&](int i, size_t kp) -> const char* {
        const int o = i * 64 * DW + lane * DW;
        int cel = (o % C::ROW_B) / ESZ;
        if (sl * 64 + cel + DW / ESZ > d) cel = 0;   // beyond the row: any chunk inside it
        return vbase + (((b * vlen + kp) * a.Hkv + kvh) * (size_t)d + sl * 64 + cel) * ESZ;
    };
    auto scale_src = [&](size_t kp) -> const float* {
        return a.vs + (kp * a.Hkv + kvh) * (size_t)a.nqg + (sl * 64) / a.qgs;   // no batch offset (:424)
    };
    auto w_src = [&](int i) -> const float* {
        const int o = i * 64 * DW + lane * DW;
        int r = pw * CD_WR + o / 256;
        int qp = qp0 + r / gq;
        if (r >= nc || qp >= a.S) {
            r = 0;
            qp = qp0;
        }
        const size_t row = (b * a.S + qp) * a.Hq + kvh * gq + r % gq;
        return a.w + row * a.wstride + (o % 256) / 4;
    };
    // rolling DMA sources, one tile further per issue (tiles are issued in
    // order); the last tile clamps its keys to the tile range instead
    const char* rp[C::ROWS_LPT];
    const float* sp = nullptr;
    const float* wp[C::W_LPT];
    if (!is_chain) {
#pragma unroll
        for (int i = 0; i < C::ROWS_LPT; i++)
            rp[i] = row_src(i, ks + pw * CD_KPW + (i * 64 * DW + lane * DW) / C::ROW_B);
        if (HYBRID) sp = scale_src(ks + pw * CD_KPW + (lane & (CD_KPW - 1)));
#pragma unroll
        for (int i = 0; i < C::W_LPT; i++) wp[i] = w_src(i);
    }
    const size_t rstep = (size_t)CD_T * krow * ESZ;
    const size_t sstep = (size_t)CD_T * a.Hkv * a.nqg;
    const int kt_len = (int)(kt_end - ks);
    auto issue = [&](int t) {
        const uint32_t slot = ring_lds + (uint32_t)((t % C::D) * C::SLOT);
        const uint32_t rdst = slot + C::ROWS_OFF + pw * CD_KPW * C::ROW_B;
        const uint32_t sdst = slot + C::SC_OFF + pw * CD_KPW * 4;
        if ((t + 1) * CD_T <= kt_len) {
#pragma unroll
            for (int i = 0; i < C::ROWS_LPT; i++) lds_dma<DW>(rp[i], rdst + i * 64 * DW);
            if (HYBRID && lane < CD_KPW) lds_dma<4>(sp, sdst);
        } else {
            const size_t tb = ks + (size_t)t * CD_T;
            const size_t klast = kt_end - 1;
#pragma unroll
            for (int i = 0; i < C::ROWS_LPT; i++) {
                size_t kp = tb + pw * CD_KPW + (i * 64 * DW + lane * DW) / C::ROW_B;
                if (kp > klast) kp = klast;
                lds_dma<DW>(row_src(i, kp), rdst + i * 64 * DW);
            }
            if (HYBRID && lane < CD_KPW) {
                size_t kp = tb + pw * CD_KPW + lane;
                if (kp > klast) kp = klast;
                lds_dma<4>(scale_src(kp), sdst);
            }
        }
#pragma unroll
        for (int i = 0; i < C::W_LPT; i++)
            if (i * 64 * DW + lane * DW < CD_WR * 256)
                lds_dma<DW>(wp[i], slot + C::W_OFF + pw * CD_WR * 256 + i * 64 * DW);
#pragma unroll
        for (int i = 0; i < C::ROWS_LPT; i++) rp[i] += rstep;
        if (HYBRID) sp += sstep;
#pragma unroll
        for (int i = 0; i < C::W_LPT; i++) wp[i] += CD_T;
    };
    auto convert = [&](int t) {
        const unsigned char* slot = ring + (t % C::D) * C::SLOT;
        float* pb = prod + (t & 1) * 64 * CD_PS;
        const int dq = lane & 15, kq = lane >> 4;
        // all LDS reads first, then the products, then the stores
        uint32_t r8[4];
        uint2 r16[4];
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int kl = pw * CD_KPW + kq * 4 + e;
            if (HYBRID) {
                r8[e] = *reinterpret_cast<const uint32_t*>(slot + C::ROWS_OFF + kl * 64 + dq * 4);
                sc[e] = *reinterpret_cast<const float*>(slot + C::SC_OFF + kl * 4);
            } else {
                r16[e] = *reinterpret_cast<const uint2*>(slot + C::ROWS_OFF + kl * 128 + dq * 8);
            }
        }
        float pr[4][4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (HYBRID) {
#pragma unroll
                for (int c = 0; c < 4; c++) pr[e][c] = (float)(int8_t)((r8[e] >> (8 * c)) & 0xFF) * sc[e];
            } else {
                pr[e][0] = h2f((uint16_t)(r16[e].x & 0xFFFF));
                pr[e][1] = h2f((uint16_t)(r16[e].x >> 16));
                pr[e][2] = h2f((uint16_t)(r16[e].y & 0xFFFF));
                pr[e][3] = h2f((uint16_t)(r16[e].y >> 16));
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++)
            *reinterpret_cast<float4*>(pb + (dq * 4 + c) * CD_PS + pw * CD_KPW + kq * 4) =
                make_float4(pr[0][c], pr[1][c], pr[2][c], pr[3][c]);
    };

    // ---- chain row
    const int qp = qp0 + (is_chain ? wv / gq : 0);
    const bool row_ok = is_chain && qp < a.S;
    const size_t row = (b * a.S + (size_t)(row_ok ? qp : 0)) * a.Hq + kvh * gq + (is_chain ? wv % gq : 0);
    size_t rks = 0, rke = 0, rbl = 0;
    int nb = 0, nb_tile = 0;
    if (row_ok) {
        kv_range<HYBRID>(a, (size_t)qp, rks, rke, rbl);
        nb = rke > rks ? (int)((rke - rks + ATT_BLOCK - 1) / ATT_BLOCK) : 0;
        nb_tile = rbl <= kt_end ? nb : min(nb, (int)((kt_end - rks) / ATT_BLOCK));
    }
    const int dim = sl * 64 + lane;
    // the first new row of the hybrid (the decode step's own key), early
    float pf_p = 0.0f, pf_w = 0.0f;
    const bool pf = HYBRID && row_ok && a.cache_len < rke;
    if (pf) {
        pf_w = a.w[row * a.wstride + (a.cache_len - rks)];
        if (dim < d) pf_p = h2f(a.v[((b * a.new_len) * a.Hkv + kvh) * (size_t)d + dim]);
    }
    if (row_ok) chain_corr(a, row, nb, corr_s + wv * nbmax, bsum_s + wv * nbmax);

    if (!is_chain && nst > 0) {
        for (int t = 0; t < C::D - 1; t++)
            if (t < nst) issue(t);
        if (nst >= C::D - 1) wait_dma<C::VM_WAIT>();
        else wait_dma<0>();
        convert(0);
    }
    const float* cw = corr_s + wv * nbmax;
    const float* cb = bsum_s + wv * nbmax;
    float acc = 0.0f, rs = 0.0f;
    for (int t = 0; t < nst; t++) {
        lds_barrier();
        if (!is_chain) {
            if (t + C::D - 1 < nst) issue(t + C::D - 1);
            if (t + 1 < nst) {
                if (t + C::D - 1 < nst) wait_dma<C::VM_WAIT>();
                else wait_dma<0>();
                convert(t + 1);
            }
            continue;
        }
        if (!row_ok) continue;
        const float* pt = prod + (t & 1) * 64 * CD_PS + lane * CD_PS;
        const float* wt = reinterpret_cast<const float*>(ring + (t % C::D) * C::SLOT + C::W_OFF) + wv * CD_T;
        const int b0 = t * (CD_T / ATT_BLOCK);
        const int b1 = min(nb_tile, b0 + CD_T / ATT_BLOCK);
        chain_tile(pt, wt, b0, b1, rks, rbl, cw, cb, acc, rs);
    }
    if (!row_ok) return;
    // blocks reaching past the tiles: tile keys from the last tile (still
    // resident), new rows read directly
    const int tl = nst - 1;
    const size_t tbase = ks + (size_t)(tl > 0 ? tl : 0) * CD_T;
    const float* pt = prod + ((tl > 0 ? tl : 0) & 1) * 64 * CD_PS + lane * CD_PS;
    const float* wt =
        reinterpret_cast<const float*>(ring + ((tl > 0 ? tl : 0) % C::D) * C::SLOT + C::W_OFF) + wv * CD_T;
    chain_tail<HYBRID>(a, b, kvh, dim, row, nb_tile, nb, rks, rbl, kt_end, tbase, pt, wt, pf, pf_p, pf_w, cw, cb,
                       acc, rs);
    if (dim < d) {
        uint16_t* ov = a.o + row * (size_t)d;
        if (!(rs > 0.0f) || dim >= da) ov[dim] = 0;
        else ov[dim] = f2h(acc * (1.0f / rs));
    }
}

// ------------------------------------------------ kernel B, many query rows
// Prefill form of the value chains.  A workgroup owns RW_CH chains -- RW_CH/gq
// consecutive query rows times the gq heads of one kv head -- on one 64-dim
// slice.  Each chain wave runs RW_CPW chains per lane (lane = dimension), so
// one LDS read of a value row feeds RW_CPW FMAs, and the chains of a lane
// interleave instead of waiting on each other's FMA latency.  Weights enter
// the FMA through DPP row_newbcast (a 16-key weight vector replicated per
// 16-lane row), so a step reads no weight from LDS.  The stage waves fetch
// the next tile's value rows into registers a whole step ahead and store the
// reference's fp32 operands (INT8 code * per-key group scale for the cache,
// fp16 -> fp32 for new rows and the FP16 path) as [dim][key] rows, plus the
// chains' weights.  Blocks that are partial or hold a zero weight run key by
// key with the reference's zero skip (kernel_attention.cpp:200-201).
constexpr int RW_T = 64;                          // keys per tile
constexpr int RW_PS = RW_T + 4;                   // floats per dim row (bank skew)
constexpr int RW_CH = 32;                         // chains per workgroup
constexpr int RW_CPW = 4;                         // chains per lane of a chain wave
constexpr int RW_NCW = RW_CH / RW_CPW;            // chain waves
constexpr int RW_NSW = 4;                         // stage waves
constexpr int RW_THREADS = 64 * (RW_NCW + RW_NSW);
constexpr int RW_PROD_B = 2 * 64 * RW_PS * 4;
constexpr int RW_W_B = 2 * RW_CH * RW_T * 4;

template <int K>
__device__ __forceinline__ void rw_step(float (&acc)[RW_CPW], const float (&wv)[RW_CPW], float p) {
#pragma unroll
    for (int c = 0; c < RW_CPW; c++) fmac_row_bcast<K>(acc[c], wv[c], p);
}
template <int... K>
__device__ __forceinline__ void rw_chain16(float (&acc)[RW_CPW], const float* p, const float (&wv)[RW_CPW],
                                           std::integer_sequence<int, K...>) {
    asm volatile("s_nop 1");   // DPP source read after a possible VALU write of wv
    (rw_step<K>(acc, wv, p[K]), ...);
}

// weight k of a 16-lane row, broadcast over the row (DPP row_newbcast:k)
template <int K>
__device__ __forceinline__ float row_bcast(float w) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, w), 0x150 + K, 0xF, 0xF, false));
}
// 16 chain steps of one chain, key k taken only where bit k of the
// wave-uniform mask nz is set
template <int... K>
__device__ __forceinline__ void rw_masked16(float& acc, const float* p, float wv, uint32_t nz,
                                            std::integer_sequence<int, K...>) {
    ((((nz >> K) & 1u) ? (void)(acc = __builtin_fmaf(p[K], row_bcast<K>(wv), acc)) : (void)0), ...);
}

template <bool HYBRID>
__global__ void __launch_bounds__(RW_THREADS) attn_rows_kernel(AttnArgs a_in, int nbmax) {
    const AttnArgs a = resolve(a_in);
    extern __shared__ __align__(16) unsigned char smem[];
    float* prod = reinterpret_cast<float*>(smem);                        // [2][64][RW_PS]
    float* wts = reinterpret_cast<float*>(smem + RW_PROD_B);             // [2][RW_CH][RW_T]
    float* corr_s = reinterpret_cast<float*>(smem + RW_PROD_B + RW_W_B); // [RW_CH][nbmax]
    float* bsum_s = corr_s + (size_t)RW_CH * nbmax;                      // [RW_CH][nbmax]
    const float NEG_INF = -__builtin_inff();

    const int d = a.d, da = (d / 8) * 8, gq = a.gq;
    const int qr = RW_CH / gq;                     // query rows of the workgroup
    const int nsl = (d + 63) / 64;
    size_t g = blockIdx.x;
    const int sl = (int)(g % nsl);
    g /= nsl;
    const int kvh = (int)(g % a.Hkv);
    g /= a.Hkv;
    const int ngrp = (a.S + qr - 1) / qr;
    const int qp0 = (int)(g % ngrp) * qr;
    const size_t b = g / ngrp;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;

    // keys of the group: every row starts at the same key (no sliding
    // window on this path); the last row reaches furthest
    size_t ks, ke_f, bl_f;
    kv_range<HYBRID>(a, (size_t)qp0, ks, ke_f, bl_f);
    const int qlast = min(qp0 + qr, a.S) - 1;
    size_t ks_l, ke_l, bl_l;
    kv_range<HYBRID>(a, (size_t)qlast, ks_l, ke_l, bl_l);
    size_t kneed = ks;
    if (ke_l > ks) {
        kneed = ks + ((ke_l - ks + ATT_BLOCK - 1) / ATT_BLOCK) * ATT_BLOCK;
        if (kneed > bl_l) kneed = bl_l;
    }
    const int nst = (int)((kneed - ks + RW_T - 1) / RW_T);
    const bool is_chain = wv < RW_NCW;

    // ---- stage waves: item (dq, kq) = 4 dims x 4 keys of a tile
    const int pl = (int)threadIdx.x - RW_NCW * 64;
    const int dq = pl & 15, kq = pl >> 4;
    const int dim0 = sl * 64 + dq * 4;
    uint32_t r8[4];
    uint2 r16[4];
    float rsc[4];
    float4 wr[2];
    auto load_raw = [&](int t) {
        const size_t tb = ks + (size_t)t * RW_T;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const size_t kp = tb + kq * 4 + e;
            r8[e] = 0;
            r16[e] = make_uint2(0, 0);
            rsc[e] = 0.0f;
            if (kp >= kneed || dim0 >= da) continue;
            if (HYBRID && kp < a.cache_len) {
                const size_t off = (b * a.cache_len + kp) * a.Hkv + kvh;
                r8[e] = *reinterpret_cast<const uint32_t*>(a.vc + off * d + dim0);
                rsc[e] = a.vs[(kp * a.Hkv + kvh) * a.nqg + dim0 / a.qgs];   // no batch offset (:424)
            } else {
                const size_t vpos = HYBRID ? kp - a.cache_len : kp;
                const size_t vlen = HYBRID ? a.new_len : a.Skv;
                r16[e] = *reinterpret_cast<const uint2*>(a.v + ((b * vlen + vpos) * a.Hkv + kvh) * (size_t)d + dim0);
            }
        }
        // weights of the chains for this tile: 32 rows x 64 keys, 8 per thread
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = pl + 256 * j;
            const int c = i >> 4, j4 = (i & 15) * 4;
            const int qp = qp0 + c / gq;
            wr[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const size_t col = (size_t)t * RW_T + j4;
            if (qp < a.S && col + 4 <= a.wstride) {
                const size_t row = (b * a.S + qp) * a.Hq + kvh * gq + (c % gq);
                wr[j] = *reinterpret_cast<const float4*>(a.w + row * a.wstride + col);
            }
        }
    };
    auto store_tile = [&](int t) {
        const size_t tb = ks + (size_t)t * RW_T;
        float* pb = prod + (t & 1) * 64 * RW_PS;
        float pr[4][4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const size_t kp = tb + kq * 4 + e;
            if (HYBRID && kp < a.cache_len) {
#pragma unroll
                for (int c = 0; c < 4; c++) pr[e][c] = (float)(int8_t)((r8[e] >> (8 * c)) & 0xFF) * rsc[e];
            } else {
                pr[e][0] = h2f((uint16_t)(r16[e].x & 0xFFFF));
                pr[e][1] = h2f((uint16_t)(r16[e].x >> 16));
                pr[e][2] = h2f((uint16_t)(r16[e].y & 0xFFFF));
                pr[e][3] = h2f((uint16_t)(r16[e].y >> 16));
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++)
            *reinterpret_cast<float4*>(pb + (dq * 4 + c) * RW_PS + kq * 4) =
                make_float4(pr[0][c], pr[1][c], pr[2][c], pr[3][c]);
        float* wb = wts + (t & 1) * RW_CH * RW_T;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = pl + 256 * j;
            *reinterpret_cast<float4*>(wb + (i >> 4) * RW_T + (i & 15) * 4) = wr[j];
        }
    };

    // ---- chain waves: chains c0..c0+3 of the workgroup
    const int c0 = wv * RW_CPW;
    size_t crow[RW_CPW];
    size_t crbl[RW_CPW];
    int cnb[RW_CPW];
#pragma unroll
    for (int c = 0; c < RW_CPW; c++) {
        const int ch = c0 + c;
        const int qp = qp0 + ch / gq;
        crow[c] = 0;
        crbl[c] = 0;
        cnb[c] = 0;
        if (is_chain && qp < a.S) {
            size_t rks, rke, rbl;
            kv_range<HYBRID>(a, (size_t)qp, rks, rke, rbl);
            crow[c] = (b * a.S + qp) * a.Hq + kvh * gq + ch % gq;
            crbl[c] = rbl;
            cnb[c] = rke > rks ? (int)((rke - rks + ATT_BLOCK - 1) / ATT_BLOCK) : 0;
            chain_corr(a, crow[c], cnb[c], corr_s + (size_t)ch * nbmax, bsum_s + (size_t)ch * nbmax);
        }
    }
    if (!is_chain && nst > 0) {
        load_raw(0);
        store_tile(0);
        if (nst > 1) load_raw(1);
    }

    float acc[RW_CPW], rs[RW_CPW];
#pragma unroll
    for (int c = 0; c < RW_CPW; c++) {
        acc[c] = 0.0f;
        rs[c] = 0.0f;
    }
    const int lr = lane & 15;
    for (int t = 0; t < nst; t++) {
        __syncthreads();
        if (!is_chain) {
            // buffer (t+1)&1 last held tile t-1, finished before this barrier
            if (t + 1 < nst) {
                store_tile(t + 1);
                if (t + 2 < nst) load_raw(t + 2);
            }
            continue;
        }
        const float* pt = prod + (t & 1) * 64 * RW_PS + lane * RW_PS;
        const float* wt = wts + (t & 1) * RW_CH * RW_T + (size_t)c0 * RW_T;
#pragma unroll
        for (int h = 0; h < RW_T / ATT_BLOCK; h++) {
            const int blk = t * (RW_T / ATT_BLOCK) + h;
            const int jo = h * ATT_BLOCK;
            const size_t bs0 = ks + (size_t)blk * ATT_BLOCK;
            bool all_fast = true;
            float bse[RW_CPW];
            int bsz[RW_CPW];
#pragma unroll
            for (int c = 0; c < RW_CPW; c++) {
                bse[c] = 0.0f;
                bsz[c] = 0;
                if (blk < cnb[c]) {
                    const float cr = corr_s[(size_t)(c0 + c) * nbmax + blk];
                    bse[c] = bsum_s[(size_t)(c0 + c) * nbmax + blk];
                    if (cr != NEG_INF) {
                        acc[c] = acc[c] * cr;
                        rs[c] = rs[c] * cr;
                    }
                    bsz[c] = (int)((bs0 + ATT_BLOCK < crbl[c] ? bs0 + ATT_BLOCK : crbl[c]) - bs0);
                    if (bsz[c] != ATT_BLOCK || __builtin_signbit(bse[c])) all_fast = false;
                } else {
                    all_fast = false;
                }
            }
            if (blk >= cnb[0] && blk >= cnb[1] && blk >= cnb[2] && blk >= cnb[3]) continue;
            float pv[ATT_BLOCK];
#pragma unroll
            for (int q = 0; q < ATT_BLOCK / 4; q++) {
                const float4 v = *reinterpret_cast<const float4*>(pt + jo + 4 * q);
                pv[4 * q] = v.x;
                pv[4 * q + 1] = v.y;
                pv[4 * q + 2] = v.z;
                pv[4 * q + 3] = v.w;
            }
            if (all_fast) {
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    float wvv[RW_CPW];
#pragma unroll
                    for (int c = 0; c < RW_CPW; c++) wvv[c] = wt[c * RW_T + jo + 16 * hh + lr];
                    rw_chain16(acc, pv + 16 * hh, wvv, std::make_integer_sequence<int, 16>{});
                }
            } else {
#pragma unroll
                for (int c = 0; c < RW_CPW; c++) {
                    if (blk >= cnb[c]) continue;
                    // keys of a partial block's end, and zero weights, are
                    // skipped: an FMA with a zero weight could turn an
                    // accumulator of -0 into +0
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int lim = bsz[c] - 16 * hh;
                        if (lim <= 0) break;
                        const float wvv = wt[c * RW_T + jo + 16 * hh + lr];
                        uint32_t nz = (uint32_t)__ballot(wvv != 0.0f) & 0xFFFFu;   // lanes 0-15: keys
                        if (lim < 16) nz &= (1u << lim) - 1u;
                        rw_masked16(acc[c], pv + 16 * hh, wvv, nz, std::make_integer_sequence<int, 16>{});
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < RW_CPW; c++)
                if (blk < cnb[c]) rs[c] = rs[c] + __builtin_fabsf(bse[c]);
        }
    }
    if (!is_chain) return;
    const int dim = sl * 64 + lane;
    if (dim >= d) return;
#pragma unroll
    for (int c = 0; c < RW_CPW; c++) {
        if (qp0 + (c0 + c) / gq >= a.S) continue;
        uint16_t* ov = a.o + crow[c] * (size_t)d;
        if (!(rs[c] > 0.0f) || dim >= da) ov[dim] = 0;
        else ov[dim] = f2h(acc[c] * (1.0f / rs[c]));
    }
}

static size_t rows_smem(int nbmax) { return (size_t)RW_PROD_B + RW_W_B + 2 * (size_t)RW_CH * nbmax * sizeof(float); }

// ------------------------------------------------ per-(device, stream) scratch
static int attn_scratch(void* stream, size_t bytes, void** out) {
    return stream_scratch(SCR_ATTN, stream, bytes, false, out);
}

template <bool HYBRID>
static int launch_attention(AttnArgs a, void* stream) {
    // largest key range over the launch (query 0 .. S-1)
    size_t maxr = 0;
    for (int qp : {0, a.S - 1}) {
        const size_t aq = a.pos_off + qp;
        size_t s0 = 0, e = a.Skv;
        if (!HYBRID) {
            if (a.window > 0 && a.window < a.Skv) {
                if (aq > a.window) s0 = aq - a.window;
                if (a.causal && aq + 1 < e) e = aq + 1;
            } else if (a.causal && aq + 1 < e) {
                e = aq + 1;
            }
        } else if (a.causal && aq + 1 < e) {
            e = aq + 1;
        }
        if (e > s0 && e - s0 > maxr) maxr = e - s0;
    }
    if (!HYBRID && a.window > 0 && a.window < a.Skv) maxr = a.Skv;  // conservative
    if (a.dyn) maxr = a.max_cache + a.new_len;
    const size_t rows = (size_t)a.B * a.S * a.Hq;
    const int nb = (int)((maxr + ATT_BLOCK - 1) / ATT_BLOCK);
    CH_REQUIRE(nb <= 1024, "attention: key range above 32768 is not supported");
    // (+64: the decode chain kernel reads one block past a row's last)
    a.wstride = ((maxr + 63) & ~(size_t)63) + 64;
    a.nbstride = nb > 0 ? nb : 1;
    const size_t wbytes = rows * a.wstride * sizeof(float);
    const size_t bbytes = rows * (size_t)a.nbstride * sizeof(float);
    void* scratch = nullptr;
    int rc = attn_scratch(stream, wbytes + 2 * bbytes + 256, &scratch);
    if (rc) return rc;
    a.w = static_cast<float*>(scratch);
    a.bmax = reinterpret_cast<float*>(static_cast<char*>(scratch) + wbytes);
    a.bsum = a.bmax + rows * a.nbstride;
    const size_t chunks = (maxr + 63) / 64;
    const bool windowed = !HYBRID && a.window > 0 && a.window < a.Skv;
    // prefill scores: several query rows per wave (16-dim DPP groups, one
    // scale per 16 dims, 16-byte key rows)
    const bool k16 = HYBRID ? ((uintptr_t)a.kc % 16 == 0 && (uintptr_t)a.ks % 4 == 0 && a.qgs % 16 == 0) : true;
    const bool rows_ok = chunks > 0 && !windowed && (a.d == 64 || a.d == 128) && a.gq <= SQ_NQ &&
                         SQ_NQ % a.gq == 0 && k16 && (uintptr_t)a.k % 16 == 0;
    CH_REQUIRE(!a.prep.q_raw || (rows_ok && (size_t)a.B * a.S <= 2 && (a.gq == 1 || a.gq == 2)),
               "decode attention with fused head preparation: needs head_dim 64 or 128, 1 or 2 query heads "
               "per KV head and 16-byte aligned rows");
    if (rows_ok && (size_t)a.B * a.S > 2) {
        const int qr = SQ_NQ / a.gq;
        dim3 ga((unsigned)((chunks + 3) / 4), (unsigned)((size_t)a.B * ((a.S + qr - 1) / qr) * a.Hkv));
        if (a.d == 64)
            hipLaunchKernelGGL((attn_scores_rows_kernel<HYBRID, 64, SQ_NQ, 4>), ga, dim3(256), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL((attn_scores_rows_kernel<HYBRID, 128, SQ_NQ, 4>), ga, dim3(256), 0, as_stream(stream), a);
        rc = check_launch("attention scores (rows)");
        if (rc) return rc;
    } else if (rows_ok && (a.gq == 1 || a.gq == 2)) {
        // decode: one query row, its gq heads per wave, one wave per 64 keys
        // (with the fused head preparation, one more workgroup per kv head
        // appends the step's key and value)
        // workgroups of kv head h on XCD h % 8, where the chain kernel's are;
        // two query heads per kv head split over two workgroups per chunk
        // (consecutive, so on one XCD: the second reads the key rows from
        // its L2), which halves each wave's dot and weight work
        a.hsplit = a.gq;
        a.xcd_chunks = (int)(chunks + (a.prep.q_raw ? 1 : 0)) * a.hsplit;
        a.xcd_rest = a.B * a.S;                          // row groups of one row, one head
        const size_t nwg = 8 * (size_t)((a.Hkv + 7) / 8) * a.xcd_chunks * a.xcd_rest;
        CH_REQUIRE(nwg < (1u << 31), "attention: decode key range too long");
        dim3 ga((unsigned)nwg);
        auto go = [&](auto kern) { hipLaunchKernelGGL(kern, ga, dim3(64), 0, as_stream(stream), a); };
        if (a.d == 64) go(attn_scores_rows_kernel<HYBRID, 64, 1, 1>);
        else go(attn_scores_rows_kernel<HYBRID, 128, 1, 1>);
        rc = check_launch("attention scores (decode)");
        if (rc) return rc;
    } else if (chunks > 0) {
        dim3 ga((unsigned)((chunks + 3) / 4), (unsigned)((size_t)a.B * a.S * a.Hkv));
        if (a.d <= 64)
            hipLaunchKernelGGL((attn_scores_kernel<HYBRID, 64>), ga, dim3(256), 0, as_stream(stream), a);
        else if (a.d <= 128)
            hipLaunchKernelGGL((attn_scores_kernel<HYBRID, 128>), ga, dim3(256), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL((attn_scores_kernel<HYBRID, 256>), ga, dim3(256), 0, as_stream(stream), a);
        rc = check_launch("attention scores");
        if (rc) return rc;
    }
    // chain kernel: rows sharing a kv head are grouped so that their value
    // tiles are staged once; a sliding window gives every row its own start
    int qpg = windowed ? 1 : ATT_MAX_GQ / a.gq;
    if (qpg > a.S) qpg = a.S;
    if (qpg < 1) qpg = 1;
    const int nbmax = a.nbstride;
    const size_t nsl = (size_t)(a.d + 63) / 64;
    if (HYBRID && a.vsh) return launch_chain_stream(a, nbmax, stream);   // decode with value product tiles
    {
        // prefill: many query rows per workgroup, several chains per lane
        const bool aligned = (HYBRID ? (uintptr_t)a.vc % 4 == 0 && (uintptr_t)a.vs % 4 == 0 : true) &&
                             (uintptr_t)a.v % 8 == 0;
        if (!windowed && (size_t)a.B * a.S > 2 && a.gq <= ATT_MAX_GQ && RW_CH % a.gq == 0 && a.d % 4 == 0 &&
            aligned && rows_smem(nbmax) <= 160 * 1024) {
            static hipError_t attr[2] = {
                hipFuncSetAttribute((const void*)attn_rows_kernel<false>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024),
                hipFuncSetAttribute((const void*)attn_rows_kernel<true>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)};
            if (attr[HYBRID] == hipSuccess) {
                const int qr = RW_CH / a.gq;
                const size_t groups = (size_t)a.B * (((size_t)a.S + qr - 1) / qr) * a.Hkv * nsl;
                hipLaunchKernelGGL(attn_rows_kernel<HYBRID>, dim3((unsigned)groups), dim3(RW_THREADS),
                                   rows_smem(nbmax), as_stream(stream), a, nbmax);
                return check_launch("attention values (rows)");
            }
            (void)hipGetLastError();  // clear the sticky attribute error before the forms below
        }
    }
    // LDS-DMA form: value rows in 16- or 4-byte chunks, one scale group per
    // 64-dim slice; otherwise the register-staged form
    const uintptr_t vp = HYBRID ? (uintptr_t)a.vc : (uintptr_t)a.v;
    const bool g64 = !HYBRID || (a.qgs % 64 == 0);
    const bool w16 = g64 && (HYBRID ? a.d % 16 == 0 : a.d % 8 == 0) && vp % 16 == 0 &&
                     (!HYBRID || (uintptr_t)a.vs % 4 == 0);
    const bool w4 = g64 && a.d % 4 == 0 && vp % 4 == 0 && (!HYBRID || (uintptr_t)a.vs % 4 == 0);
    auto dma_smem = [&](int q) -> size_t {
        const size_t slot = w16 ? CdCfg<HYBRID, 16>::SLOT : CdCfg<HYBRID, 4>::SLOT;
        const size_t depth = w16 ? CdCfg<HYBRID, 16>::D : CdCfg<HYBRID, 4>::D;
        return depth * slot + (2 * 64 * CD_PS + 2 * (size_t)q * a.gq * nbmax) * sizeof(float);
    };
    if (w16 || w4) {
        while (qpg > 1 && dma_smem(qpg) > 160 * 1024) qpg = (qpg + 1) / 2;
        if (dma_smem(qpg) <= 160 * 1024) {
            static bool attr_set[2][2] = {{false, false}, {false, false}};
            const size_t smem = dma_smem(qpg);
            const size_t ngrp = ((size_t)a.S + qpg - 1) / qpg;
            const size_t groups = (size_t)a.B * ngrp * a.Hkv * nsl;
            const dim3 blk(64 * (qpg * a.gq + CD_NP));
            if (w16) {
                if (!attr_set[HYBRID][1]) {
                    CH_HIP(hipFuncSetAttribute((const void*)attn_chain_dma_kernel<HYBRID, 16>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
                    attr_set[HYBRID][1] = true;
                }
                hipLaunchKernelGGL((attn_chain_dma_kernel<HYBRID, 16>), dim3((unsigned)groups), blk, smem,
                                   as_stream(stream), a, qpg, nbmax);
            } else {
                if (!attr_set[HYBRID][0]) {
                    CH_HIP(hipFuncSetAttribute((const void*)attn_chain_dma_kernel<HYBRID, 4>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
                    attr_set[HYBRID][0] = true;
                }
                hipLaunchKernelGGL((attn_chain_dma_kernel<HYBRID, 4>), dim3((unsigned)groups), blk, smem,
                                   as_stream(stream), a, qpg, nbmax);
            }
            return check_launch("attention values");
        }
        qpg = 1;
    }
    const int nc = qpg * a.gq;
    const uintptr_t hp = (uintptr_t)a.v;
    const int vec_ok = (a.d % 4 == 0) && ((HYBRID ? (uintptr_t)a.vc : 0) % 4 == 0) && (hp % 8 == 0);
    const size_t smem = (2 * 64 * CH_PS + 2 * (size_t)nc * CH_T + 2 * (size_t)nc * nbmax) * sizeof(float);
    CH_REQUIRE(smem <= 160 * 1024, "attention: key range too long for the chain kernel");
    static bool attr_set[2] = {false, false};
    if (!attr_set[HYBRID]) {
        CH_HIP(hipFuncSetAttribute((const void*)attn_chain_kernel<HYBRID>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set[HYBRID] = true;
    }
    const size_t ngrp = ((size_t)a.S + qpg - 1) / qpg;
    const size_t groups = (size_t)a.B * ngrp * a.Hkv * nsl;
    hipLaunchKernelGGL(attn_chain_kernel<HYBRID>, dim3((unsigned)groups), dim3(64 * (nc + CH_NP)), smem,
                       as_stream(stream), a, qpg, nbmax, vec_ok);
    return check_launch("attention values");
}

// Hybrid attention of one decode step whose cache length and position are
// read from the device step state (see AttnArgs::dyn).
int attention_hybrid_decode(const uint16_t* q, const int8_t* kc, const int8_t* vc, const float* ks,
                            const float* vs, const uint16_t* k_new, const uint16_t* v_new,
                            uint16_t* o, int Hq, int Hkv, int d, float scale, const uint32_t* state,
                            size_t max_cache, const float* v_shadow, size_t shadow_tiles, void* stream) {
    AttnArgs a{};
    a.q = q; a.k = k_new; a.v = v_new; a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs; a.o = o;
    a.B = 1; a.S = 1; a.Hq = Hq; a.Hkv = Hkv; a.gq = Hq / Hkv; a.d = d;
    a.new_len = 1; a.cache_len = max_cache; a.Skv = max_cache + 1; a.pos_off = max_cache;
    a.causal = 1; a.scale = scale; a.qgs = 128; a.nqg = (d + 127) / 128;
    a.dyn = state; a.max_cache = max_cache;
    a.vsh = v_shadow; a.sh_ntile = shadow_tiles;
    CH_REQUIRE(!v_shadow || shadow_tiles * CD_T >= max_cache, "decode attention: product tiles too short");
    return launch_attention<true>(a, stream);
}

int attention_hybrid_decode_prep(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                 const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                 const uint16_t* cos_t, const uint16_t* sin_t, uint32_t table_pos,
                                 int8_t* kc, int8_t* vc, float* ks, float* vs, float* v_shadow,
                                 uint16_t* o, int Hq, int Hkv, int d, float scale, const uint32_t* state,
                                 size_t max_cache, size_t shadow_tiles, void* stream) {
    AttnArgs a{};
    a.q = q_raw; a.k = k_raw; a.v = v_raw; a.kc = kc; a.vc = vc; a.ks = ks; a.vs = vs; a.o = o;
    a.B = 1; a.S = 1; a.Hq = Hq; a.Hkv = Hkv; a.gq = Hq / Hkv; a.d = d;
    a.new_len = 1; a.cache_len = max_cache; a.Skv = max_cache + 1; a.pos_off = max_cache;
    a.causal = 1; a.scale = scale; a.qgs = 128; a.nqg = (d + 127) / 128;
    a.dyn = state; a.max_cache = max_cache;
    a.vsh = v_shadow; a.sh_ntile = shadow_tiles;
    a.prep.q_raw = q_raw; a.prep.k_raw = k_raw; a.prep.v_raw = v_raw;
    a.prep.q_norm = q_norm; a.prep.k_norm = k_norm; a.prep.cos_t = cos_t; a.prep.sin_t = sin_t;
    a.prep.eps = eps; a.prep.table_pos = table_pos;
    a.prep.kc = kc; a.prep.vc = vc; a.prep.ks = ks; a.prep.vs = vs; a.prep.vsh = v_shadow;
    CH_REQUIRE(!v_shadow || shadow_tiles * CD_T >= max_cache, "decode attention: product tiles too short");
    return launch_attention<true>(a, stream);
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
    CH_REQUIRE(num_q_heads / num_kv_heads <= (size_t)ATT_MAX_GQ,
               "attention_f16: more than 8 query heads per KV head is not supported");
    CH_REQUIRE(head_dim <= (size_t)ATT_MAX_D, "attention_f16: head_dim > 256 not supported");
    CH_REQUIRE(head_dim % 4 == 0, "attention_f16: head_dim must be a multiple of 4");
    CH_REQUIRE(batch * seq_len * num_kv_heads < (1u << 31), "attention_f16: too many rows");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    AttnArgs a{};
    a.q = q; a.k = k; a.v = v; a.o = o; a.mask = mask;
    a.B = (int)batch; a.S = (int)seq_len; a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads;
    a.gq = (int)(num_q_heads / num_kv_heads);
    a.d = (int)head_dim; a.Skv = kv_seq_len; a.pos_off = position_offset; a.window = window_size;
    a.causal = is_causal ? 1 : 0; a.scale = scale; a.qgs = 1; a.nqg = 1;
    return launch_attention<false>(a, stream);
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
    CH_REQUIRE(num_q_heads / num_kv_heads <= (size_t)ATT_MAX_GQ,
               "attention_hybrid: more than 8 query heads per KV head is not supported");
    CH_REQUIRE(head_dim <= (size_t)ATT_MAX_D && head_dim % 8 == 0,
               "attention_hybrid: head_dim must be a multiple of 8 and <= 256");
    CH_REQUIRE(quant_group_size > 0, "attention_hybrid: quant_group_size must be > 0");
    CH_REQUIRE(batch * seq_len * num_kv_heads < (1u << 31), "attention_hybrid: too many rows");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)head_dim);
    AttnArgs a{};
    a.q = q; a.k = k_new; a.v = v_new; a.kc = k_cached; a.vc = v_cached; a.ks = k_scales;
    a.vs = v_scales; a.o = o;
    a.B = (int)batch; a.S = (int)seq_len; a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads;
    a.gq = (int)(num_q_heads / num_kv_heads);
    a.d = (int)head_dim; a.Skv = cache_len + new_len; a.cache_len = cache_len; a.new_len = new_len;
    a.pos_off = position_offset; a.causal = is_causal ? 1 : 0; a.scale = scale;
    a.qgs = (int)quant_group_size;
    a.nqg = (int)((head_dim + quant_group_size - 1) / quant_group_size);
    return launch_attention<true>(a, stream);
}

}  // extern "C"
