// gemv.hip -- grouped INT8 / packed-INT4 matmul for small M (decode GEMV).
//
// Weights are streamed as a flat run of 16-byte chunks: consecutive weight
// rows ([rows][K] int8, or [rows][K/2] packed INT4) are one contiguous run,
// so the loads are fully coalesced whatever K is.  The main kernel
// (gemv_wave_kernel) gives each wave its own tiles of whole rows and needs
// no workgroup barrier after the prologue; the block-tiled kernel
// (gemv_grouped_kernel) serves rows longer than a wave tile.  Each chunk is
// dotted with the int8 activation codes held in LDS (v_dot4_i32_i8); the
// lanes that share one quantization group are summed exactly in int32 with
// cross-lane shuffles and the group sum goes to LDS.  One lane per output
// then runs the reference epilogue (kernel_gemm.cpp:311-324):
//     r = fma((float)acc_g, (float)B_scale[n][g], r)   for g = 0..G-1
//     C = fp16(r * A_scale[m])
// With an FP16 activation input the per-row quantization of
// graph_ops_nn.cpp:35-66 runs in the workgroup prologue (every workgroup
// recomputes it from L2; it is a K-element pass against rows*K weight bytes).
#include "gemv_device.h"

namespace cactus_hip {

struct GemvArgs {
    const uint16_t* A16;    // fp16 activations [M][K]      (F16ACT)
    const int8_t* A8;       // int8 codes [M][K]             (!F16ACT)
    const float* As;        // row scales [M]                (!F16ACT)
    const uint8_t* B;       // weights, int8 [N][K] or packed int4 [N][K/2]
    const uint16_t* Bs;     // fp16 group scales [N][G]
    uint16_t* C;            // fp16 out [M][N]
    int M, K, N, gs, rows, tiles;
    size_t sA, sB, sBs, sC; // batch strides: elements of A/Bs/C, bytes of B
};


// Streaming grouped GEMV for M <= 4 activation rows.
//
// Grid (blocks_per_problem, batch).  A workgroup owns `tiles` consecutive
// row tiles of one problem; a tile is `rows` weight rows = rows*cpr 16-byte
// chunks, at most CH per thread.  The loads of tile t+1 are in flight while
// tile t is dotted, and the activation prologue runs while tile 0 loads.
// Group sums of a tile go to one of two LDS buffers; after a barrier the
// tile's epilogue (one thread per output) runs the reference fma chain.
// the reference epilogue of one output, r = fma((float)acc_g, Bs_g, r) over
// ascending groups (kernel_gemm.cpp:311-324), from the group sums and
// scales in LDS: the reads of EPB groups are issued together, so the chain
// waits for LDS once per EPB steps instead of once per step (8: the
// headline kernel stays at 64 VGPRs, 8 waves per SIMD)
template <int EPB = 8>
__device__ __forceinline__ float group_epilogue(const int32_t* ag, const uint16_t* sg, int G) {
    float rs = 0.0f;
    int g = 0;
    for (; g + EPB <= G; g += EPB) {
        int av[EPB];
        uint16_t sv[EPB];
#pragma unroll
        for (int j = 0; j < EPB; j++) {
            av[j] = ag[g + j];
            sv[j] = sg[g + j];
        }
#pragma unroll
        for (int j = 0; j < EPB; j++) rs = __builtin_fmaf((float)av[j], h2f(sv[j]), rs);
    }
    for (; g < G; g++) rs = __builtin_fmaf((float)ag[g], h2f(sg[g]), rs);
    return rs;
}

// group_epilogue for G % 4 == 0 over 16-byte aligned rows of sums and
// 8-byte aligned rows of scales: four groups per pair of LDS reads
__device__ __forceinline__ float group_epilogue_v4(const int32_t* ag, const uint16_t* sg, int G) {
    float rs = 0.0f;
#pragma unroll 4
    for (int g = 0; g < G; g += 4) {
        const i32x4 a4 = *reinterpret_cast<const i32x4*>(ag + g);
        const uint2 s4 = *reinterpret_cast<const uint2*>(sg + g);
        rs = __builtin_fmaf((float)a4.x, h2f((uint16_t)(s4.x & 0xFFFFu)), rs);
        rs = __builtin_fmaf((float)a4.y, h2f((uint16_t)(s4.x >> 16)), rs);
        rs = __builtin_fmaf((float)a4.z, h2f((uint16_t)(s4.y & 0xFFFFu)), rs);
        rs = __builtin_fmaf((float)a4.w, h2f((uint16_t)(s4.y >> 16)), rs);
    }
    return rs;
}

// The same chain over group sums and scales that the lanes producing them
// already converted to fp32 ((float)acc and the fp16 scale are exact): the
// chain lane only reads and FMAs, eight groups per pair of 16-byte reads of
// each row (rows 16-byte aligned: their stride is a multiple of 4 floats).
__device__ __forceinline__ float group_epilogue_f(const float* ag, const float* sg, int G) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    float rs = 0.0f;
    int g = 0;
#pragma unroll 2
    for (; g + 8 <= G; g += 8) {
        const f4v a0 = *reinterpret_cast<const f4v*>(ag + g), a1 = *reinterpret_cast<const f4v*>(ag + g + 4);
        const f4v s0 = *reinterpret_cast<const f4v*>(sg + g), s1 = *reinterpret_cast<const f4v*>(sg + g + 4);
        rs = __builtin_fmaf(a0.x, s0.x, rs);
        rs = __builtin_fmaf(a0.y, s0.y, rs);
        rs = __builtin_fmaf(a0.z, s0.z, rs);
        rs = __builtin_fmaf(a0.w, s0.w, rs);
        rs = __builtin_fmaf(a1.x, s1.x, rs);
        rs = __builtin_fmaf(a1.y, s1.y, rs);
        rs = __builtin_fmaf(a1.z, s1.z, rs);
        rs = __builtin_fmaf(a1.w, s1.w, rs);
    }
    for (; g < G; g++) rs = __builtin_fmaf(ag[g], sg[g], rs);
    return rs;
}

template <int MR, bool F16ACT, bool INT4, int CH>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_grouped_kernel(GemvArgs a, int m0) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = a.K, gs = a.gs, G = K / gs;
    const int rows = a.rows;
    const size_t bi = blockIdx.y;
    const int mr = min(MR, a.M - m0);
    const int tid = threadIdx.x;
    const int tile0 = blockIdx.x * a.tiles;
    const int ntiles_all = (a.N + rows - 1) / rows;
    const int tile_end = min(tile0 + a.tiles, ntiles_all);
    if (tile0 >= tile_end) return;

    int8_t* actq = reinterpret_cast<int8_t*>(smem);                           // MR*K
    int32_t* acc = reinterpret_cast<int32_t*>(smem + ((MR * K + 15) & ~15));  // 2*MR*rows*G
    uint16_t* scl = reinterpret_cast<uint16_t*>(acc + 2 * MR * rows * G);     // 2*rows*G
    float* rsc = reinterpret_cast<float*>(scl + 2 * rows * G);                // MR
    float* red = rsc + MR;                                                    // 4

    const int cpr = INT4 ? K / 32 : K / 16;       // 16-byte chunks per row
    const int P = INT4 ? gs / 32 : gs / 16;       // chunks per group (power of 2)
    const size_t row_bytes = INT4 ? (size_t)K / 2 : (size_t)K;
    const uint8_t* Bbase = a.B + bi * a.sB;
    const uint16_t* Bsbase = a.Bs + bi * a.sBs;

    // per-thread chunk coordinates inside a full tile (the same for every tile)
    int crow[CH], ccol[CH];
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + i * GEMV_THREADS;
        crow[i] = c / cpr;
        ccol[i] = c - crow[i] * cpr;
    }
    auto load_tile = [&](int t, i32x4 (&w)[CH]) {
        const int n0 = t * rows;
        const int total = min(rows, a.N - n0) * cpr;
        const uint8_t* Bw = Bbase + (size_t)n0 * row_bytes;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            w[i] = (i32x4){0, 0, 0, 0};
            if (tid + i * GEMV_THREADS < total)
                w[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(
                    Bw + (size_t)crow[i] * row_bytes + (size_t)ccol[i] * 16));
        }
    };

    i32x4 wcur[CH], wnext[CH];
    load_tile(tile0, wcur);
    for (int i = tid; i < min(rows, a.N - tile0 * rows) * G; i += GEMV_THREADS)
        scl[i] = Bsbase[(size_t)tile0 * rows * G + i];

    // activation codes (the per-row quantization of the matmul node)
    const int body = (K / 8) * 8;
    for (int m = 0; m < mr; m++) {
        if (F16ACT) {
            const uint16_t* x = a.A16 + bi * a.sA + (size_t)(m0 + m) * K;
            const float mx = block_max_abs_f16(x, K, red);
            const float s = row_scale_from_max(mx);
            const float inv = 1.0f / s;
            if constexpr (INT4) {
                for (int r = tid; r < K / 8; r += GEMV_THREADS) {
                    uint32_t w2[2] = {0, 0};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        w2[e >> 2] |= (uint32_t)(uint8_t)quant_code(h2f(x[8 * r + e]), inv, 8 * r + e >= body)
                                      << (8 * (e & 3));
                    nib_store8(actq + m * K, K, r, nib_pack8(w2[0], w2[1]));
                }
            } else {
                for (int i = tid; i < K; i += GEMV_THREADS) actq[m * K + i] = quant_code(h2f(x[i]), inv, i >= body);
            }
            if (tid == 0) rsc[m] = s;
        } else {
            const int8_t* x = a.A8 + bi * a.sA + (size_t)(m0 + m) * K;
            if constexpr (INT4) {
                for (int r = tid; r < K / 8; r += GEMV_THREADS) {
                    uint32_t w2[2] = {0, 0};   // byte loads: the codes carry no alignment promise
#pragma unroll
                    for (int e = 0; e < 8; e++) w2[e >> 2] |= (uint32_t)(uint8_t)x[8 * r + e] << (8 * (e & 3));
                    nib_store8(actq + m * K, K, r, nib_pack8(w2[0], w2[1]));
                }
            } else {
                for (int i = tid; i < K; i += GEMV_THREADS) actq[m * K + i] = x[i];
            }
            if (tid == 0) rsc[m] = a.As[bi * (a.sA / K) + m0 + m];
        }
    }
    __syncthreads();

    // One barrier per tile: the dot products of tile t fill accumulator
    // buffer t%2; after the barrier the epilogue of tile t reads it while
    // other waves already dot tile t+1 into the other buffer.
    for (int t = tile0; t < tile_end; t++) {
        const int buf = (t - tile0) & 1;
        const int n0 = t * rows;
        const int nr = min(rows, a.N - n0);
        const int total = nr * cpr;
        int32_t* accb = acc + buf * MR * rows * G;
        uint16_t* sclb = scl + buf * rows * G;
        if (t + 1 < tile_end) load_tile(t + 1, wnext);
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const bool valid = tid + i * GEMV_THREADS < total;
            int dot[MR];
#pragma unroll
            for (int m = 0; m < MR; m++) {
                dot[m] = (valid && m < mr) ? chunk_dot<INT4>(actq + m * K, ccol[i], wcur[i], K / 2) : 0;
                dot[m] = group_lane_sum(dot[m], P);
            }
            if (valid && ((tid + i * GEMV_THREADS) & (P - 1)) == 0) {
                const int g = (ccol[i] * (INT4 ? 32 : 16)) / gs;
#pragma unroll
                for (int m = 0; m < MR; m++)
                    if (m < mr) accb[(m * rows + crow[i]) * G + g] = dot[m];
            }
        }
        __syncthreads();
        // scales of tile t+1 into the other buffer: its last reader, the
        // epilogue of tile t-1, finished before the barrier above
        if (t + 1 < tile_end) {
            const int n1 = n0 + rows;
            uint16_t* scln = scl + (buf ^ 1) * rows * G;
            for (int i = tid; i < min(rows, a.N - n1) * G; i += GEMV_THREADS)
                scln[i] = Bsbase[(size_t)n1 * G + i];
        }

        // reference epilogue, one thread per output of this tile
        for (int o = tid; o < mr * nr; o += GEMV_THREADS) {
            const int m = o / nr, r = o % nr;
            const int32_t* ag = accb + (m * rows + r) * G;
            const uint16_t* sg = sclb + r * G;
            const float rs = group_epilogue(ag, sg, G);
            a.C[bi * a.sC + (size_t)(m0 + m) * a.N + n0 + r] = f2h(rs * rsc[m]);
        }
#pragma unroll
        for (int i = 0; i < CH; i++) wcur[i] = wnext[i];
    }
}

static size_t gemv_smem(int MR, int K, int rows, int G) {
    size_t s = (size_t)((MR * K + 15) & ~15);
    s += (size_t)2 * MR * rows * G * 4;
    s += (size_t)2 * rows * G * 2;
    s += (size_t)MR * 4 + 16;
    return (s + 15) & ~(size_t)15;
}

// Wave-streaming grouped GEMV for M <= 4 activation rows.
//
// A wave tile is `rows` consecutive weight rows, a contiguous run of
// rows*cpr 16-byte chunks that one wave loads as CH coalesced 1 KB slots
// (chunk f = slot*64 + lane).  The four waves of a workgroup share only the
// activation codes, quantized once in the prologue; after that each wave
// streams its own tiles (t0+wave, t0+wave+4, ...) with no workgroup barrier:
// dot products and exact group sums, group sums and the tile's fp16 group
// scales into the wave's own LDS slice, the loads of its next tile, then the
// reference epilogue (kernel_gemm.cpp:311-324) by one lane per output while
// those loads are in flight.
//
// FE (INT4 with 32-wide groups: one 16-byte chunk per group): the lane that
// owns a chunk also owns its group, so it stores the group sum and the
// group scale already converted to fp32, in rows padded by 4 floats (the
// epilogue lanes read distinct banks); the K=3072 epilogue of 96 groups per
// output then costs one FMA per group instead of two converts and an FMA.
template <int MR, bool F16ACT, bool INT4, int CH, bool FE = false>
__global__ void __launch_bounds__(GEMV_THREADS) gemv_wave_kernel(GemvArgs a, int m0) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = a.K, gs = a.gs, G = K / gs;
    const int rows = a.rows;
    const size_t bi = blockIdx.y;
    const int mr = min(MR, a.M - m0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ntiles_all = (a.N + rows - 1) / rows;
    const int t0 = blockIdx.x * a.tiles;
    const int t1 = min(t0 + a.tiles, ntiles_all);
    if (t0 >= t1) return;  // uniform over the workgroup

    const int cpr = INT4 ? K / 32 : K / 16;  // 16-byte chunks per row
    const int P = INT4 ? gs / 32 : gs / 16;  // chunks per group (power of 2, <= 64)
    const size_t row_bytes = INT4 ? (size_t)K / 2 : (size_t)K;
    // row stride of the group sums and scales (FE: whole 16-byte vectors,
    // plus 16 bytes so that consecutive rows start four banks apart)
    const int Gs = FE ? ((G + 3) & ~3) + 4 : G;
    const int acc_words = MR * rows * Gs;
    const int wave_bytes = ((acc_words * 4 + 15) & ~15) + ((rows * Gs * (FE ? 4 : 2) + 15) & ~15);

    int8_t* actq = reinterpret_cast<int8_t*>(smem);  // MR*K
    unsigned char* wbase = smem + ((MR * K + 15) & ~15) + wid * wave_bytes;
    int32_t* acc = reinterpret_cast<int32_t*>(wbase);                                 // [MR][rows][G]
    uint16_t* scl = reinterpret_cast<uint16_t*>(wbase + ((acc_words * 4 + 15) & ~15));  // [rows][G]
    float* accf = reinterpret_cast<float*>(acc);                                      // FE: [MR][rows][Gs]
    float* sclf = reinterpret_cast<float*>(scl);                                      // FE: [rows][Gs]
    float* rsc = reinterpret_cast<float*>(smem + ((MR * K + 15) & ~15) + 4 * wave_bytes);  // MR
    float* red = rsc + MR;                                                                // 4

    const uint8_t* Bbase = a.B + bi * a.sB;
    const uint16_t* Bsbase = a.Bs + bi * a.sBs;

    // chunk f = i*64 + lane of a tile: row f / cpr, column f % cpr (the same
    // for every tile; a short last tile only masks chunks off)
    int crow[CH], ccol[CH];
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int f = i * 64 + lane;
        crow[i] = f / cpr;
        ccol[i] = f - crow[i] * cpr;
    }
    i32x4 w[CH];
    uint16_t sv[CH];
    auto load_tile = [&](int t) {
        const int n0 = t * rows;
        const int nr = min(rows, a.N - n0);
        const i32x4* Bw = reinterpret_cast<const i32x4*>(Bbase + (size_t)n0 * row_bytes);
        const uint16_t* Sw = Bsbase + (size_t)n0 * G;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            w[i] = (i32x4){0, 0, 0, 0};
            if (i * 64 + lane < nr * cpr) w[i] = __builtin_nontemporal_load(Bw + i * 64 + lane);
        }
        // rows*G <= 64*CH for every tile shape the launcher picks
#pragma unroll
        for (int i = 0; i < CH; i++) {
            sv[i] = 0;
            if (i * 64 + lane < nr * G) sv[i] = Sw[i * 64 + lane];
        }
    };

    int t = t0 + wid;
    if (t < t1) load_tile(t);

    // activation codes (the per-row quantization of the matmul node)
    const int body = (K / 8) * 8;
    for (int m = 0; m < mr; m++) {
        if (F16ACT) {
            const uint16_t* x = a.A16 + bi * a.sA + (size_t)(m0 + m) * K;
            const float mx = block_max_abs_f16(x, K, red);
            const float s = row_scale_from_max(mx);
            const float inv = 1.0f / s;
            if constexpr (INT4) {
                for (int r = tid; r < K / 8; r += GEMV_THREADS) {
                    uint32_t w2[2] = {0, 0};
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        w2[e >> 2] |= (uint32_t)(uint8_t)quant_code(h2f(x[8 * r + e]), inv, 8 * r + e >= body)
                                      << (8 * (e & 3));
                    nib_store8(actq + m * K, K, r, nib_pack8(w2[0], w2[1]));
                }
            } else {
                for (int i = tid; i < K; i += GEMV_THREADS) actq[m * K + i] = quant_code(h2f(x[i]), inv, i >= body);
            }
            if (tid == 0) rsc[m] = s;
        } else {
            const int8_t* x = a.A8 + bi * a.sA + (size_t)(m0 + m) * K;
            if constexpr (INT4) {
                for (int r = tid; r < K / 8; r += GEMV_THREADS) {
                    uint32_t w2[2] = {0, 0};   // byte loads: the codes carry no alignment promise
#pragma unroll
                    for (int e = 0; e < 8; e++) w2[e >> 2] |= (uint32_t)(uint8_t)x[8 * r + e] << (8 * (e & 3));
                    nib_store8(actq + m * K, K, r, nib_pack8(w2[0], w2[1]));
                }
            } else {
                for (int i = tid; i < K; i += GEMV_THREADS) actq[m * K + i] = x[i];
            }
            if (tid == 0) rsc[m] = a.As[bi * (a.sA / K) + m0 + m];
        }
    }
    __syncthreads();
    float rsm[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) rsm[m] = m < mr ? rsc[m] : 0.0f;

    for (; t < t1; t += 4) {
        const int n0 = t * rows;
        const int nr = min(rows, a.N - n0);
        const int nch = nr * cpr;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            if constexpr (FE) {
                // one group per chunk: scale index = chunk index
                if (i * 64 + lane < nch) sclf[crow[i] * Gs + ccol[i]] = h2f(sv[i]);
            } else {
                if (i * 64 + lane < nr * G) scl[i * 64 + lane] = sv[i];
            }
        }
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const bool valid = i * 64 + lane < nch;
            int dot[MR];
#pragma unroll
            for (int m = 0; m < MR; m++) {
                dot[m] = (valid && m < mr) ? chunk_dot<INT4>(actq + m * K, ccol[i], w[i], K / 2) : 0;
                dot[m] = group_lane_sum(dot[m], P);
            }
            if (valid && (lane & (P - 1)) == 0) {
                const int g = ccol[i] / P;
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    if (m < mr) {
                        if constexpr (FE) accf[(m * rows + crow[i]) * Gs + g] = (float)dot[m];
                        else acc[(m * rows + crow[i]) * G + g] = dot[m];
                    }
                }
            }
        }
        if (t + 4 < t1) load_tile(t + 4);
        wave_lds_order();
        // reference epilogue, one lane per output of this tile
        for (int o = lane; o < mr * nr; o += 64) {
            const int m = o / nr, r = o - (o / nr) * nr;
            float rs;
            if constexpr (FE) {
                rs = group_epilogue_f(accf + (m * rows + r) * Gs, sclf + r * Gs, G);
            } else {
                const int32_t* ag = acc + (m * rows + r) * G;
                const uint16_t* sg = scl + r * G;
                // rows start 16-byte (sums) and 8-byte (scales) aligned when G % 4 == 0
                rs = (G & 3) == 0 ? group_epilogue_v4(ag, sg, G) : group_epilogue(ag, sg, G);
            }
            float s = rsm[0];
#pragma unroll
            for (int mm = 1; mm < MR; mm++)
                if (m == mm) s = rsm[mm];
            a.C[bi * a.sC + (size_t)(m0 + m) * a.N + n0 + r] = f2h(rs * s);
        }
        wave_lds_order();
    }
}

static size_t gemv_wave_smem(int MR, int K, int rows, int G, bool fe = false) {
    const int Gs = fe ? ((G + 3) & ~3) + 4 : G;
    const size_t wave = (size_t)((MR * rows * Gs * 4 + 15) & ~15) + (size_t)((rows * Gs * (fe ? 4 : 2) + 15) & ~15);
    return (size_t)((MR * K + 15) & ~15) + 4 * wave + (size_t)(MR + 4) * 4;
}

template <int MR, bool F16ACT, bool INT4, int CH>
static int launch_gemv_wave_t(const GemvArgs& a, size_t batch, int m0, size_t smem, hipStream_t st, bool fe) {
    const int ntiles = (a.N + a.rows - 1) / a.rows;
    dim3 grid(ceil_div(ntiles, a.tiles), (unsigned)batch);
    if constexpr (INT4) {
        if (fe) {
            hipLaunchKernelGGL((gemv_wave_kernel<MR, F16ACT, INT4, CH, true>), grid, dim3(GEMV_THREADS), smem,
                               st, a, m0);
            return check_launch("gemv_wave");
        }
    }
    hipLaunchKernelGGL((gemv_wave_kernel<MR, F16ACT, INT4, CH>), grid, dim3(GEMV_THREADS), smem,
                       st, a, m0);
    return check_launch("gemv_wave");
}

template <int MR, bool F16ACT, bool INT4>
static int launch_gemv_wave_ch(const GemvArgs& a, size_t batch, int m0, size_t smem, int ch,
                               hipStream_t st, bool fe) {
    switch (ch) {
        case 1: return launch_gemv_wave_t<MR, F16ACT, INT4, 1>(a, batch, m0, smem, st, fe);
        case 2: return launch_gemv_wave_t<MR, F16ACT, INT4, 2>(a, batch, m0, smem, st, fe);
        case 3: return launch_gemv_wave_t<MR, F16ACT, INT4, 3>(a, batch, m0, smem, st, fe);
        case 4: return launch_gemv_wave_t<MR, F16ACT, INT4, 4>(a, batch, m0, smem, st, fe);
        case 5: return launch_gemv_wave_t<MR, F16ACT, INT4, 5>(a, batch, m0, smem, st, fe);
        case 6: return launch_gemv_wave_t<MR, F16ACT, INT4, 6>(a, batch, m0, smem, st, fe);
        default: return launch_gemv_wave_t<MR, F16ACT, INT4, 8>(a, batch, m0, smem, st, fe);
    }
}

// Wave tile shape for the streaming kernel: CH chunks per lane and the rows
// (whole rows only) that fill them.  Prefers the slot count that wastes the
// fewest lanes, 5 or 4 chunks per lane at equal waste, then fewer chunks
// while the problem has too few tiles to give every CU several waves.
// Returns false when a row does not fit 8 slots (cpr > 512).
static bool pick_wave_tile(int cpr, size_t N, size_t batch, int* ch_out, int* rows_out) {
    static const int kCh[] = {5, 4, 6, 8, 3, 2, 1};
    int best_ch = 0;
    double best_util = 0.0;
    for (int ch : kCh) {
        const int rows = 64 * ch / cpr;
        if (rows < 1) continue;
        const double util = (double)rows * cpr / (64.0 * ch);
        if (util > best_util + 0.02) { best_util = util; best_ch = ch; }
    }
    if (!best_ch) return false;
    int ch = best_ch;
    // >= 4096 wave tiles in flight (1024 workgroups) when the problem allows
    while (ch > 1) {
        const int rows = 64 * ch / cpr;
        if ((size_t)ceil_div(N, (size_t)rows) * batch >= 4096) break;
        int next = 0;
        for (int c = ch - 1; c >= 1; c--)
            if (64 * c / cpr >= 1) { next = c; break; }
        if (!next) break;
        ch = next;
    }
    *ch_out = ch;
    *rows_out = min((size_t)(64 * ch / cpr), N);
    return true;
}

template <int MR, bool F16ACT, bool INT4, int CH>
static int launch_gemv_t(const GemvArgs& a, size_t batch, int m0, size_t smem, hipStream_t st) {
    const int ntiles = (a.N + a.rows - 1) / a.rows;
    dim3 grid(ceil_div(ntiles, a.tiles), (unsigned)batch);
    hipLaunchKernelGGL((gemv_grouped_kernel<MR, F16ACT, INT4, CH>), grid, dim3(GEMV_THREADS), smem,
                       st, a, m0);
    return check_launch("gemv_grouped");
}

template <int MR, bool F16ACT, bool INT4>
static int launch_gemv_ch(const GemvArgs& a, size_t batch, int m0, size_t smem, int ch,
                          hipStream_t st) {
    switch (ch) {
        case 1: return launch_gemv_t<MR, F16ACT, INT4, 1>(a, batch, m0, smem, st);
        case 2: return launch_gemv_t<MR, F16ACT, INT4, 2>(a, batch, m0, smem, st);
        case 4: return launch_gemv_t<MR, F16ACT, INT4, 4>(a, batch, m0, smem, st);
        case 6: return launch_gemv_t<MR, F16ACT, INT4, 6>(a, batch, m0, smem, st);
        default: return launch_gemv_t<MR, F16ACT, INT4, 8>(a, batch, m0, smem, st);
    }
}

template <bool F16ACT, bool INT4>
static int launch_gemv(GemvArgs a, size_t batch, hipStream_t st) {
    const int G = a.K / a.gs;
    const int cpr = INT4 ? a.K / 32 : a.K / 16;
    const int MR = a.M >= 4 ? 4 : (a.M >= 2 ? 2 : 1);
    int wch = 0, wrows = 0;
    // INT4 with 32-wide groups: one group per chunk, fp32 epilogue operands
    const bool fe = INT4 && a.gs == 32;
    if (pick_wave_tile(cpr, a.N, batch, &wch, &wrows) &&
        gemv_wave_smem(MR, a.K, wrows, G, fe) <= 60 * 1024) {
        // wave tiles per workgroup: 4 (one per wave) up to 4 * cap.  Every
        // workgroup quantizes the activation row once, so INT4 rows (the
        // K = 3072 MLP down shape) take more tiles per workgroup: swept on
        // MI355X over 604 / 768 rotated weight sets, INT4 K=3072 streams at
        // 0.751-0.753 of HBM with 8 per wave (0.745-0.753 with 12 or 16;
        // with the earlier scalar-read epilogue 0.706-0.710 with 8,
        // 0.68-0.69 with 6) and INT8 K=640 at 6.85 TB/s with 3-4 (6.72 with 8)
        const size_t nt = ceil_div(a.N, (size_t)wrows);
        size_t per = nt * batch / (4 * 2048 * (INT4 ? 2 : 3));
        if (per < 1) per = 1;
        if (per > (INT4 ? 8u : 4u)) per = INT4 ? 8 : 4;
        size_t nb = ceil_div(nt, 4 * per);
        a.rows = wrows;
        a.tiles = (int)ceil_div(nt, nb);  // balanced: every workgroup but the last full
        const size_t smem = gemv_wave_smem(MR, a.K, wrows, G, fe);
        for (int m0 = 0; m0 < a.M; m0 += MR) {
            int rc;
            if (MR == 4) rc = launch_gemv_wave_ch<4, F16ACT, INT4>(a, batch, m0, smem, wch, st, fe);
            else if (MR == 2) rc = launch_gemv_wave_ch<2, F16ACT, INT4>(a, batch, m0, smem, wch, st, fe);
            else rc = launch_gemv_wave_ch<1, F16ACT, INT4>(a, batch, m0, smem, wch, st, fe);
            if (rc) return rc;
        }
        return CACTUS_HIP_OK;
    }
    // a tile is about 4 chunks per thread (measured best: more registers per
    // thread cost occupancy); fewer rows when the whole problem would leave
    // CUs idle (256 CUs, aim for >= 4 workgroups each)
    int rows = (4 * GEMV_THREADS) / cpr;
    if (rows < 1) rows = 1;
    if (rows > a.N) rows = a.N;
    while (rows > 1 && (size_t)ceil_div(a.N, rows) * batch < 1024) rows = (rows + 1) / 2;
    while (rows > 1 && gemv_smem(MR, a.K, rows, G) > 60 * 1024) rows = (rows + 1) / 2;
    if (gemv_smem(MR, a.K, rows, G) > 60 * 1024 || rows * cpr > 8 * GEMV_THREADS)
        return fail(CACTUS_HIP_EUNSUPPORTED, "grouped matmul: K too large for the GEMV path");
    const int chunks = (rows * cpr + GEMV_THREADS - 1) / GEMV_THREADS;
    const int ch = chunks <= 1 ? 1 : chunks <= 2 ? 2 : chunks <= 4 ? 4 : chunks <= 6 ? 6 : 8;
    // tiles per workgroup: up to 8 once there are >= 2048 tiles in flight
    const size_t ntiles = ceil_div(a.N, rows);
    size_t per = ntiles * batch / 2048;
    if (per < 1) per = 1;
    if (per > 8) per = 8;
    a.rows = rows;
    a.tiles = (int)per;
    const size_t smem = gemv_smem(MR, a.K, rows, G);
    for (int m0 = 0; m0 < a.M; m0 += MR) {
        int rc;
        if (MR == 4) rc = launch_gemv_ch<4, F16ACT, INT4>(a, batch, m0, smem, ch, st);
        else if (MR == 2) rc = launch_gemv_ch<2, F16ACT, INT4>(a, batch, m0, smem, ch, st);
        else rc = launch_gemv_ch<1, F16ACT, INT4>(a, batch, m0, smem, ch, st);
        if (rc) return rc;
    }
    return CACTUS_HIP_OK;
}

static bool is_pow2(size_t v) { return v && !(v & (v - 1)); }

int check_grouped_shape(size_t M, size_t K, size_t N, size_t gs, bool int4) {
    CH_REQUIRE(gs > 0 && K % gs == 0, "grouped matmul: group_size must divide K");
    CH_REQUIRE(is_pow2(gs) && gs >= (int4 ? 32u : 16u) && gs <= (int4 ? 2048u : 1024u),
               "grouped matmul: group_size must be a power of two in [16,1024] (INT8) or "
               "[32,2048] (INT4)");
    CH_REQUIRE(M < (1u << 30) && K < (1u << 20) && N < (1u << 30), "grouped matmul: shape too large");
    return CACTUS_HIP_OK;
}

}  // namespace cactus_hip

using namespace cactus_hip;

// Internal dispatch shared with the MFMA prefill path (gemm.hip).
namespace cactus_hip {
int gemm_grouped_mfma(const uint16_t* A16, const int8_t* A8, const float* As, const uint8_t* B,
                      const uint16_t* Bs, uint16_t* C, size_t M, size_t K, size_t N, size_t gs,
                      bool int4, hipStream_t st, bool* handled,
                      const uint16_t* R = nullptr, void* ext_scratch = nullptr);
int gemm_grouped_mfma_multi(const int8_t* A8, const float* As, int np, const uint8_t* const* B,
                            const uint16_t* const* Bs, uint16_t* const* C, const size_t* N, size_t M, size_t K,
                            size_t gs, bool int4, hipStream_t st, bool* handled);

// C[i] = fp16(C[i] + R[i]): the residual add node after a small-M matmul
__global__ void add_residual_kernel(uint16_t* C, const uint16_t* R, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        C[i] = hadd(C[i], R[i]);
}

// ext_scratch: caller-provided device memory for the MFMA path's activation
// codes and row scales (at least gemm_act_scratch_bytes(M, K)), or null for
// the library's own per-stream buffer.
int grouped_dispatch(const uint16_t* A16, const int8_t* A8, const float* As,
                     const uint8_t* B, const uint16_t* Bs, uint16_t* C, size_t M, size_t K,
                     size_t N, size_t gs, bool int4, hipStream_t st, const uint16_t* R = nullptr,
                     void* ext_scratch = nullptr) {
    if (M == 0 || K == 0 || N == 0) return CACTUS_HIP_OK;
    int rc = check_grouped_shape(M, K, N, gs, int4);
    if (rc) return rc;
    CH_REQUIRE(B && Bs && C && (A16 || (A8 && As)), "grouped matmul: null pointer");
    CH_REQUIRE(((uintptr_t)B & 15) == 0, "grouped matmul: weights must be 16-byte aligned");
    bool handled = false;
    rc = gemm_grouped_mfma(A16, A8, As, B, Bs, C, M, K, N, gs, int4, st, &handled, R, ext_scratch);
    if (rc || handled) return rc;
    GemvArgs a{};
    a.A16 = A16; a.A8 = A8; a.As = As; a.B = B; a.Bs = Bs; a.C = C;
    a.M = (int)M; a.K = (int)K; a.N = (int)N; a.gs = (int)gs;
    a.sA = M * K; a.sB = 0; a.sBs = 0; a.sC = 0;
    if (A16) rc = int4 ? launch_gemv<true, true>(a, 1, st) : launch_gemv<true, false>(a, 1, st);
    else rc = int4 ? launch_gemv<false, true>(a, 1, st) : launch_gemv<false, false>(a, 1, st);
    // small M: the residual add runs as its own kernel, in place on C
    if (rc == 0 && R) {
        const size_t n = M * N;
        const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 65535);
        hipLaunchKernelGGL(add_residual_kernel, dim3(blocks), dim3(256), 0, st, C, R, n);
        rc = check_launch("matmul_add (residual)");
    }
    return rc;
}
}  // namespace cactus_hip

extern "C" {

int cactus_hip_matmul_int8(const int8_t* A, const float* A_scales, const int8_t* B,
                           const uint16_t* B_scales, uint16_t* C, size_t M, size_t K, size_t N,
                           size_t group_size, void* stream) {
    return grouped_dispatch(nullptr, A, A_scales, reinterpret_cast<const uint8_t*>(B), B_scales, C,
                            M, K, N, group_size, false, as_stream(stream));
}

int cactus_hip_matmul_int4(const int8_t* A, const float* A_scales, const uint8_t* B_packed,
                           const uint16_t* B_scales, uint16_t* C, size_t M, size_t K, size_t N,
                           size_t group_size, void* stream) {
    return grouped_dispatch(nullptr, A, A_scales, B_packed, B_scales, C, M, K, N, group_size, true,
                            as_stream(stream));
}

int cactus_hip_matmul_int8_f16act(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                  uint16_t* C, size_t M, size_t K, size_t N, size_t group_size,
                                  void* stream) {
    return grouped_dispatch(A, nullptr, nullptr, reinterpret_cast<const uint8_t*>(B), B_scales, C,
                            M, K, N, group_size, false, as_stream(stream));
}

int cactus_hip_matmul_int4_f16act(const uint16_t* A, const uint8_t* B_packed,
                                  const uint16_t* B_scales, uint16_t* C, size_t M, size_t K,
                                  size_t N, size_t group_size, void* stream) {
    return grouped_dispatch(A, nullptr, nullptr, B_packed, B_scales, C, M, K, N, group_size, true,
                            as_stream(stream));
}

int cactus_hip_matmul_int8_add(const int8_t* A, const float* A_scales, const int8_t* B, const uint16_t* B_scales,
                               const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                               size_t group_size, void* stream) {
    CH_REQUIRE(residual || M * K * N == 0, "matmul_add: null residual");
    return grouped_dispatch(nullptr, A, A_scales, reinterpret_cast<const uint8_t*>(B), B_scales, C, M, K, N,
                            group_size, false, as_stream(stream), residual);
}

int cactus_hip_matmul_int4_add(const int8_t* A, const float* A_scales, const uint8_t* B_packed,
                               const uint16_t* B_scales, const uint16_t* residual, uint16_t* C, size_t M, size_t K,
                               size_t N, size_t group_size, void* stream) {
    CH_REQUIRE(residual || M * K * N == 0, "matmul_add: null residual");
    return grouped_dispatch(nullptr, A, A_scales, B_packed, B_scales, C, M, K, N, group_size, true,
                            as_stream(stream), residual);
}

int cactus_hip_matmul_int8_f16act_add(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                      const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                                      size_t group_size, void* stream) {
    CH_REQUIRE(residual || M * K * N == 0, "matmul_add: null residual");
    return grouped_dispatch(A, nullptr, nullptr, reinterpret_cast<const uint8_t*>(B), B_scales, C, M, K, N,
                            group_size, false, as_stream(stream), residual);
}

int cactus_hip_matmul_int4_f16act_add(const uint16_t* A, const uint8_t* B_packed, const uint16_t* B_scales,
                                      const uint16_t* residual, uint16_t* C, size_t M, size_t K, size_t N,
                                      size_t group_size, void* stream) {
    CH_REQUIRE(residual || M * K * N == 0, "matmul_add: null residual");
    return grouped_dispatch(A, nullptr, nullptr, B_packed, B_scales, C, M, K, N, group_size, true,
                            as_stream(stream), residual);
}

int cactus_hip_matmul_grouped_multi(const int8_t* A, const float* A_scales, size_t count, const void* const* B,
                                    const uint16_t* const* B_scales, uint16_t* const* C, const size_t* N, size_t M,
                                    size_t K, size_t group_size, int int4, void* stream) {
    CH_REQUIRE(count >= 1 && count <= 3, "matmul_grouped_multi: count must be 1, 2 or 3");
    CH_REQUIRE(B && B_scales && C && N, "matmul_grouped_multi: null pointer");
    if (M == 0 || K == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(A && A_scales, "matmul_grouped_multi: null pointer");
    const uint8_t* bp[3];
    for (size_t i = 0; i < count; i++) {
        int rc = check_grouped_shape(M, K, N[i], group_size, int4 != 0);
        if (rc) return rc;
        CH_REQUIRE(B[i] && B_scales[i] && C[i], "matmul_grouped_multi: null pointer");
        CH_REQUIRE(((uintptr_t)B[i] & 15) == 0, "matmul_grouped_multi: weights must be 16-byte aligned");
        CH_REQUIRE(N[i] > 0, "matmul_grouped_multi: every N must be positive");
        bp[i] = static_cast<const uint8_t*>(B[i]);
    }
    const hipStream_t st = as_stream(stream);
    bool handled = false;
    int rc = gemm_grouped_mfma_multi(A, A_scales, (int)count, bp, B_scales, C, N, M, K, group_size, int4 != 0, st,
                                     &handled);
    if (rc || handled) return rc;
    // one launch per problem: the same per-output arithmetic
    for (size_t i = 0; i < count && rc == 0; i++)
        rc = grouped_dispatch(nullptr, A, A_scales, bp[i], B_scales[i], C[i], M, K, N[i], group_size, int4 != 0, st);
    return rc;
}

int cactus_hip_matmul_int8_f16act_batched(const uint16_t* A, const int8_t* B,
                                          const uint16_t* B_scales, uint16_t* C, size_t M,
                                          size_t K, size_t N, size_t group_size, size_t batch,
                                          size_t stride_a, size_t stride_b, size_t stride_bs,
                                          size_t stride_c, void* stream) {
    if (M == 0 || K == 0 || N == 0 || batch == 0) return CACTUS_HIP_OK;
    int rc = check_grouped_shape(M, K, N, group_size, false);
    if (rc) return rc;
    CH_REQUIRE(A && B && B_scales && C, "matmul_int8_f16act_batched: null pointer");
    CH_REQUIRE(batch <= 65535, "matmul_int8_f16act_batched: batch must be <= 65535");
    CH_REQUIRE(((uintptr_t)B & 15) == 0 && stride_b % 16 == 0,
               "matmul_int8_f16act_batched: weights must be 16-byte aligned");
    GemvArgs a{};
    a.A16 = A; a.B = reinterpret_cast<const uint8_t*>(B); a.Bs = B_scales; a.C = C;
    a.M = (int)M; a.K = (int)K; a.N = (int)N; a.gs = (int)group_size;
    a.sA = stride_a; a.sB = stride_b; a.sBs = stride_bs; a.sC = stride_c;
    return launch_gemv<true, false>(a, batch, as_stream(stream));
}

int cactus_hip_matmul_int4_f16act_batched(const uint16_t* A, const uint8_t* B_packed,
                                          const uint16_t* B_scales, uint16_t* C, size_t M,
                                          size_t K, size_t N, size_t group_size, size_t batch,
                                          size_t stride_a, size_t stride_b, size_t stride_bs,
                                          size_t stride_c, void* stream) {
    if (M == 0 || K == 0 || N == 0 || batch == 0) return CACTUS_HIP_OK;
    int rc = check_grouped_shape(M, K, N, group_size, true);
    if (rc) return rc;
    CH_REQUIRE(A && B_packed && B_scales && C, "matmul_int4_f16act_batched: null pointer");
    CH_REQUIRE(batch <= 65535, "matmul_int4_f16act_batched: batch must be <= 65535");
    CH_REQUIRE(((uintptr_t)B_packed & 15) == 0 && stride_b % 16 == 0,
               "matmul_int4_f16act_batched: weights must be 16-byte aligned");
    GemvArgs a{};
    a.A16 = A; a.B = B_packed; a.Bs = B_scales; a.C = C;
    a.M = (int)M; a.K = (int)K; a.N = (int)N; a.gs = (int)group_size;
    a.sA = stride_a; a.sB = stride_b; a.sBs = stride_bs; a.sC = stride_c;
    return launch_gemv<true, true>(a, batch, as_stream(stream));
}

}  // extern "C"
