// gemm.hip -- grouped INT8 / INT4 matmul for prefill-sized M on INT8 MFMA.
//
// C[m][n] = fp16( (fma-chain over groups g ascending of (float)acc_{m,n,g} *
// Bs[n][g]) * As[m] ), acc = exact int32 group sum (kernel_gemm.cpp:128-327
// for INT8, :329-529 for INT4; epilogue :311-324).
//
// gfx950's v_mfma_i32_32x32x32_i8 contracts exactly 32 k per instruction, so
// one instruction (or gs/32 chained into the same zeroed accumulator) yields
// one group's exact int32 sums for a 32x32 output tile.  The reference's fp32
// group epilogue then runs on the VALU while the matrix core works on the
// next group: the bit-exact epilogue (a convert and an FMA per output and
// group) is what bounds this kernel, not the MFMA rate.
//
// Operand layout of v_mfma_i32_32x32x32_i8 (checked on the device): lane l
// holds A[l % 32][16 (l / 32) .. +16) and B[16 (l / 32) .. +16)[l % 32] (so a
// row of the [N][K] weight matrix, read contiguously); result register r of
// lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
//
// INT4 weights are expanded to bytes holding code << 4 (low nibble = even k,
// kernel_utils.h:165-185): the MFMA sum is then 16 acc, and (float)(16 acc)
// = 16 (float)acc exactly, so fma((float)(16 acc), Bs / 16, r) is the
// reference's fma((float)acc, Bs, r) bit for bit.
#include "hip_common.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <type_traits>
#include <mutex>

namespace cactus_hip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// 16 k-values of one operand row: INT8 directly, INT4 expanded (code << 4)
template <bool INT4>
__device__ __forceinline__ v4i load_b16(const uint8_t* p) {
    if constexpr (!INT4) {
        return *reinterpret_cast<const v4i*>(p);
    } else {
        const uint2 w = *reinterpret_cast<const uint2*>(p);
        v4i o;
        const uint32_t l0 = (w.x << 4) & 0xF0F0F0F0u, h0 = w.x & 0xF0F0F0F0u;
        const uint32_t l1 = (w.y << 4) & 0xF0F0F0F0u, h1 = w.y & 0xF0F0F0F0u;
        o.x = (int)__builtin_amdgcn_perm(h0, l0, 0x05010400u);
        o.y = (int)__builtin_amdgcn_perm(h0, l0, 0x07030602u);
        o.z = (int)__builtin_amdgcn_perm(h1, l1, 0x05010400u);
        o.w = (int)__builtin_amdgcn_perm(h1, l1, 0x07030602u);
        return o;
    }
}

struct GemmArgs {
    const int8_t* A;      // [M][K] int8 codes
    const float* As;      // [M]
    const uint8_t* B;     // [N][K] int8 or [N][K/2] packed int4
    const uint16_t* Bs;   // [N][K/gs] fp16
    uint16_t* C;          // [M][N] fp16
    int M, K, N, gs;
    const uint16_t* R = nullptr;   // [M][N] fp16 residual added to C (the add node), or null
    // Up to two further problems over the same A, M, K and group size (the
    // LDS kernel only): workgroups with blockIdx.x >= bx[i] take problem
    // i + 1, with its own weights, scales, output and N (no residual).
    int np = 1;
    int bx[2] = {0, 0};
    const uint8_t* Bx[2] = {nullptr, nullptr};
    const uint16_t* Bsx[2] = {nullptr, nullptr};
    uint16_t* Cx[2] = {nullptr, nullptr};
    int Nx[2] = {0, 0};
};

// Workgroup: 4 waves, 64 rows x 64*NW columns; wave (wv >> 1, wv & 1) owns
// 32 rows x 32*NW columns (NW MFMA tiles side by side, sharing the A operand).
template <bool INT4, int NW>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(GemmArgs a) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int K = a.K, N = a.N, M = a.M;
    const int G = K / a.gs, ksub = a.gs / 32;
    const int m0 = blockIdx.y * 64 + (wv >> 1) * 32;
    const int n0 = blockIdx.x * (64 * NW) + (wv & 1) * 32 * NW;
    if (m0 >= M || n0 >= N) return;
    const int li = lane & 31, kh = lane >> 5;
    const int8_t* ap = a.A + (size_t)min(m0 + li, M - 1) * K + kh * 16;
    const size_t brow = INT4 ? (size_t)K / 2 : (size_t)K;
    const uint8_t* bp[NW];
    const uint16_t* sp[NW];
#pragma unroll
    for (int s = 0; s < NW; s++) {
        const int col = min(n0 + s * 32 + li, N - 1);
        bp[s] = a.B + (size_t)col * brow + (INT4 ? kh * 8 : kh * 16);
        sp[s] = a.Bs + (size_t)col * G;
    }
    const float sdiv = INT4 ? 0.0625f : 1.0f;   // Bs / 16 for the nibble << 4 codes
    constexpr int BSTEP = INT4 ? 16 : 32;       // operand bytes per 32 k

    float r[NW][16];
#pragma unroll
    for (int s = 0; s < NW; s++)
#pragma unroll
        for (int e = 0; e < 16; e++) r[s][e] = 0.0f;

    auto epilogue = [&](const v16i* acc, const float* sc) {
#pragma unroll
        for (int s = 0; s < NW; s++)
#pragma unroll
            for (int e = 0; e < 16; e++) r[s][e] = __builtin_fmaf((float)acc[s][e], sc[s], r[s][e]);
    };

    if (ksub == 1) {
        // one MFMA per group and tile.  Operands stream through a 4-deep
        // register ring (loaded three groups ahead), and the next group's
        // MFMA is issued before the current group's epilogue.
        struct Frag {
            v4i a;
            v4i b[NW];
            float sc[NW];
        };
        Frag F[4];
        auto load = [&](Frag& f, int g) {
            f.a = *reinterpret_cast<const v4i*>(ap + (size_t)g * 32);
#pragma unroll
            for (int s = 0; s < NW; s++) {
                f.b[s] = load_b16<INT4>(bp[s] + (size_t)g * BSTEP);
                f.sc[s] = h2f(sp[s][g]) * sdiv;
            }
        };
        v16i acc[2][NW];
#pragma unroll
        for (int j = 0; j < 3; j++)
            if (j < G) load(F[j], j);
#pragma unroll
        for (int s = 0; s < NW; s++) acc[0][s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(F[0].a, F[0].b[s], (v16i){}, 0, 0, 0);
        for (int g = 0; g < G; g += 4) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int gg = g + j;
                if (gg >= G) break;
                if (gg + 3 < G) load(F[(j + 3) & 3], gg + 3);
                if (gg + 1 < G) {
#pragma unroll
                    for (int s = 0; s < NW; s++)
                        acc[(j + 1) & 1][s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(F[(j + 1) & 3].a, F[(j + 1) & 3].b[s],
                                                                                 (v16i){}, 0, 0, 0);
                }
                epilogue(acc[j & 1], F[j & 3].sc);
            }
        }
    } else {
        // groups of 64..1024 k: gs / 32 MFMAs chained into one accumulator
        for (int g = 0; g < G; g++) {
            v16i acc[NW];
#pragma unroll
            for (int s = 0; s < NW; s++) acc[s] = (v16i){};
            for (int t = 0; t < ksub; t++) {
                const size_t kk = (size_t)g * ksub + t;
                const v4i fa = *reinterpret_cast<const v4i*>(ap + kk * 32);
#pragma unroll
                for (int s = 0; s < NW; s++)
                    acc[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, load_b16<INT4>(bp[s] + kk * BSTEP), acc[s],
                                                                   0, 0, 0);
            }
            float sc[NW];
#pragma unroll
            for (int s = 0; s < NW; s++) sc[s] = h2f(sp[s][g]) * sdiv;
            epilogue(acc, sc);
        }
    }

    // C = fp16(r * As[row])
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int row = m0 + 8 * (e / 4) + 4 * kh + (e % 4);
        if (row >= M) continue;
        const float as = a.As[row];
#pragma unroll
        for (int s = 0; s < NW; s++) {
            const int col = n0 + s * 32 + li;
            if (col < N) {
                const uint16_t c = f2h(r[s][e] * as);
                a.C[(size_t)row * N + col] = a.R ? hadd(c, a.R[(size_t)row * N + col]) : c;
            }
        }
    }
}

// ------------------------------------------------ LDS-staged 16x16 tiling
// v_mfma_i32_16x16x32_i8: lane l holds A[l % 16][8 (l / 16) .. +8) and
// B[8 (l / 16) .. +8)[l % 16] (8 bytes each); result register i of lane l is
// C[4 (l / 16) + i][l % 16].  One instruction covers one 32-k chunk of a
// 16x16 output tile, so an output tile costs 8 VALU instructions per group
// (4 converts + 4 FMAs) against one MFMA: the epilogue, not the matrix core,
// sets the pace, and the tiling is chosen to keep every SIMD's VALU busy.
//
// Workgroup = WGM x WGN waves, each WM x WN outputs.  A single wave issues
// at most one VALU instruction per ~7 cycles on gfx950, so the epilogue only
// reaches the SIMD's rate with two or more waves per SIMD.
// The K loop runs over stages of SG 32-k chunks.  A stage holds, for each of
// the workgroup's BM rows of A and BN columns of B, that row's SG * 32 (INT4:
// SG * 16) contiguous bytes, moved by global_load_lds_dwordx4 with
// consecutive lanes on consecutive 16-byte pieces of one row (whole cache
// lines per 8 lanes), and each column's GPS group scales (global_load_lds_dword).
// NS stages form a ring; loads run NS - 1 stages ahead of the MFMAs.
// In LDS a row is [pieces][16 B] with piece p stored in slot p ^ (row & 7)
// (INT4 columns of 4 pieces: p ^ (col & 3)), so the 16 rows one operand read
// spans land on distinct banks; scales are [col][GPS] fp16.
template <bool INT4, int WM_, int WN_, int WGM_, int WGN_, int KSUB_, int NS_ = 3>
struct LdsCfg {
    static constexpr int WM = WM_, WN = WN_, WGM = WGM_, WGN = WGN_, KSUB = KSUB_;
    static constexpr int NW = WGM * WGN, NT = 64 * NW;  // waves, threads
    static constexpr int BM = WGM * WM, BN = WGN * WN;
    static constexpr int TM = WM / 16, TN = WN / 16;
    static constexpr int SG = KSUB == 4 ? 8 : 4;        // chunks per stage: an even number of groups
    static constexpr int GPS = SG / KSUB;               // groups per stage (2 or 4)
    static constexpr int PA = SG * 2;                   // 16-byte pieces per A row and stage
    static constexpr int PB = INT4 ? SG : SG * 2;       // per B column and stage
    static constexpr int BMASK = PB >= 8 ? 7 : 3;       // B piece swizzle
    static constexpr int NBJ = INT4 ? SG : 4;           // precomputed B read offsets per tile
    static constexpr int A_U = BM * PA;                 // 16-byte units of A per stage
    static constexpr int U = A_U + BN * PB;
    static constexpr int NI = (U + NT - 1) / NT;        // 16-byte DMA instructions per wave per stage
    static constexpr int OPND = NI * NW * 1024;         // operand bytes per ring slot (padded)
    static constexpr int SC_U = BN * GPS / 2;           // dword units of scales per stage
    static constexpr int NSI = (SC_U + NT - 1) / NT;    // dword DMA instructions per wave per stage
    static constexpr int STAGE = OPND + NSI * NW * 256; // bytes per ring slot
    static constexpr int VM_STAGE = NI + NSI;           // vmcnt per stage and wave
    static constexpr int NS = NS_;                      // ring slots
    static constexpr int UNR = NS % 2 == 0 ? NS : 2 * NS;   // stage loop unroll: slot and scale parity static
    static constexpr int CSTEP_B = INT4 ? 16 : 32;      // B bytes per chunk and column
    static_assert(WM % 16 == 0 && WN % 16 == 0 && NW <= 16, "tile");
    static_assert(GPS % 2 == 0, "accumulator parity is static within a stage");
    static_assert(BM * BN * 2 <= STAGE, "output transpose fits one ring slot");
    static_assert(VM_STAGE * (NS - 2) <= 63, "vmcnt range");
    static_assert(NS == 3 || NS == 4, "ring of three or four slots");
};

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <class C, bool INT4>
__global__ void __launch_bounds__(C::NT) gemm_lds_kernel(GemmArgs a0) {
    extern __shared__ __align__(16) uint8_t smem[];
    // the problem of this workgroup (selects, not indexing: the arguments stay scalar)
    GemmArgs a = a0;
    int bxi = blockIdx.x;
    if (a0.np > 1 && bxi >= a0.bx[0]) {
        const bool p2 = a0.np > 2 && bxi >= a0.bx[1];
        bxi -= p2 ? a0.bx[1] : a0.bx[0];
        a.B = p2 ? a0.Bx[1] : a0.Bx[0];
        a.Bs = p2 ? a0.Bsx[1] : a0.Bsx[0];
        a.C = p2 ? a0.Cx[1] : a0.Cx[0];
        a.N = p2 ? a0.Nx[1] : a0.Nx[0];
        a.R = nullptr;
    }
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int K = a.K, N = a.N, M = a.M;
    const int NK = K / 32, G = NK / C::KSUB, NSTAGE = NK / C::SG;
    const int mb = blockIdx.y * C::BM, nb = bxi * C::BN;
    const int wm = wv / C::WGN, wn = wv % C::WGN;
    const size_t brow = INT4 ? (size_t)K / 2 : (size_t)K;
    const int q = lane >> 4, l16 = lane & 15;

    // row scales of this lane's output rows, fetched up front
    float as[C::TM][4];
#pragma unroll
    for (int x = 0; x < C::TM; x++)
#pragma unroll
        for (int e = 0; e < 4; e++) as[x][e] = a.As[min(mb + wm * C::WM + x * 16 + 4 * q + e, M - 1)];

    // DMA sources: 16-byte instruction i of this wave moves unit u = (wv + NW i) * 64 + lane,
    // dword instruction i moves scale unit v = (wv + NW i) * 64 + lane
    const uint8_t* src[C::NI];
    uint32_t inc[C::NI];
#pragma unroll
    for (int i = 0; i < C::NI; i++) {
        const int u = (wv + C::NW * i) * 64 + lane;
        // units past U pad the last instruction: a fixed 16-byte read of the
        // weights, never used
        src[i] = a.B;
        inc[i] = 0;
        if (u < C::A_U) {
            const int row = u / C::PA, p = (u % C::PA) ^ (row & 7);
            src[i] = reinterpret_cast<const uint8_t*>(a.A) + (size_t)min(mb + row, M - 1) * K + p * 16;
            inc[i] = C::SG * 32;
        } else if (u < C::U) {
            const int u2 = u - C::A_U;
            const int col = u2 / C::PB, p = (u2 % C::PB) ^ (col & C::BMASK);
            src[i] = a.B + (size_t)min(nb + col, N - 1) * brow + p * 16;
            inc[i] = C::SG * C::CSTEP_B;
        }
    }
    const uint16_t* ssrc[C::NSI];
    uint32_t sinc[C::NSI];
#pragma unroll
    for (int i = 0; i < C::NSI; i++) {
        const int v = (wv + C::NW * i) * 64 + lane;
        ssrc[i] = a.Bs;
        sinc[i] = 0;
        if (v < C::SC_U) {
            const int col = v / (C::GPS / 2), d = v % (C::GPS / 2);
            ssrc[i] = a.Bs + (size_t)min(nb + col, N - 1) * G + 2 * d;
            sinc[i] = C::GPS;
        }
    }
    const uint32_t ring = (uint32_t)(uintptr_t)smem;
    auto issue = [&](int s, int slot) {
        const uint32_t base = ring + (uint32_t)(slot * C::STAGE);
#pragma unroll
        for (int i = 0; i < C::NI; i++)
            lds_dma<16>(src[i] + (size_t)s * inc[i], base + (uint32_t)((wv + C::NW * i) * 1024));
#pragma unroll
        for (int i = 0; i < C::NSI; i++)
            lds_dma<4>(ssrc[i] + (size_t)s * sinc[i], base + (uint32_t)(C::OPND + (wv + C::NW * i) * 256));
    };
#pragma unroll
    for (int s = 0; s < C::NS - 1; s++)
        if (s < NSTAGE) issue(s, s);

    // operand read offsets within a stage (bytes): A / INT8 B piece
    // p = 2 j + (q >> 1) of row r sits at slot p ^ (r & 7), i.e. at
    // 128 (j >> 2) + 32 ((j & 3) ^ ((r >> 1) & 3)) + 16 ((q >> 1) ^ (r & 1))
    uint32_t ao[C::TM][4], bo[C::TN][C::NBJ], so[C::TN];
#pragma unroll
    for (int t = 0; t < C::TM; t++) {
        const int r = wm * C::WM + t * 16 + l16;
#pragma unroll
        for (int m = 0; m < 4; m++)
            ao[t][m] = (uint32_t)(r * C::PA * 16 + 32 * (m ^ ((r >> 1) & 3)) + 16 * ((q >> 1) ^ (r & 1)) + 8 * (q & 1));
    }
#pragma unroll
    for (int t = 0; t < C::TN; t++) {
        const int c = wn * C::WN + t * 16 + l16;
        const uint32_t cb = (uint32_t)(C::A_U * 16 + c * C::PB * 16);
#pragma unroll
        for (int m = 0; m < C::NBJ; m++)
            bo[t][m] = INT4 ? cb + 16 * (m ^ (c & C::BMASK)) + 4 * q
                            : cb + 32 * (m ^ ((c >> 1) & 3)) + 16 * ((q >> 1) ^ (c & 1)) + 8 * (q & 1);
        so[t] = (uint32_t)(C::OPND + c * C::GPS * 2);
    }

    float r[C::TM][C::TN][4];
#pragma unroll
    for (int x = 0; x < C::TM; x++)
#pragma unroll
        for (int y = 0; y < C::TN; y++)
#pragma unroll
            for (int e = 0; e < 4; e++) r[x][y][e] = 0.0f;
    i32x4 acc[2][C::TM][C::TN];
    // this stage's and the previous stage's group scales (fp16 pairs)
    uint32_t scw[2][C::TN][C::GPS / 2];

    struct Frag {
        long fa[C::TM];
        long fb[C::TN];
    };
    auto read = [&](const uint8_t* stage, int j, Frag& f) {
#pragma unroll
        for (int t = 0; t < C::TM; t++)
            f.fa[t] = *reinterpret_cast<const long*>(stage + ao[t][j & 3] + 128 * (j >> 2));
#pragma unroll
        for (int t = 0; t < C::TN; t++) {
            if constexpr (INT4) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(stage + bo[t][j]);
                const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                const uint32_t x0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                const uint32_t x1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
                f.fb[t] = (long)(((uint64_t)x1 << 32) | x0);
            } else {
                f.fb[t] = *reinterpret_cast<const long*>(stage + bo[t][j & 3] + 128 * (j >> 2));
            }
        }
    };
    auto read_scales = [&](const uint8_t* stage, int sb) {
#pragma unroll
        for (int t = 0; t < C::TN; t++) {
            if constexpr (C::GPS == 4) {
                const uint2 w = *reinterpret_cast<const uint2*>(stage + so[t]);
                scw[sb][t][0] = w.x;
                scw[sb][t][1] = w.y;
            } else {
                scw[sb][t][0] = *reinterpret_cast<const uint32_t*>(stage + so[t]);
            }
        }
    };
    // r = fma((float)acc, Bs, r) per output; for INT4 the MFMA sums are 16 acc
    // and r carries 16 r (exact: power-of-two scaling), undone at the store
    auto epilogue = [&](int buf, int sb, int gl) {
#pragma unroll
        for (int y = 0; y < C::TN; y++) {
            const uint32_t w = scw[sb][y][gl >> 1];
            const float sc = h2f((uint16_t)((gl & 1) ? (w >> 16) : (w & 0xFFFFu)));
#pragma unroll
            for (int x = 0; x < C::TM; x++)
#pragma unroll
                for (int e = 0; e < 4; e++) r[x][y][e] = __builtin_fmaf((float)acc[buf][x][y][e], sc, r[x][y][e]);
        }
    };

    // one stage; the ring slot is a compile-time constant so the LDS offsets
    // fold into the read instructions
    auto stage = [&](auto slotc, int s) {
        constexpr int SL = decltype(slotc)::value;
        constexpr int SB = SL & 1;   // scale register set of this stage (ring of two)
        static_assert(SL < C::UNR, "slot index");
        // stage s landed once at most the younger stages s + 1 .. s + NS - 2 fly
        const int younger = min(NSTAGE - 1 - s, C::NS - 2);
        if (younger >= C::NS - 2) wait_dma<C::VM_STAGE * (C::NS - 2)>();
        else if (younger == 1) wait_dma<C::VM_STAGE>();
        else wait_dma<0>();
        lds_barrier();
        if (s + C::NS - 1 < NSTAGE) issue(s + C::NS - 1, (SL + C::NS - 1) % C::NS);
        const uint8_t* st = smem + (SL % C::NS) * C::STAGE;
        Frag f[2];
        read(st, 0, f[0]);
        read_scales(st, SB);
#pragma unroll
        for (int j = 0; j < C::SG; j++) {
            if (j + 1 < C::SG) read(st, j + 1, f[(j + 1) & 1]);
            const int gl = j / C::KSUB, buf = gl & 1;
            const bool first = (j % C::KSUB) == 0;
#pragma unroll
            for (int x = 0; x < C::TM; x++)
#pragma unroll
                for (int y = 0; y < C::TN; y++)
                    acc[buf][x][y] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                        f[j & 1].fa[x], f[j & 1].fb[y], first ? (i32x4){0, 0, 0, 0} : acc[buf][x][y], 0, 0, 0);
            // the previous group's epilogue runs behind this chunk's MFMAs
            if (first) {
                if (j == 0) {
                    if (s > 0) epilogue(1, SB ^ 1, C::GPS - 1);
                } else {
                    epilogue(buf ^ 1, SB, gl - 1);
                }
            }
        }
    };
    // ring slot (s % NS) and scale register set (s % 2) are compile-time
    // constants in the unrolled body
    for (int s = 0; s < NSTAGE; s += C::UNR)
        static_for(std::make_integer_sequence<int, C::UNR>{}, [&](auto ic) {
            constexpr int I = decltype(ic)::value;
            if (s + I < NSTAGE) stage(ic, s + I);
        });
    epilogue(1, (NSTAGE - 1) & 1, C::GPS - 1);

    // store: fp16(r * As) into a wave-private 16x16 block per tile in a ring
    // slot no wave reads any more (that of stage NSTAGE - 2, consumed before
    // the last stage's barrier, or one never filled), then 16-byte rows to
    // global memory
    const float post = INT4 ? 0.0625f : 1.0f;
    uint16_t* ob = reinterpret_cast<uint16_t*>(smem + ((NSTAGE + C::NS - 2) % C::NS) * C::STAGE) +
                   wv * (C::TM * C::TN * 256);
#pragma unroll
    for (int x = 0; x < C::TM; x++)
#pragma unroll
        for (int y = 0; y < C::TN; y++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                ob[(x * C::TN + y) * 256 + (4 * q + e) * 16 + l16] = f2h((r[x][y][e] * post) * as[x][e]);
    const bool vec_ok = (N & 7) == 0 && ((uintptr_t)a.C & 15) == 0;
    // lane -> (tile, row, half): 32 lanes per tile
#pragma unroll
    for (int t0 = 0; t0 < C::TM * C::TN; t0 += 2) {
        const int t = t0 + (lane >> 5);
        if (t < C::TM * C::TN) {
            const int x = t / C::TN, y = t % C::TN;
            const int rr = (lane >> 1) & 15, hh = lane & 1;
            uint4 v = *reinterpret_cast<const uint4*>(ob + t * 256 + rr * 16 + hh * 8);
            const int row = mb + wm * C::WM + x * 16 + rr;
            const int col = nb + wn * C::WN + y * 16 + hh * 8;
            if (row < M) {
                uint16_t* dst = a.C + (size_t)row * N + col;
                const uint16_t* res = a.R ? a.R + (size_t)row * N + col : nullptr;
                const bool vec = vec_ok && col + 8 <= N && (!res || ((uintptr_t)a.R & 15) == 0);
                if (vec) {
                    if (res) {
                        // the residual add node, fused: fp16(fp16(acc) + r)
                        const uint4 rv = *reinterpret_cast<const uint4*>(res);
                        uint16_t* h = reinterpret_cast<uint16_t*>(&v);
                        const uint16_t* rh = reinterpret_cast<const uint16_t*>(&rv);
#pragma unroll
                        for (int i = 0; i < 8; i++) h[i] = hadd(h[i], rh[i]);
                    }
                    *reinterpret_cast<uint4*>(dst) = v;
                } else {
                    const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        if (col + i < N) dst[i] = res ? hadd(h[i], res[i]) : h[i];
                }
            }
        }
    }
}

template <class C>
static size_t lds_bytes() {
    return (size_t)C::NS * C::STAGE;
}

template <bool INT4, int WM, int WN, int WGM, int WGN, int KSUB>
static bool launch_lds(const GemmArgs& a, hipStream_t st) {
    using C = LdsCfg<INT4, WM, WN, WGM, WGN, KSUB>;
    if ((a.K / 32) % C::SG != 0) return false;
    const size_t lds = lds_bytes<C>();
    if (lds > 160 * 1024) return false;
    if (lds > 64 * 1024) {
        static const hipError_t attr = hipFuncSetAttribute((const void*)gemm_lds_kernel<C, INT4>,
                                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        if (attr != hipSuccess) {
            (void)hipGetLastError();   // leave no error behind; the register-streamed kernel runs instead
            return false;
        }
    }
    GemmArgs b = a;
    int gx = ceil_div(a.N, C::BN);
    for (int i = 0; i + 1 < a.np; i++) {
        b.bx[i] = gx;
        gx += ceil_div(a.Nx[i], C::BN);
    }
    const dim3 grid(gx, ceil_div(a.M, C::BM));
    hipLaunchKernelGGL((gemm_lds_kernel<C, INT4>), grid, dim3(C::NT), lds, st, b);
    return true;
}

// Workgroup tiles (wave tile, wave grid).  Each is scored by a rough time
// model: per CU, max(VALU cycles, DMA cycles) plus a quarter of the other,
// times the workgroups it runs in turn.  VALU: 2 instructions per output and group at ~7 cycles per
// instruction for one wave per SIMD, ~3.5 for two, ~2.4 for three; DMA: ~20
// bytes per cycle and CU (both measured on MI355X).
struct TileChoice {
    int wm, wn, wgm, wgn;
};
static constexpr TileChoice kTiles[] = {
    {16, 16, 1, 4},   // 16 x 64, 4 waves
    {16, 16, 2, 2},   // 32 x 32, 4 waves
    {16, 48, 4, 2},   // 64 x 96, 8 waves
    {16, 32, 4, 2},   // 64 x 64, 8 waves
    {32, 32, 2, 4},   // 64 x 128, 8 waves
    {16, 32, 4, 3},   // 64 x 96, 12 waves
};
static int pick_tile(const GemmArgs& a, bool int4) {
    constexpr double kCUs = 256.0;
    int best = 0;
    double best_t = 1e300;
    for (int i = 0; i < (int)(sizeof(kTiles) / sizeof(kTiles[0])); i++) {
        const TileChoice& t = kTiles[i];
        const int nw = t.wgm * t.wgn, bm = t.wm * t.wgm, bn = t.wn * t.wgn;
        int nblk = ceil_div(a.N, bn);
        for (int p = 0; p + 1 < a.np; p++) nblk += ceil_div(a.Nx[p], bn);
        const double wgs = (double)ceil_div(a.M, bm) * nblk;
        const double rounds = std::ceil(wgs / kCUs);
        const double waves_per_simd = nw / 4.0;
        const double cyc_per_instr = waves_per_simd >= 3 ? 2.4 : waves_per_simd >= 2 ? 3.5 : 7.0;
        const double valu = (double)bm * bn * (a.K / a.gs) * 2.0 / 64.0 / 4.0 * cyc_per_instr;
        const double dma = (double)(bm + (int4 ? bn / 2.0 : bn)) * a.K / 20.0;
        // the smaller of the two only partly overlaps the larger
        const double tt = rounds * (std::max(valu, dma) + 0.25 * std::min(valu, dma));
        if (tt < best_t * 0.999) {
            best_t = tt;
            best = i;
        }
    }
    return best;
}

template <bool INT4, int KSUB>
static bool launch_lds_ksub(const GemmArgs& a, hipStream_t st) {
    switch (pick_tile(a, INT4)) {
        case 0: return launch_lds<INT4, 16, 16, 1, 4, KSUB>(a, st);
        case 1: return launch_lds<INT4, 16, 16, 2, 2, KSUB>(a, st);
        case 2: return launch_lds<INT4, 16, 48, 4, 2, KSUB>(a, st);
        case 3: return launch_lds<INT4, 16, 32, 4, 2, KSUB>(a, st);
        case 4: return launch_lds<INT4, 32, 32, 2, 4, KSUB>(a, st);
        default: return launch_lds<INT4, 16, 32, 4, 3, KSUB>(a, st);
    }
}

template <bool INT4>
static bool launch_lds_any(const GemmArgs& a, hipStream_t st) {
    switch (a.gs / 32) {
        case 1: return launch_lds_ksub<INT4, 1>(a, st);
        case 2: return launch_lds_ksub<INT4, 2>(a, st);
        case 4: return launch_lds_ksub<INT4, 4>(a, st);
        default: return false;
    }
}

// ------------------------------------------------ activation scratch
static int gemm_scratch(hipStream_t st, size_t bytes, void** out) {
    return stream_scratch(SCR_GEMM_ACT, st, bytes, false, out);
}

// Rows from which the MFMA path pays off over the streaming GEMV.
constexpr size_t GEMM_MIN_M = 32;

// Returns *handled = false when the shape is left to the GEMV path.
// Activation codes ([M][K] int8, padded to 256 bytes) and row scales
// ([M] fp32) of the MFMA path with FP16 activations.
size_t gemm_act_scratch_bytes(size_t M, size_t K) { return ((M * K + 255) & ~(size_t)255) + M * sizeof(float); }

int gemm_grouped_mfma(const uint16_t* A16, const int8_t* A8, const float* As, const uint8_t* B,
                      const uint16_t* Bs, uint16_t* C, size_t M, size_t K, size_t N, size_t gs,
                      bool int4, hipStream_t st, bool* handled, const uint16_t* R, void* ext_scratch) {
    *handled = false;
    if (M < GEMM_MIN_M || gs % 32 != 0 || N < 32) return CACTUS_HIP_OK;
    if (((uintptr_t)B & 15) != 0) return CACTUS_HIP_OK;
    if (!A16 && (((uintptr_t)A8 & 15) != 0)) return CACTUS_HIP_OK;
    if (M >= (1u << 30) || N >= (1u << 30) || K >= (1u << 20)) return CACTUS_HIP_OK;
    const int8_t* Aq = A8;
    const float* Asc = As;
    if (A16) {
        // per-row quantization into scratch (bit-identical to the fused GEMV's)
        const size_t qbytes = (M * K + 255) & ~(size_t)255;
        void* scr = ext_scratch;
        if (!scr) {
            int rc = gemm_scratch(st, gemm_act_scratch_bytes(M, K), &scr);
            if (rc) return rc;
        }
        int rc;
        int8_t* q = static_cast<int8_t*>(scr);
        float* s = reinterpret_cast<float*>(static_cast<char*>(scr) + qbytes);
        rc = cactus_hip_quantize_activations(A16, q, s, M, K, st);
        if (rc) return rc;
        Aq = q;
        Asc = s;
    }
    GemmArgs a{Aq, Asc, B, Bs, C, (int)M, (int)K, (int)N, (int)gs, R};
    // the LDS path moves group scales as dwords
    const bool scales4 = ((uintptr_t)Bs & 3) == 0;
    if (scales4 && (int4 ? launch_lds_any<true>(a, st) : launch_lds_any<false>(a, st))) {
        *handled = true;
        return check_launch("grouped matmul (mfma, lds)");
    }
    // register-streamed fallback: two MFMA tiles per wave when the grid still fills the GPU
    const size_t mblk = ceil_div(M, 64);
    const bool wide = mblk * ceil_div(N, 128) >= 512;
    const dim3 grid((unsigned)ceil_div(N, wide ? 128 : 64), (unsigned)mblk);
    if (int4) {
        if (wide) hipLaunchKernelGGL((gemm_mfma_kernel<true, 2>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((gemm_mfma_kernel<true, 1>), grid, dim3(256), 0, st, a);
    } else {
        if (wide) hipLaunchKernelGGL((gemm_mfma_kernel<false, 2>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((gemm_mfma_kernel<false, 1>), grid, dim3(256), 0, st, a);
    }
    *handled = true;
    return check_launch("grouped matmul (mfma)");
}

// Matmuls of one pre-quantized activation against np weight matrices (same
// K, group size and format) in one launch of the LDS kernel.  Returns
// *handled = false when the shape is left to one launch per problem.
int gemm_grouped_mfma_multi(const int8_t* A8, const float* As, int np, const uint8_t* const* B,
                            const uint16_t* const* Bs, uint16_t* const* C, const size_t* N, size_t M, size_t K,
                            size_t gs, bool int4, hipStream_t st, bool* handled) {
    *handled = false;
    if (np < 1 || np > 3 || M < GEMM_MIN_M || gs % 32 != 0) return CACTUS_HIP_OK;
    if (((uintptr_t)A8 & 15) != 0 || M >= (1u << 30) || K >= (1u << 20)) return CACTUS_HIP_OK;
    for (int p = 0; p < np; p++)
        if (N[p] < 32 || N[p] >= (1u << 30) || ((uintptr_t)B[p] & 15) != 0 || ((uintptr_t)Bs[p] & 3) != 0)
            return CACTUS_HIP_OK;
    GemmArgs a{A8, As, B[0], Bs[0], C[0], (int)M, (int)K, (int)N[0], (int)gs, nullptr};
    a.np = np;
    for (int p = 1; p < np; p++) {
        a.Bx[p - 1] = B[p];
        a.Bsx[p - 1] = Bs[p];
        a.Cx[p - 1] = C[p];
        a.Nx[p - 1] = (int)N[p];
    }
    if (!(int4 ? launch_lds_any<true>(a, st) : launch_lds_any<false>(a, st))) return CACTUS_HIP_OK;
    *handled = true;
    return check_launch("grouped matmul (mfma, lds, several weights)");
}

}  // namespace cactus_hip

// ------------------------------------------------ no-allocation entry point
// Activation codes and row scales of cactus_hip_matmul_int8_f16act_noalloc
// live in this file-scope device array: each GPU the library runs on holds
// its own copy until the process ends.  Host code never passes the array's
// name to a kernel (on the host it names a stand-in, not device memory); it
// uses the device address hipGetSymbolAddress returns, looked up once per
// device with that device current.
namespace cactus_hip {

constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;   // 4 MiB
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_noalloc_mu;
static void* g_noalloc_ptr[kMaxDevices];

int grouped_dispatch(const uint16_t* A16, const int8_t* A8, const float* As, const uint8_t* B,
                     const uint16_t* Bs, uint16_t* C, size_t M, size_t K, size_t N, size_t gs, bool int4,
                     hipStream_t st, const uint16_t* R, void* ext_scratch);

static int noalloc_scratch(void** out) {
    int dev = 0;
    CH_HIP(hipGetDevice(&dev));
    CH_REQUIRE(dev >= 0 && dev < kMaxDevices, "matmul_int8_f16act_noalloc: device index above 63");
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(CACTUS_HIP_ERUNTIME, std::string("matmul_int8_f16act_noalloc: hipGetSymbolAddress(scratch): ") +
                                                 hipGetErrorString(e));
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return CACTUS_HIP_OK;
}

}  // namespace cactus_hip

extern "C" int cactus_hip_matmul_int8_f16act_noalloc(const uint16_t* A, const int8_t* B, const uint16_t* B_scales,
                                                     uint16_t* C, size_t M, size_t K, size_t N, size_t group_size,
                                                     void* stream) {
    using namespace cactus_hip;
    if (M == 0 || K == 0 || N == 0) return CACTUS_HIP_OK;
    const size_t need = gemm_act_scratch_bytes(M, K);
    if (need > kNoAllocScratchBytes)
        return fail(CACTUS_HIP_EINVAL, "matmul_int8_f16act_noalloc: M x K = " + std::to_string(M) + " x " +
                                           std::to_string(K) + " needs " + std::to_string(need) +
                                           " bytes of activation scratch, above the 4 MiB static buffer");
    void* scr = nullptr;
    const int rc = noalloc_scratch(&scr);
    if (rc) return rc;
    return grouped_dispatch(A, nullptr, nullptr, reinterpret_cast<const uint8_t*>(B), B_scales, C, M, K, N,
                            group_size, false, as_stream(stream), nullptr, scr);
}
