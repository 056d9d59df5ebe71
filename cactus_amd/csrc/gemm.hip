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

#include <map>
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
            if (col < N) a.C[(size_t)row * N + col] = f2h(r[s][e] * as);
        }
    }
}

// ------------------------------------------------ activation scratch
struct GemmScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
};
static std::mutex g_gemm_mu;
static std::map<std::pair<int, void*>, GemmScratch> g_gemm_scratch;

static int gemm_scratch(hipStream_t st, size_t bytes, void** out) {
    int dev = 0;
    CH_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_gemm_mu);
    GemmScratch& s = g_gemm_scratch[std::make_pair(dev, (void*)st)];
    if (s.bytes < bytes) {
        // the previous buffer is kept: kernels queued on the stream may use it
        const size_t want = bytes + bytes / 4;
        void* p = nullptr;
        CH_HIP(hipMalloc(&p, want));
        s.ptr = p;
        s.bytes = want;
    }
    *out = s.ptr;
    return CACTUS_HIP_OK;
}

// Rows from which the MFMA path pays off over the streaming GEMV.
constexpr size_t GEMM_MIN_M = 32;

// Returns *handled = false when the shape is left to the GEMV path.
int gemm_grouped_mfma(const uint16_t* A16, const int8_t* A8, const float* As, const uint8_t* B,
                      const uint16_t* Bs, uint16_t* C, size_t M, size_t K, size_t N, size_t gs,
                      bool int4, hipStream_t st, bool* handled) {
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
        void* scr = nullptr;
        int rc = gemm_scratch(st, qbytes + M * sizeof(float), &scr);
        if (rc) return rc;
        int8_t* q = static_cast<int8_t*>(scr);
        float* s = reinterpret_cast<float*>(static_cast<char*>(scr) + qbytes);
        rc = cactus_hip_quantize_activations(A16, q, s, M, K, st);
        if (rc) return rc;
        Aq = q;
        Asc = s;
    }
    GemmArgs a{Aq, Asc, B, Bs, C, (int)M, (int)K, (int)N, (int)gs};
    // two MFMA tiles per wave when the grid still fills the GPU
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

}  // namespace cactus_hip
