// lmhead.hip -- FP16 matmul with FP16 accumulation (a4) and the fused
// LM-head + greedy-sample path (a4 + a14).
//
// Reference arithmetic (kernel_gemm.cpp:17-126): for each output, eight fp16
// lanes; lane j accumulates k = j (mod 8) in increasing k with fp16 FMA; the
// result is ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) in fp16.
//
// Mapping: one lane owns one output row and keeps its eight chains as four
// packed halves (v_pk_fma_f16 does two chains per instruction).  A wave
// stages 64 rows x 64 k-values (8 KiB) through LDS with coalesced 16-byte
// loads, then every lane walks its own row out of LDS.  The activation row
// is broadcast from LDS.
#include "lm_device.h"

#include <map>
#include <mutex>

namespace cactus_hip {

struct LmArgs {
    const uint16_t* a;   // [M][K]
    const uint16_t* b;   // [N][K]
    uint16_t* c;         // [M][N] (may be null when only the argmax is wanted)
    int M, K, N;
    float* part_val;     // per-workgroup argmax partials (fused path)
    uint32_t* part_idx;
    uint32_t* counter;
    uint32_t* token;
};

template <bool ARGMAX>
__global__ void __launch_bounds__(LM_THREADS) f16_matmul_kernel(LmArgs p, int m0) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = p.K;
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int mr = min(LM_MR, p.M - m0);
    uint16_t* as = reinterpret_cast<uint16_t*>(smem);                       // [LM_MR][K]
    unsigned char* stage = smem + LM_MR * K * 2 + wid * LM_ROWS_PER_WAVE * LM_ROW_STRIDE;

    for (int i = threadIdx.x; i < mr * K; i += LM_THREADS) as[i] = p.a[(size_t)m0 * K + i];
    __syncthreads();

    const int row0 = (blockIdx.x * (LM_THREADS / 64) + wid) * LM_ROWS_PER_WAVE;
    const int my_row = row0 + lane;
    h2v acc[LM_MR][4];
#pragma unroll
    for (int m = 0; m < LM_MR; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[m][j] = (h2v){(f16)0.0f, (f16)0.0f};

    const int K16 = (K / 16) * 16;
    for (int k0 = 0; k0 < K16; k0 += LM_KC) {
        const int kc = min(LM_KC, K16 - k0);   // multiple of 16
        const int cpr = kc / 8;                // 16-byte chunks per row in this step
        // stage 64 rows x kc values: lane -> (row, chunk) coalesced
        for (int i = lane; i < LM_ROWS_PER_WAVE * cpr; i += 64) {
            const int r = i / cpr, ch = i % cpr;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row0 + r < p.N)
                v = *reinterpret_cast<const uint4*>(p.b + (size_t)(row0 + r) * K + k0 + ch * 8);
            *reinterpret_cast<uint4*>(stage + r * LM_ROW_STRIDE + ch * 16) = v;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int ch = 0; ch < cpr; ch++) {
            const uint4 bv = *reinterpret_cast<const uint4*>(stage + lane * LM_ROW_STRIDE + ch * 16);
#pragma unroll
            for (int m = 0; m < LM_MR; m++)
                if (m < mr) {
                    const uint4 av = *reinterpret_cast<const uint4*>(as + m * K + k0 + ch * 8);
                    f16_step(acc[m], av, bv);
                }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // K16..K8 step and the scalar tail (kernel_gemm.cpp:68-91), straight from global
    if (my_row < p.N) {
        const int K8 = (K / 8) * 8;
        const uint16_t* br = p.b + (size_t)my_row * K;
        for (int k = K16; k < K8; k += 8) {
            uint4 bv;
            bv.x = (uint32_t)br[k] | ((uint32_t)br[k + 1] << 16);
            bv.y = (uint32_t)br[k + 2] | ((uint32_t)br[k + 3] << 16);
            bv.z = (uint32_t)br[k + 4] | ((uint32_t)br[k + 5] << 16);
            bv.w = (uint32_t)br[k + 6] | ((uint32_t)br[k + 7] << 16);
#pragma unroll
            for (int m = 0; m < LM_MR; m++)
                if (m < mr) {
                    const uint16_t* ar = as + m * K + k;
                    uint4 av;
                    av.x = (uint32_t)ar[0] | ((uint32_t)ar[1] << 16);
                    av.y = (uint32_t)ar[2] | ((uint32_t)ar[3] << 16);
                    av.z = (uint32_t)ar[4] | ((uint32_t)ar[5] << 16);
                    av.w = (uint32_t)ar[6] | ((uint32_t)ar[7] << 16);
                    f16_step(acc[m], av, bv);
                }
        }
        for (int k = K8; k < K; k++) {
#pragma unroll
            for (int m = 0; m < LM_MR; m++)
                if (m < mr) {
                    // __fp16 promoted to float and contracted, rounded back to fp16
                    const float l0 = (float)acc[m][0].x;
                    const float r = __builtin_fmaf(h2f(as[m * K + k]), h2f(br[k]), l0);
                    acc[m][0].x = hbits(f2h(r));
                }
        }
    }
    float best = -__builtin_inff();
    uint32_t best_i = 0xFFFFFFFFu;
    if (my_row < p.N) {
#pragma unroll
        for (int m = 0; m < LM_MR; m++)
            if (m < mr) {
                const uint16_t r = f16_hsum(acc[m]);
                if (p.c) p.c[(size_t)(m0 + m) * p.N + my_row] = r;
                if (ARGMAX && m == 0) { best = h2f(r); best_i = (uint32_t)my_row; }
            }
    }
    if (ARGMAX) {
        // workgroup (max, first index), then the last workgroup reduces all
        __shared__ float bv_s[LM_THREADS];
        __shared__ uint32_t bi_s[LM_THREADS];
        __shared__ bool last;
        bv_s[threadIdx.x] = best;
        bi_s[threadIdx.x] = best_i;
        __syncthreads();
        for (int w = LM_THREADS / 2; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) {
                const float ov = bv_s[threadIdx.x + w];
                const uint32_t oi = bi_s[threadIdx.x + w];
                const float mv = bv_s[threadIdx.x];
                const uint32_t mi = bi_s[threadIdx.x];
                bool take = oi != 0xFFFFFFFFu &&
                            (mi == 0xFFFFFFFFu || ov > mv || (ov == mv && oi < mi));
                if (take) { bv_s[threadIdx.x] = ov; bi_s[threadIdx.x] = oi; }
            }
            __syncthreads();
        }
        if (threadIdx.x == 0) {
            p.part_val[blockIdx.x] = bv_s[0];
            p.part_idx[blockIdx.x] = bi_s[0];
            __threadfence();
            const uint32_t done = atomicAdd(p.counter, 1u);
            last = (done == gridDim.x - 1);
        }
        __syncthreads();
        if (last) {
            __threadfence();
            float bv = -__builtin_inff();
            uint32_t bi = 0xFFFFFFFFu;
            for (unsigned i = threadIdx.x; i < gridDim.x; i += LM_THREADS) {
                const float v = p.part_val[i];
                const uint32_t ix = p.part_idx[i];
                if (ix != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || v > bv || (v == bv && ix < bi))) {
                    bv = v; bi = ix;
                }
            }
            bv_s[threadIdx.x] = bv;
            bi_s[threadIdx.x] = bi;
            __syncthreads();
            for (int w = LM_THREADS / 2; w > 0; w >>= 1) {
                if ((int)threadIdx.x < w) {
                    const float ov = bv_s[threadIdx.x + w];
                    const uint32_t oi = bi_s[threadIdx.x + w];
                    const float mv = bv_s[threadIdx.x];
                    const uint32_t mi = bi_s[threadIdx.x];
                    bool take = oi != 0xFFFFFFFFu &&
                                (mi == 0xFFFFFFFFu || ov > mv || (ov == mv && oi < mi));
                    if (take) { bv_s[threadIdx.x] = ov; bi_s[threadIdx.x] = oi; }
                }
                __syncthreads();
            }
            if (threadIdx.x == 0) {
                *p.token = bi_s[0] == 0xFFFFFFFFu ? 0u : bi_s[0];
                *p.counter = 0u;  // leave the counter ready for the next call
            }
        }
    }
}

// Any-K / any-alignment form: one thread per output, scalar loads, same
// lane order and final tree.
__global__ void f16_matmul_scalar_kernel(const uint16_t* __restrict__ a,
                                         const uint16_t* __restrict__ b, uint16_t* __restrict__ c,
                                         int M, int K, int N) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)M * N) return;
    const int m = (int)(t / N), n = (int)(t % N);
    const uint16_t* ar = a + (size_t)m * K;
    const uint16_t* br = b + (size_t)n * K;
    h2v acc[4];
    for (int j = 0; j < 4; j++) acc[j] = (h2v){(f16)0.0f, (f16)0.0f};
    const int K8 = (K / 8) * 8;
    for (int k = 0; k < K8; k += 8) {
        uint4 av, bv;
        av.x = (uint32_t)ar[k] | ((uint32_t)ar[k + 1] << 16);
        av.y = (uint32_t)ar[k + 2] | ((uint32_t)ar[k + 3] << 16);
        av.z = (uint32_t)ar[k + 4] | ((uint32_t)ar[k + 5] << 16);
        av.w = (uint32_t)ar[k + 6] | ((uint32_t)ar[k + 7] << 16);
        bv.x = (uint32_t)br[k] | ((uint32_t)br[k + 1] << 16);
        bv.y = (uint32_t)br[k + 2] | ((uint32_t)br[k + 3] << 16);
        bv.z = (uint32_t)br[k + 4] | ((uint32_t)br[k + 5] << 16);
        bv.w = (uint32_t)br[k + 6] | ((uint32_t)br[k + 7] << 16);
        f16_step(acc, av, bv);
    }
    for (int k = K8; k < K; k++) {
        const float r = __builtin_fmaf(h2f(ar[k]), h2f(br[k]), (float)acc[0].x);
        acc[0].x = hbits(f2h(r));
    }
    c[t] = f16_hsum(acc);
}

// ------------------------------------------------ per-(device, stream) scratch
// one buffer: the completion counter (zeroed when the buffer is made; the
// last workgroup of every call leaves it at zero), then the per-workgroup
// partial maxima and their indices
struct LmScratch {
    float* val = nullptr;
    uint32_t* idx = nullptr;
    uint32_t* counter = nullptr;
};

static int lm_scratch(void* stream, size_t blocks, LmScratch* out) {
    void* p = nullptr;
    int rc = stream_scratch(SCR_LM, stream, 256 + 8 * blocks, true, &p);
    if (rc) return rc;
    out->counter = static_cast<uint32_t*>(p);
    out->val = reinterpret_cast<float*>(static_cast<char*>(p) + 256);
    out->idx = reinterpret_cast<uint32_t*>(out->val + blocks);
    return CACTUS_HIP_OK;
}

static size_t lm_smem(int K) {
    return (size_t)LM_MR * K * 2 + (size_t)(LM_THREADS / 64) * LM_ROWS_PER_WAVE * LM_ROW_STRIDE;
}

// kernels needing more than the default 64 KiB of dynamic LDS (large K) raise
// their limit once, to exactly what the largest supported K needs
static int lm_prepare(size_t smem) {
    if (smem <= 64 * 1024) return CACTUS_HIP_OK;
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        const int need = (int)lm_smem(LM_MAX_K);
        err = hipFuncSetAttribute((const void*)f16_matmul_kernel<false>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, need);
        if (err == hipSuccess)
            err = hipFuncSetAttribute((const void*)f16_matmul_kernel<true>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, need);
    });
    if (err != hipSuccess)
        return fail(CACTUS_HIP_ERUNTIME, std::string("hipFuncSetAttribute: ") + hipGetErrorString(err));
    return CACTUS_HIP_OK;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_matmul_f16(const uint16_t* a, const uint16_t* b_transposed, uint16_t* c, size_t M,
                          size_t K, size_t N, void* stream) {
    if (M == 0 || N == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(a && b_transposed && c, "matmul_f16: null pointer");
    CH_REQUIRE(K <= (size_t)LM_MAX_K, "matmul_f16: K > 8192 not supported");
    CH_REQUIRE(M < (1u << 30) && N < (1u << 30), "matmul_f16: shape too large");
    if (((uintptr_t)b_transposed & 15) != 0 || K % 8 != 0 || ((uintptr_t)a & 15) != 0) {
        const size_t outs = M * N;
        hipLaunchKernelGGL(f16_matmul_scalar_kernel, dim3(ceil_div(outs, 256)), dim3(256), 0,
                           as_stream(stream), a, b_transposed, c, (int)M, (int)K, (int)N);
        return check_launch("matmul_f16");
    }
    int rc0 = lm_prepare(lm_smem((int)K));
    if (rc0) return rc0;
    LmArgs p{};
    p.a = a; p.b = b_transposed; p.c = c; p.M = (int)M; p.K = (int)K; p.N = (int)N;
    const unsigned blocks = ceil_div(N, (LM_THREADS / 64) * LM_ROWS_PER_WAVE);
    for (size_t m0 = 0; m0 < M; m0 += LM_MR) {
        hipLaunchKernelGGL(f16_matmul_kernel<false>, dim3(blocks), dim3(LM_THREADS), lm_smem((int)K),
                           as_stream(stream), p, (int)m0);
        int rc = check_launch("matmul_f16");
        if (rc) return rc;
    }
    return CACTUS_HIP_OK;
}

int cactus_hip_lm_head_argmax_f16(const uint16_t* a, const uint16_t* b_transposed,
                                  uint16_t* logits, uint32_t* token, size_t K, size_t N,
                                  void* stream) {
    CH_REQUIRE(token, "lm_head_argmax: null token pointer");
    if (N == 0) return cactus_hip_memset(token, 0, 4, stream);
    CH_REQUIRE(a && b_transposed, "lm_head_argmax: null pointer");
    CH_REQUIRE(K <= (size_t)LM_MAX_K, "lm_head_argmax: K > 8192 not supported");
    CH_REQUIRE(N < (1u << 30), "lm_head_argmax: N too large");
    CH_REQUIRE(((uintptr_t)b_transposed & 15) == 0 && K % 8 == 0,
               "lm_head_argmax: b must be 16-byte aligned with K a multiple of 8");
    const unsigned blocks = ceil_div(N, (LM_THREADS / 64) * LM_ROWS_PER_WAVE);
    int rc = lm_prepare(lm_smem((int)K));
    if (rc) return rc;
    LmScratch s;
    rc = lm_scratch(stream, blocks, &s);
    if (rc) return rc;
    LmArgs p{};
    p.a = a; p.b = b_transposed; p.c = logits; p.M = 1; p.K = (int)K; p.N = (int)N;
    p.part_val = s.val; p.part_idx = s.idx; p.counter = s.counter; p.token = token;
    hipLaunchKernelGGL(f16_matmul_kernel<true>, dim3(blocks), dim3(LM_THREADS), lm_smem((int)K),
                       as_stream(stream), p, 0);
    return check_launch("lm_head_argmax");
}

}  // extern "C"
