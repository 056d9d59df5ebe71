// kv_shadow.hip -- fp32 value-product tiles mirroring the INT8 value cache.
//
// The hybrid attention accumulates, per cached key, (float)code * scale
// rounded to fp32 (kernel_attention.cpp:424-441).  The decode path keeps
// those products precomputed in HBM, laid out as the value chains read them
// from LDS, so that staging a tile is a plain memory copy (LDS DMA):
//
//   [kv head][64-dim slice][64-key tile][64 dims][68 keys]   (4 keys padding)
//
// The INT8 cache stays the reference state; the tiles are derived data,
// rewritten whenever keys are appended (prefill chunks here, decode steps in
// decode.hip).  Batch 1.
#include "hip_common.h"

namespace cactus_hip {

constexpr int KS_T = 64;
constexpr int KS_PS = 68;

__global__ void kv_shadow_kernel(const int8_t* __restrict__ vc, const float* __restrict__ vs,
                                 float* __restrict__ sh, size_t start, int Hkv, int d, int qgs,
                                 size_t ntile) {
    const size_t key = start + blockIdx.x;
    const int kvh = blockIdx.y;
    const int nqg = (d + 127) / 128;
    const int da = (d / 8) * 8, nsl = (d + 63) / 64;
    const size_t off = key * Hkv + kvh;
    const size_t t = key / KS_T;
    const int j = (int)(key % KS_T);
    for (int dim = threadIdx.x; dim < nsl * 64; dim += blockDim.x) {
        float p = 0.0f;
        if (dim < da) p = (float)vc[off * d + dim] * vs[off * nqg + ((dim / 8) * 8) / qgs];
        const int sl = dim / 64, dl = dim % 64;
        sh[(((size_t)kvh * nsl + sl) * ntile + t) * (KS_T * KS_PS) + dl * KS_PS + j] = p;
    }
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_kv_shadow_bytes(size_t max_seq, size_t kv_heads, size_t head_dim, size_t* bytes) {
    CH_REQUIRE(bytes, "kv_shadow_bytes: null");
    const size_t ntile = (max_seq + KS_T - 1) / KS_T;
    *bytes = kv_heads * ((head_dim + 63) / 64) * ntile * (size_t)(KS_T * KS_PS) * sizeof(float);
    return CACTUS_HIP_OK;
}

int cactus_hip_kv_shadow_update(const int8_t* v_cache, const float* v_scales, float* shadow, size_t start,
                                size_t count, size_t kv_heads, size_t head_dim, size_t quant_group_size,
                                size_t max_seq, void* stream) {
    if (count == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(v_cache && v_scales && shadow, "kv_shadow_update: null pointer");
    CH_REQUIRE(head_dim % 8 == 0 && head_dim <= 256 && quant_group_size == 128,
               "kv_shadow_update: head_dim must be a multiple of 8 (<= 256), group size 128");
    CH_REQUIRE(start + count <= max_seq, "kv_shadow_update: keys beyond the cache capacity");
    CH_REQUIRE(kv_heads > 0 && kv_heads < 65536 && count < (1u << 31), "kv_shadow_update: bad sizes");
    const size_t ntile = (max_seq + KS_T - 1) / KS_T;
    hipLaunchKernelGGL(kv_shadow_kernel, dim3((unsigned)count, (unsigned)kv_heads), dim3(128), 0,
                       as_stream(stream), v_cache, v_scales, shadow, start, (int)kv_heads, (int)head_dim,
                       (int)quant_group_size, ntile);
    return check_launch("kv_shadow_update");
}

}  // extern "C"
