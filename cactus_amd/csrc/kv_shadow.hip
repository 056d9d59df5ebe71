// kv_shadow.hip -- fp32 value-product tiles mirroring the INT8 value cache.
//
// The hybrid attention accumulates, per cached key, (float)code * scale
// rounded to fp32 (kernel_attention.cpp:424-441).  The decode path keeps
// those products precomputed in HBM, laid out as the value chains load them
// into registers (hip_common.h, sh_index):
//
//   [kv head][64-dim slice][key / 4][64 dims][4 keys]
//
// The INT8 cache stays the reference state; the tiles are derived data,
// rewritten whenever keys are appended (prefill chunks here, decode steps in
// decode.hip).  Batch 1.
#include "hip_common.h"
#include "quant_device.h"

#include <algorithm>

namespace cactus_hip {

constexpr int KS_T = SH_TILE_KEYS;

__global__ void kv_shadow_kernel(const int8_t* __restrict__ vc, const float* __restrict__ vs,
                                 float* __restrict__ sh, size_t start, int Hkv, int d, int qgs,
                                 size_t ntile) {
    const size_t key = start + blockIdx.x;
    const int kvh = blockIdx.y;
    const int nqg = (d + 127) / 128;
    const int da = (d / 8) * 8, nsl = (d + 63) / 64;
    const size_t off = key * Hkv + kvh;
    for (int dim = threadIdx.x; dim < nsl * 64; dim += blockDim.x) {
        float p = 0.0f;
        if (dim < da) p = (float)vc[off * d + dim] * vs[off * nqg + ((dim / 8) * 8) / qgs];
        sh[sh_index(kvh, nsl, dim / 64, ntile, key, dim % 64)] = p;
    }
}

// ---------------------------------------------------------------- window shift
// Moving cached tokens [src, src + count) to [dst, dst + count) in every
// layer (the sliding window's memmove, engine_cache.cpp:268-306).  The
// ranges may overlap, so the move goes through `temp` in two launches: the
// first copies the source tokens out, the second writes them to their new
// slots and recomputes their value products with kv_shadow_kernel's
// expression.  Grid (count, layers); a workgroup moves one token of one
// layer: Hkv*d code bytes and Hkv*ng scales for keys and for values.
struct KvLayer {
    int8_t* k;
    int8_t* v;
    float* ks;
    float* vs;
    float* sh;
};

__global__ void kv_shift_out_kernel(const KvLayer* __restrict__ layers, unsigned char* __restrict__ temp,
                                    size_t src, int Hkv, int d, size_t count) {
    const KvLayer L = layers[blockIdx.y];
    const size_t i = blockIdx.x;
    const int nqg = (d + 127) / 128;
    const size_t cb = (size_t)Hkv * d, sb = (size_t)Hkv * nqg;
    unsigned char* t = temp + ((size_t)blockIdx.y * count + i) * (2 * cb + 2 * sb * 4);
    const size_t tok = src + i;
    for (size_t j = threadIdx.x; j < cb; j += blockDim.x) {
        t[j] = (unsigned char)L.k[tok * cb + j];
        t[cb + j] = (unsigned char)L.v[tok * cb + j];
    }
    float* ts = reinterpret_cast<float*>(t + 2 * cb);
    for (size_t j = threadIdx.x; j < sb; j += blockDim.x) {
        ts[j] = L.ks[tok * sb + j];
        ts[sb + j] = L.vs[tok * sb + j];
    }
}

__global__ void kv_shift_in_kernel(const KvLayer* __restrict__ layers, const unsigned char* __restrict__ temp,
                                   size_t dst, int Hkv, int d, size_t count, size_t ntile, uint32_t* state,
                                   uint32_t cache_len) {
    const KvLayer L = layers[blockIdx.y];
    const size_t i = blockIdx.x;
    const int nqg = (d + 127) / 128;
    const size_t cb = (size_t)Hkv * d, sb = (size_t)Hkv * nqg;
    const unsigned char* t = temp + ((size_t)blockIdx.y * count + i) * (2 * cb + 2 * sb * 4);
    const float* ts = reinterpret_cast<const float*>(t + 2 * cb);
    const size_t key = dst + i;
    for (size_t j = threadIdx.x; j < cb; j += blockDim.x) {
        L.k[key * cb + j] = (int8_t)t[j];
        L.v[key * cb + j] = (int8_t)t[cb + j];
    }
    for (size_t j = threadIdx.x; j < sb; j += blockDim.x) {
        L.ks[key * sb + j] = ts[j];
        L.vs[key * sb + j] = ts[sb + j];
    }
    if (L.sh) {
        // products from the moved codes and scales (same expression and
        // layout as kv_shadow_kernel)
        const int da = (d / 8) * 8, nsl = (d + 63) / 64;
        for (int x = threadIdx.x; x < Hkv * nsl * 64; x += blockDim.x) {
            const int kvh = x / (nsl * 64), dim = x % (nsl * 64);
            float p = 0.0f;
            if (dim < da)
                p = (float)(int8_t)t[cb + (size_t)kvh * d + dim] * ts[sb + (size_t)kvh * nqg + ((dim / 8) * 8) / 128];
            L.sh[sh_index(kvh, nsl, dim / 64, ntile, key, dim % 64)] = p;
        }
    }
    if (state && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) state[2] = cache_len;
}

// ---------------------------------------------------------------- append
// New K/V rows of every layer into the cache in one launch: grid (tokens,
// layers, unit slices), 256 threads.  Wave w of slice z takes the (K or V,
// head, 128-group) units 4 z + w, 4 z + w + 4 Z, ... (one each when Z
// covers them: their load -> max -> store chains run side by side in
// separate workgroups); each unit is quantized as
// quantize_kv_kernel does it (group max, scale, codes: body rne-saturating,
// tail roundf), and a value unit also writes its products (float)code *
// scale into the tile layout of kv_shadow_kernel.
constexpr int KV_APPEND_MAX_LAYERS = 64;
struct KvAppendSrc {
    const uint16_t* k[KV_APPEND_MAX_LAYERS];
    const uint16_t* v[KV_APPEND_MAX_LAYERS];
};

__global__ void __launch_bounds__(256) kv_append_kernel(const KvLayer* __restrict__ layers, KvAppendSrc src,
                                                        size_t at, int Hkv, int d, size_t ntile) {
    const int l = blockIdx.y;
    const KvLayer L = layers[l];
    const size_t i = blockIdx.x, key = at + i;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ng = (d + 127) / 128, nsl = (d + 63) / 64;
    const int units = Hkv * ng;
    for (int w = wave + 4 * (int)blockIdx.z; w < 2 * units; w += 4 * (int)gridDim.z) {
        const bool isv = w >= units;
        const int hg = isv ? w - units : w, h = hg / ng, g = hg % ng;
        const int g0 = g * 128, cnt = min(128, d - g0);
        const uint16_t* x = (isv ? src.v[l] : src.k[l]) + (i * Hkv + h) * d + g0;
        int8_t* o = (isv ? L.v : L.k) + (key * Hkv + h) * d + g0;
        float m = 0.0f;
        for (int j = lane; j < cnt; j += 64) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(x[j])));
        m = wave_max(m);
        const float sc = row_scale_from_max(m);
        const float inv = 1.0f / sc;
        const int body = (cnt / 8) * 8;
        for (int j = lane; j < cnt; j += 64) {
            const float v = h2f(x[j]) * inv;
            const int32_t c = (j < body) ? cvt_rne_sat(v) : (int32_t)__builtin_roundf(v);
            const int8_t code = (int8_t)sat8(c);
            o[j] = code;
            if (isv && L.sh) {
                const int dim = g0 + j;
                L.sh[sh_index(h, nsl, dim / 64, ntile, key, dim % 64)] = (float)code * sc;
            }
        }
        if (lane == 0) (isv ? L.vs : L.ks)[(key * Hkv + h) * ng + g] = sc;
    }
    // product rows of the padding dimensions [d, 64 nsl) hold zeros
    const int pad = nsl * 64 - d;
    if (L.sh && pad > 0 && blockIdx.z == 0)
        for (int x = threadIdx.x; x < Hkv * pad; x += blockDim.x) {
            const int h = x / pad, dim = d + x % pad;
            L.sh[sh_index(h, nsl, dim / 64, ntile, key, dim % 64)] = 0.0f;
        }
}

__global__ void kv_set_len_kernel(uint32_t* state, uint32_t cache_len) {
    if (threadIdx.x == 0) state[2] = cache_len;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_kv_shadow_bytes(size_t max_seq, size_t kv_heads, size_t head_dim, size_t* bytes) {
    CH_REQUIRE(bytes, "kv_shadow_bytes: null");
    const size_t ntile = (max_seq + KS_T - 1) / KS_T;
    *bytes = kv_heads * ((head_dim + 63) / 64) * sh_region_floats(ntile) * sizeof(float);
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

int cactus_hip_kv_append_layers(const cactus_hip_kv_layer* layers, const uint16_t* const* k_rows,
                                const uint16_t* const* v_rows, size_t nlayers, size_t count, size_t at,
                                size_t kv_heads, size_t head_dim, size_t group_size, size_t max_seq,
                                void* stream) {
    if (count == 0 || nlayers == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(layers && k_rows && v_rows, "kv_append_layers: null pointer");
    CH_REQUIRE(head_dim % 8 == 0 && head_dim > 0 && head_dim <= 256 && group_size == 128,
               "kv_append_layers: head_dim must be a multiple of 8 (<= 256), group size 128");
    CH_REQUIRE(kv_heads > 0 && kv_heads <= 4096 && count < (1u << 31) && nlayers < 65536,
               "kv_append_layers: bad sizes");
    CH_REQUIRE(at + count <= max_seq, "kv_append_layers: keys beyond the cache capacity");
    const size_t ntile = (max_seq + KS_T - 1) / KS_T;
    const KvLayer* L = reinterpret_cast<const KvLayer*>(layers);
    for (size_t l0 = 0; l0 < nlayers; l0 += KV_APPEND_MAX_LAYERS) {
        const size_t nl = std::min<size_t>(KV_APPEND_MAX_LAYERS, nlayers - l0);
        KvAppendSrc src{};
        for (size_t l = 0; l < nl; l++) {
            CH_REQUIRE(k_rows[l0 + l] && v_rows[l0 + l], "kv_append_layers: null row pointer");
            src.k[l] = k_rows[l0 + l];
            src.v[l] = v_rows[l0 + l];
        }
        // one unit per wave: 2 * kv_heads * groups units over slices of 4
        const unsigned slices = (unsigned)((2 * kv_heads * ((head_dim + 127) / 128) + 3) / 4);
        hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)count, (unsigned)nl, slices), dim3(256), 0,
                           as_stream(stream), L + l0, src, at, (int)kv_heads, (int)head_dim, ntile);
        const int rc = check_launch("kv_append_layers");
        if (rc) return rc;
    }
    return CACTUS_HIP_OK;
}

static size_t kv_shift_token_bytes(size_t kv_heads, size_t head_dim) {
    const size_t nqg = (head_dim + 127) / 128;
    return 2 * kv_heads * head_dim + 2 * kv_heads * nqg * sizeof(float);
}

int cactus_hip_kv_shift_temp_bytes(size_t nlayers, size_t count, size_t kv_heads, size_t head_dim,
                                   size_t* bytes) {
    CH_REQUIRE(bytes, "kv_shift_temp_bytes: null");
    *bytes = nlayers * count * kv_shift_token_bytes(kv_heads, head_dim);
    return CACTUS_HIP_OK;
}

int cactus_hip_kv_window_shift(const cactus_hip_kv_layer* layers, size_t nlayers, size_t kv_heads,
                               size_t head_dim, size_t max_seq, size_t dst, size_t src, size_t count,
                               void* temp, size_t temp_bytes, uint32_t* state, uint32_t cache_len,
                               void* stream) {
    static_assert(sizeof(cactus_hip_kv_layer) == sizeof(KvLayer), "layer record layout");
    CH_REQUIRE(layers || count == 0, "kv_window_shift: null layer table");
    CH_REQUIRE(head_dim % 8 == 0 && head_dim <= 256 && kv_heads > 0 && kv_heads * head_dim <= (1u << 20),
               "kv_window_shift: head_dim must be a multiple of 8 (<= 256)");
    CH_REQUIRE(nlayers < 65536 && count < (1u << 31), "kv_window_shift: bad sizes");
    CH_REQUIRE(dst <= src, "kv_window_shift: tokens move towards the start only");
    CH_REQUIRE(src + count <= max_seq && dst + count <= max_seq, "kv_window_shift: tokens beyond the cache");
    if (count == 0 || nlayers == 0) {
        if (!state) return CACTUS_HIP_OK;
        hipLaunchKernelGGL(kv_set_len_kernel, dim3(1), dim3(64), 0, as_stream(stream), state, cache_len);
        return check_launch("kv_window_shift");
    }
    CH_REQUIRE(temp && temp_bytes >= nlayers * count * kv_shift_token_bytes(kv_heads, head_dim),
               "kv_window_shift: temp buffer too small (cactus_hip_kv_shift_temp_bytes)");
    const size_t ntile = (max_seq + KS_T - 1) / KS_T;
    const KvLayer* L = reinterpret_cast<const KvLayer*>(layers);
    const dim3 grid((unsigned)count, (unsigned)nlayers);
    hipLaunchKernelGGL(kv_shift_out_kernel, grid, dim3(256), 0, as_stream(stream), L,
                       static_cast<unsigned char*>(temp), src, (int)kv_heads, (int)head_dim, count);
    int rc = check_launch("kv_window_shift (out)");
    if (rc) return rc;
    hipLaunchKernelGGL(kv_shift_in_kernel, grid, dim3(256), 0, as_stream(stream), L,
                       static_cast<const unsigned char*>(temp), dst, (int)kv_heads, (int)head_dim, count, ntile,
                       state, cache_len);
    return check_launch("kv_window_shift (in)");
}

}  // extern "C"
