// elementwise.hip -- RMSNorm (a8), RoPE (a9), softmax (a10), SiLU (a11),
// fp16 add/multiply (a12) and the embedding gather (a13).
#include "decode_device.h"
#include "hip_common.h"

#include <cmath>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace cactus_hip {

// ---------------------------------------------------------------- RMSNorm
// One wave per row.  The row is staged in LDS; lanes 0..15 each run one of
// the reference's 16 fp32 FMA chains (element i -> chain i mod 16, i.e.
// accumulator (i%16)/4, lane i%4, kernel_attention.cpp:500-523), which are
// combined as ((v0+v1)+v2)+v3 per lane and then (l0+l1)+(l2+l3) (:525-530).
// Output: y = fp16(fp16(x * fp16(1/rms)) * w) on the 8-aligned prefix.
constexpr int RMS_MAX_DIMS = 8192;

__global__ void __launch_bounds__(256) rms_norm_kernel(const uint16_t* __restrict__ X,
                                                       const uint16_t* __restrict__ W,
                                                       uint16_t* __restrict__ Y, size_t rows,
                                                       int dims, float eps) {
    extern __shared__ __align__(16) uint16_t srow[];
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t row = (size_t)blockIdx.x * 4 + wid;
    uint16_t* xs = srow + wid * dims;
    const bool active = row < rows;
    const uint16_t* x = X + row * dims;
    if (active)
        for (int i = lane; i < dims; i += 64) xs[i] = x[i];
    __syncthreads();
    float ss = 0.0f;
    float chain = 0.0f;
    const int n16 = dims / 16;
    const int end8 = (dims / 8) * 8;
    if (active && lane < 16) {
        for (int i = 0; i < n16; i++) {
            const float a = h2f(xs[i * 16 + lane]);
            chain = __builtin_fmaf(a, a, chain);
        }
        if (lane < 8 && n16 * 16 + 8 <= dims) {
            const float a = h2f(xs[n16 * 16 + lane]);
            chain = __builtin_fmaf(a, a, chain);
        }
    }
    const float c4 = __shfl(chain, (lane + 4) & 63, 64);
    const float c8 = __shfl(chain, (lane + 8) & 63, 64);
    const float c12 = __shfl(chain, (lane + 12) & 63, 64);
    const float t = ((chain + c4) + c8) + c12;
    const float t1 = __shfl(t, 1, 64), t2 = __shfl(t, 2, 64), t3 = __shfl(t, 3, 64);
    const float t0 = __shfl(t, 0, 64);
    ss = (t0 + t1) + (t2 + t3);
    for (int k = end8; k < dims; k++) {
        const float a = h2f(xs[k]);
        ss = __builtin_fmaf(a, a, ss);
    }
    const float rms = __builtin_sqrtf(ss / (float)dims + eps);
    const float inv = 1.0f / rms;
    const uint16_t hinv = f2h(inv);
    if (active) {
        uint16_t* y = Y + row * dims;
        for (int i = lane; i < dims; i += 64) {
            if (i < end8) y[i] = hmul(hmul(xs[i], hinv), W[i]);
            else y[i] = f2h((h2f(xs[i]) * inv) * h2f(W[i]));
        }
    }
}

// ---------------------------------------------------------------- RoPE
// RopeTable is declared in hip_common.h
static std::mutex g_rope_mu;
static std::map<std::tuple<int, size_t, uint32_t>, RopeTable> g_rope;

// Table of precompute_rope_tables_f16 (kernel_attention.cpp:588-612), built
// on the host with the host libm and uploaded.  Tables only grow; a replaced
// table stays allocated because queued kernels may still read it.
int rope_table(size_t npos, size_t d, float theta, RopeTable* out) {
    int dev = 0;
    CH_HIP(hipGetDevice(&dev));
    uint32_t tb;
    memcpy(&tb, &theta, 4);
    std::lock_guard<std::mutex> lk(g_rope_mu);
    RopeTable& t = g_rope[std::make_tuple(dev, d, tb)];
    if (t.npos < npos) {
        size_t want = t.npos * 2 > npos ? t.npos * 2 : npos;
        if (want < 256) want = 256;
        const size_t half = d / 2;
        std::vector<uint16_t> hc(want * half), hs(want * half);
        for (size_t p = 0; p < want; p++) {
            const float pf = (float)p;
            for (size_t i = 0; i < half; i++) {
                const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)d);
                const float ang = pf * freq;
                const float c = cosf(ang), s = sinf(ang);
                hc[p * half + i] = host_f2h(c);
                hs[p * half + i] = host_f2h(s);
            }
        }
        RopeTable nt;
        CH_HIP(hipMalloc(&nt.cos_d, hc.size() * 2 + 2));
        CH_HIP(hipMalloc(&nt.sin_d, hs.size() * 2 + 2));
        CH_HIP(hipMemcpy(nt.cos_d, hc.data(), hc.size() * 2, hipMemcpyHostToDevice));
        CH_HIP(hipMemcpy(nt.sin_d, hs.data(), hs.size() * 2, hipMemcpyHostToDevice));
        nt.npos = want;
        t = nt;  // previous buffers intentionally kept (see above)
    }
    *out = t;
    return CACTUS_HIP_OK;
}

__global__ void rope_kernel(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
                            const uint16_t* __restrict__ ct, const uint16_t* __restrict__ st,
                            size_t total_pairs, int S, int H, int d, size_t start_pos) {
    const int half = d / 2;
    const int vh = (half / 8) * 8;
    for (size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x; p < total_pairs;
         p += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(p % half);
        const size_t rowi = p / half;               // (b*S + s)*H + h
        const int s = (int)((rowi / H) % S);
        const size_t off = rowi * d;
        const size_t toff = (start_pos + s) * half + i;
        const uint16_t c = ct[toff], sn = st[toff];
        const uint16_t x1 = X[off + i], x2 = X[off + i + half];
        if (i < vh) {
            Y[off + i] = hfma(x2 ^ 0x8000u, sn, hmul(x1, c));
            Y[off + i + half] = hfma(x1, sn, hmul(x2, c));
        } else {
            const float a = h2f(x1), b = h2f(x2), cf = h2f(c), sf = h2f(sn);
            Y[off + i] = f2h(a * cf - b * sf);
            Y[off + i + half] = f2h(b * cf + a * sf);
        }
    }
}

// ---------------------------------------------------------------- softmax
// One workgroup per row.  Max is order-free; the sum runs the reference's
// 32 fp32 chains (element i -> sum_vec[(i%32)/4] lane i%4, kernel_nn.cpp:
// 191-214), combined sequentially over the 8 vectors then pairwise over lanes.
__global__ void __launch_bounds__(256) softmax_kernel(const uint16_t* __restrict__ X,
                                                      uint16_t* __restrict__ Y, int V) {
    __shared__ float red[4];
    __shared__ float chains[32];
    const size_t row = blockIdx.x;
    const uint16_t* x = X + row * (size_t)V;
    uint16_t* y = Y + row * (size_t)V;
    const int tid = threadIdx.x;
    float m = -__builtin_inff();
    for (int i = tid; i < V; i += 256) m = __builtin_fmaxf(m, h2f(x[i]));
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const int vv = (V / 32) * 32;
    for (int i = tid; i < vv; i += 256) y[i] = f2h(fast_exp(h2f(x[i]) - mx));
    for (int i = vv + tid; i < V; i += 256) y[i] = f2h(cactus_expf(h2f(x[i]) - mx));
    if (tid < 32) {
        float s = 0.0f;
        for (int i = tid; i < vv; i += 32) s = s + fast_exp(h2f(x[i]) - mx);
        chains[tid] = s;
    }
    __syncthreads();
    float sum = 0.0f;
    {
        float t[4];
        for (int l = 0; l < 4; l++) {
            float a = chains[l];
            for (int u = 1; u < 8; u++) a = a + chains[u * 4 + l];
            t[l] = a;
        }
        sum = (t[0] + t[1]) + (t[2] + t[3]);
        for (int i = vv; i < V; i++) sum = sum + cactus_expf(h2f(x[i]) - mx);
    }
    const float inv = 1.0f / sum;
    const uint16_t hinv = f2h(inv);
    __syncthreads();  // all fp16 exps written before they are rescaled
    for (int i = tid; i < vv; i += 256) y[i] = hmul(y[i], hinv);
    for (int i = vv + tid; i < V; i += 256) y[i] = f2h(h2f(y[i]) * inv);
}

// ---------------------------------------------------------------- SiLU, add, mul
// The per-head RMSNorm of q and k (the q_norm / k_norm nodes,
// kernel_attention.cpp:484-563) followed by RoPE (:565-676) at the rows'
// positions: one wave per (token, head) row.  Every global load of a row --
// its values, the norm weights, the two table entries of each pair -- is
// issued up front (clamped indices, no branches), so the wave waits for
// memory once; the row and its normalized values pass through LDS for the
// RMS chains and the pairing.  Up to two problems (q and k) per launch:
// workgroups from nblk0 on take problem 1.  The same results as
// cactus_hip_rms_norm_f16 then cactus_hip_rope_f16.
struct RopeRowsArgs {
    const uint16_t* X[2];
    const uint16_t* W[2];
    uint16_t* Y[2];
    size_t rows[2];
    int H[2];
    int nblk0;
    const uint16_t* ct;
    const uint16_t* stb;
    int S, d;
    size_t start_pos;
    float eps;
};

__global__ void __launch_bounds__(256) rms_rope_rows_kernel(RopeRowsArgs a) {
    __shared__ uint16_t buf[4][2][256];
    constexpr int EPL = 4, PPL = 2;   // elements and pairs per lane (d <= 256)
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool p1 = (int)blockIdx.x >= a.nblk0;
    const size_t r = (size_t)(p1 ? (int)blockIdx.x - a.nblk0 : (int)blockIdx.x) * 4 + wv;
    if (r >= (p1 ? a.rows[1] : a.rows[0])) return;   // the whole wave: no workgroup barrier below
    const uint16_t* X = p1 ? a.X[1] : a.X[0];
    const uint16_t* W = p1 ? a.W[1] : a.W[0];
    uint16_t* Y = p1 ? a.Y[1] : a.Y[0];
    const int H = p1 ? a.H[1] : a.H[0];
    const int d = a.d, half = d / 2, end8 = (d / 8) * 8, vh = (half / 8) * 8;
    const int s = (int)((r / H) % a.S);   // row = (b * S + s) * H + h
    const uint16_t* xr = X + r * d;
    const size_t toff = (a.start_pos + s) * (size_t)half;
    uint16_t xv[EPL], wgt[EPL], cv[PPL], sv[PPL];
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        const int i = min(lane + 64 * k, d - 1);
        xv[k] = xr[i];
        wgt[k] = W[i];
    }
#pragma unroll
    for (int k = 0; k < PPL; k++) {
        const int i = min(lane + 64 * k, half - 1);
        cv[k] = a.ct[toff + i];
        sv[k] = a.stb[toff + i];
    }
    uint16_t* xs = buf[wv][0];
    uint16_t* ys = buf[wv][1];
#pragma unroll
    for (int k = 0; k < EPL; k++)
        if (lane + 64 * k < d) xs[lane + 64 * k] = xv[k];
    wave_lds_order();
    float inv;
    uint16_t hinv;
    rms_stats_wave(xs, d, a.eps, inv, hinv);
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        const int i = lane + 64 * k;
        if (i < d) ys[i] = rms_apply(xv[k], wgt[k], i, end8, inv, hinv);
    }
    wave_lds_order();
    uint16_t* yr = Y + r * d;
#pragma unroll
    for (int k = 0; k < PPL; k++) {
        const int i = lane + 64 * k;
        if (i < half) {
            uint16_t o1, o2;
            rope_pair(ys[i], ys[i + half], cv[k], sv[k], i < vh, o1, o2);
            yr[i] = o1;
            yr[i + half] = o2;
        }
    }
}

__global__ void silu_kernel(const uint16_t* __restrict__ X, uint16_t* __restrict__ Y, size_t n) {
    const size_t body = (n / 8) * 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const float x = h2f(X[i]);
        const float e = (i < body) ? fast_exp(-x) : cactus_expf(-x);
        const float sig = 1.0f / (1.0f + e);
        Y[i] = f2h(x * sig);
    }
}

__global__ void add_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                           uint16_t* __restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        Y[i] = hadd(A[i], B[i]);
}

__global__ void mul_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                           uint16_t* __restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        Y[i] = hmul(A[i], B[i]);
}

// ---------------------------------------------------------------- transpose
__global__ void transpose_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                 size_t rows, size_t cols) {
    __shared__ uint16_t tile[32][33];
    const size_t c0 = (size_t)blockIdx.x * 32, r0 = (size_t)blockIdx.y * 32;
    for (int i = threadIdx.y; i < 32; i += 8) {
        const size_t r = r0 + i, c = c0 + threadIdx.x;
        if (r < rows && c < cols) tile[i][threadIdx.x] = src[r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += 8) {
        const size_t c = c0 + i, r = r0 + threadIdx.x;
        if (r < rows && c < cols) dst[c * rows + r] = tile[threadIdx.x][i];
    }
}

// ---------------------------------------------------------------- embedding
__global__ void embedding_kernel(const uint16_t* __restrict__ table, const float* __restrict__ ids,
                                 uint16_t* __restrict__ out, size_t n, int hidden, size_t vocab,
                                 int* err) {
    const size_t row = blockIdx.x;
    if (row >= n) return;
    const float f = ids[row];
    const bool ok = (f >= 0.0f) && (f < (float)vocab) && ((size_t)f < vocab);
    uint16_t* o = out + row * (size_t)hidden;
    if (!ok) {
        for (int j = threadIdx.x; j < hidden; j += blockDim.x) o[j] = 0;
        if (err && threadIdx.x == 0) *err = 1;
        return;
    }
    const uint16_t* src = table + (size_t)f * hidden;
    for (int j = threadIdx.x; j < hidden; j += blockDim.x) o[j] = src[j];
}

static unsigned grid_for(size_t n, unsigned block) {
    size_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > 65535) g = 65535;
    return (unsigned)g;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_rms_norm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t rows,
                            size_t dims, float eps, void* stream) {
    if (rows == 0 || dims == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && w && y, "rms_norm: null pointer");
    CH_REQUIRE(dims <= (size_t)RMS_MAX_DIMS, "rms_norm: dims > 8192 not supported");
    CH_REQUIRE(rows < (1ull << 33), "rms_norm: too many rows");
    const size_t smem = 4 * dims * sizeof(uint16_t);
    hipLaunchKernelGGL(rms_norm_kernel, dim3(ceil_div(rows, 4)), dim3(256), smem, as_stream(stream),
                       x, w, y, rows, (int)dims, eps);
    return check_launch("rms_norm");
}

int cactus_hip_rope_reserve(size_t max_pos, size_t head_dim, float theta) {
    CH_REQUIRE(head_dim >= 2 && head_dim % 2 == 0, "rope: head_dim must be even");
    RopeTable t;
    return rope_table(max_pos, head_dim, theta, &t);
}

int cactus_hip_rope_f16(const uint16_t* x, uint16_t* y, size_t batch, size_t seq_len,
                        size_t num_heads, size_t head_dim, size_t start_pos, float theta,
                        void* stream) {
    if (batch == 0 || seq_len == 0 || num_heads == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && y, "rope: null pointer");
    CH_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim < (1u << 16),
               "rope: head_dim must be even");
    RopeTable t;
    int rc = rope_table(seq_len + start_pos, head_dim, theta, &t);
    if (rc) return rc;
    const size_t pairs = batch * seq_len * num_heads * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0, as_stream(stream), x,
                       y, t.cos_d, t.sin_d, pairs, (int)seq_len, (int)num_heads, (int)head_dim,
                       start_pos);
    return check_launch("rope");
}

int cactus_hip_rms_norm_rope_f16(const uint16_t* x, const uint16_t* weight, uint16_t* y, size_t batch,
                                 size_t seq_len, size_t num_heads, size_t head_dim, size_t start_pos, float theta,
                                 float eps, void* stream) {
    return cactus_hip_rms_norm_rope_qk_f16(x, weight, y, num_heads, nullptr, nullptr, nullptr, 0, batch, seq_len,
                                           head_dim, start_pos, theta, eps, stream);
}

int cactus_hip_rms_norm_rope_qk_f16(const uint16_t* q, const uint16_t* q_weight, uint16_t* q_out, size_t q_heads,
                                    const uint16_t* k, const uint16_t* k_weight, uint16_t* k_out, size_t kv_heads,
                                    size_t batch, size_t seq_len, size_t head_dim, size_t start_pos, float theta,
                                    float eps, void* stream) {
    const size_t rq = batch * seq_len * q_heads, rk = batch * seq_len * kv_heads;
    if (rq + rk == 0) return CACTUS_HIP_OK;
    CH_REQUIRE((rq == 0 || (q && q_weight && q_out)) && (rk == 0 || (k && k_weight && k_out)),
               "rms_norm_rope: null pointer");
    CH_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 256, "rms_norm_rope: head_dim must be even, <= 256");
    CH_REQUIRE((rq + 3) / 4 + (rk + 3) / 4 < (1u << 31), "rms_norm_rope: too many rows");
    RopeTable t;
    int rc = rope_table(seq_len + start_pos, head_dim, theta, &t);
    if (rc) return rc;
    RopeRowsArgs a{};
    // problem 0 is the first non-empty one
    const bool only_k = rq == 0;
    a.X[0] = only_k ? k : q;  a.W[0] = only_k ? k_weight : q_weight;  a.Y[0] = only_k ? k_out : q_out;
    a.rows[0] = only_k ? rk : rq;  a.H[0] = (int)(only_k ? kv_heads : q_heads);
    a.X[1] = k;  a.W[1] = k_weight;  a.Y[1] = k_out;
    a.rows[1] = only_k ? 0 : rk;  a.H[1] = (int)(kv_heads ? kv_heads : 1);
    a.nblk0 = (int)((a.rows[0] + 3) / 4);
    a.ct = t.cos_d;  a.stb = t.sin_d;
    a.S = (int)seq_len;  a.d = (int)head_dim;  a.start_pos = start_pos;  a.eps = eps;
    const size_t blocks = a.nblk0 + (a.rows[1] + 3) / 4;
    hipLaunchKernelGGL(rms_rope_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), a);
    return check_launch("rms_norm_rope");
}

int cactus_hip_softmax_f16(const uint16_t* x, uint16_t* y, size_t batch, size_t seq_len,
                           size_t vocab, void* stream) {
    const size_t rows = batch * seq_len;
    if (rows == 0 || vocab == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && y, "softmax: null pointer");
    CH_REQUIRE(vocab < (1u << 30) && rows < (1u << 31), "softmax: shape too large");
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)rows), dim3(256), 0, as_stream(stream), x, y,
                       (int)vocab);
    return check_launch("softmax");
}

int cactus_hip_silu_f16(const uint16_t* x, uint16_t* y, size_t n, void* stream) {
    if (n == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(x && y, "silu: null pointer");
    hipLaunchKernelGGL(silu_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), x, y, n);
    return check_launch("silu");
}

int cactus_hip_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n, void* stream) {
    if (n == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(a && b && y, "add: null pointer");
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), a, b, y, n);
    return check_launch("add");
}

int cactus_hip_multiply_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n,
                            void* stream) {
    if (n == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(a && b && y, "multiply: null pointer");
    hipLaunchKernelGGL(mul_kernel, dim3(grid_for(n, 256)), dim3(256), 0, as_stream(stream), a, b, y, n);
    return check_launch("multiply");
}

int cactus_hip_transpose_2d_f16(const uint16_t* src, uint16_t* dst, size_t rows, size_t cols,
                                void* stream) {
    if (rows == 0 || cols == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(src && dst, "transpose: null pointer");
    CH_REQUIRE(rows / 32 < 65535 && cols / 32 < (1u << 30), "transpose: shape too large");
    hipLaunchKernelGGL(transpose_kernel, dim3(ceil_div(cols, 32), ceil_div(rows, 32)), dim3(32, 8), 0,
                       as_stream(stream), src, dst, rows, cols);
    return check_launch("transpose");
}

int cactus_hip_embedding_f16(const uint16_t* table, const float* ids, uint16_t* out,
                             size_t num_ids, size_t hidden, size_t vocab, int* error_flag,
                             void* stream) {
    if (num_ids == 0 || hidden == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(table && ids && out, "embedding: null pointer");
    CH_REQUIRE(num_ids <= 0x7FFFFFFF && hidden < (1u << 30), "embedding: shape too large");
    hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)num_ids), dim3(256), 0, as_stream(stream),
                       table, ids, out, num_ids, (int)hidden, vocab, error_flag);
    return check_launch("embedding");
}

}  // extern "C"
