// family.hip -- ops of the other model families the reference runs through
// the same kernel layer: GELU (tanh form, Gemma), GELU-erf, LayerNorm
// (Whisper, Nomic), causal depthwise conv1d (LFM2) and the 3-tap conv1d
// (Whisper's front end).  Each output follows the reference's operation
// order (lanes, pairwise reductions, fused multiply-adds) bit for bit:
//
//   cactus_gelu_f16 / _erf             kernel_nn.cpp:46-150
//   fast_tanh_f32x4                    kernel_utils.h:143-163
//   compute_layernorm_node             graph_ops_nn.cpp:373-457
//   cactus_conv1d_causal_depthwise_f16 kernel_conv.cpp:15-110
//   cactus_conv1d_f16_k3               kernel_conv.cpp:112-236
//
// These are memory-light element or row operations off the Qwen3 path; one
// thread per output (per row for LayerNorm's sequential sums) keeps the
// reference's order with no cross-lane reduction.  tanhf (the GELU tail)
// and erff are evaluated in double and rounded once to float, the same
// libm boundary as cactus_expf.
#include "hip_common.h"

namespace cactus_hip {

__device__ __forceinline__ float fast_tanh_f(float x) {
    if (x > 4.5f) return 1.0f;
    if (x < -4.5f) return -1.0f;
    const float x2 = x * x;
    const float num = 27.0f + x2;
    const float den = __builtin_fmaf(9.0f, x2, 27.0f);
    return x * (num / den);
}

__global__ void gelu_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out, size_t n) {
    const float s2pi = 0.7978845608028654f, coeff = 0.044715f;
    const size_t body = (n / 8) * 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float x = h2f(in[i]);
        float g;
        if (i < body) {
            const float x3 = (x * x) * x;
            const float inner = s2pi * __builtin_fmaf(coeff, x3, x);
            g = (0.5f * x) * (1.0f + fast_tanh_f(inner));
        } else {
            const float inner = s2pi * __builtin_fmaf((coeff * x) * x, x, x);
            g = (0.5f * x) * (1.0f + (float)tanh((double)inner));
        }
        out[i] = f2h(g);
    }
}

__global__ void gelu_erf_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out, size_t n) {
    const float inv_sqrt2 = 0.70710678118654752440f;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float x = h2f(in[i]);
        out[i] = f2h((x * 0.5f) * (1.0f + (float)erf((double)(x * inv_sqrt2))));
    }
}

// one thread per row for the mean and variance chains, then the row's
// outputs by the workgroup's 64 threads of that row's wave
__global__ void __launch_bounds__(256) layer_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ b, uint16_t* __restrict__ y,
                                                         size_t rows, size_t F, float eps) {
    __shared__ float stats[4][2];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * 4 + wv;
    if (r >= rows) return;   // the whole wave leaves: no barrier below
    const uint16_t* xr = x + r * F;
    if (lane == 0) {
        float mean = 0.0f;
        for (size_t i = 0; i < F; i++) mean += h2f(xr[i]);
        mean /= (float)F;
        float var = 0.0f;
        for (size_t i = 0; i < F; i++) {
            const float d = h2f(xr[i]) - mean;
            var = __builtin_fmaf(d, d, var);
        }
        var /= (float)F;
        stats[wv][0] = mean;
        stats[wv][1] = 1.0f / __builtin_sqrtf(var + eps);
    }
    wave_lds_order();
    const float mean = stats[wv][0], inv = stats[wv][1];
    for (size_t i = lane; i < F; i += 64)
        y[r * F + i] = f2h(__builtin_fmaf((h2f(xr[i]) - mean) * inv, h2f(w[i]), h2f(b[i])));
}

// x [N][L][C], w [C][K]; thread per output (n, t, c)
__global__ void conv1d_causal_dw_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                        uint16_t* __restrict__ y, size_t N, size_t L, size_t C, size_t K,
                                        size_t dil) {
    const size_t total = N * L * C;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (size_t)gridDim.x * blockDim.x) {
        const size_t c = o % C, t = (o / C) % L, n = o / (C * L);
        const uint16_t* wc = w + c * K;
        float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        size_t k = 0;
        for (; k + 8 <= K; k += 8) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const size_t kk = k + 4 * h + j;
                    const long long a = (long long)t - (long long)(kk * dil);
                    const float xv = a >= 0 ? h2f(x[(n * L + (size_t)a) * C + c]) : 0.0f;
                    lane[j] = __builtin_fmaf(xv, h2f(wc[K - 1 - kk]), lane[j]);
                }
            }
        }
        float acc = (lane[0] + lane[1]) + (lane[2] + lane[3]);
        for (; k < K; k++) {
            const long long a = (long long)t - (long long)(k * dil);
            if (a >= 0) acc = __builtin_fmaf(h2f(wc[K - 1 - k]), h2f(x[(n * L + (size_t)a) * C + c]), acc);
        }
        y[o] = f2h(acc);
    }
}

// x [N][C_in][L], w [C_out][C_in][3], y [N][C_out][out_len]; thread per output
__global__ void conv1d_k3_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                 uint16_t* __restrict__ y, size_t N, size_t L, size_t Cin, size_t Cout,
                                 size_t stride, size_t out_len) {
    const size_t total = N * Cout * out_len;
    for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += (size_t)gridDim.x * blockDim.x) {
        const size_t oi = o % out_len, oc = (o / out_len) % Cout, n = o / (out_len * Cout);
        const size_t t = oi * stride;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (size_t ic = 0; ic < Cin; ic++) {
            const uint16_t* xc = x + (n * Cin + ic) * L;
            const uint16_t* wc = w + (oc * Cin + ic) * 3;
            const float xm = t >= 1 ? h2f(xc[t - 1]) : 0.0f;
            const float x0 = h2f(xc[t]);
            const float xp = t + 1 < L ? h2f(xc[t + 1]) : 0.0f;
            a0 = __builtin_fmaf(xm, h2f(wc[0]), a0);
            a1 = __builtin_fmaf(x0, h2f(wc[1]), a1);
            a2 = __builtin_fmaf(xp, h2f(wc[2]), a2);
            a3 = __builtin_fmaf(0.0f, 0.0f, a3);
        }
        y[o] = f2h((a0 + a2) + (a1 + a3));
    }
}

static unsigned blocks_for(size_t n, unsigned block) {
    size_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > 65535) g = 65535;
    return (unsigned)g;
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_gelu_f16(const uint16_t* in, uint16_t* out, size_t n, void* stream) {
    if (n == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(in && out, "gelu: null pointer");
    hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), in, out, n);
    return check_launch("gelu");
}

int cactus_hip_gelu_erf_f16(const uint16_t* in, uint16_t* out, size_t n, void* stream) {
    if (n == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(in && out, "gelu_erf: null pointer");
    hipLaunchKernelGGL(gelu_erf_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, as_stream(stream), in, out, n);
    return check_launch("gelu_erf");
}

int cactus_hip_layer_norm_f16(const uint16_t* x, const uint16_t* weight, const uint16_t* bias, uint16_t* y,
                              size_t rows, size_t features, float eps, void* stream) {
    if (rows == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(features > 0, "layer_norm: LayerNorm requires non-empty input tensor");
    CH_REQUIRE(x && weight && bias && y, "layer_norm: null pointer");
    CH_REQUIRE(rows / 4 < (1u << 31), "layer_norm: too many rows");
    hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, as_stream(stream), x,
                       weight, bias, y, rows, features, eps);
    return check_launch("layer_norm");
}

int cactus_hip_conv1d_causal_depthwise_f16(const uint16_t* input, const uint16_t* weight, uint16_t* output,
                                           size_t N, size_t L, size_t C, size_t K, size_t dilation,
                                           void* stream) {
    if (N == 0 || L == 0 || C == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(input && weight && output, "conv1d_causal_depthwise: null pointer");
    CH_REQUIRE(K > 0 && dilation > 0, "conv1d_causal_depthwise: kernel size and dilation must be positive");
    hipLaunchKernelGGL(conv1d_causal_dw_kernel, dim3(blocks_for(N * L * C, 256)), dim3(256), 0, as_stream(stream),
                       input, weight, output, N, L, C, K, dilation);
    return check_launch("conv1d_causal_depthwise");
}

int cactus_hip_conv1d_f16_k3(const uint16_t* input, const uint16_t* weight, uint16_t* output, size_t N, size_t L,
                             size_t C_in, size_t C_out, size_t stride, void* stream) {
    if (N == 0 || C_out == 0) return CACTUS_HIP_OK;
    CH_REQUIRE(input && weight && output, "conv1d_k3: null pointer");
    CH_REQUIRE(L > 0 && stride > 0 && C_in > 0, "conv1d_k3: length, stride and input channels must be positive");
    const size_t out_len = (L - 1) / stride + 1;
    hipLaunchKernelGGL(conv1d_k3_kernel, dim3(blocks_for(N * C_out * out_len, 256)), dim3(256), 0,
                       as_stream(stream), input, weight, output, N, L, C_in, C_out, stride, out_len);
    return check_launch("conv1d_k3");
}

}  // extern "C"
