/*
 * family_oracle.c -- CPU restatement of the ops other model families use
 * (test infrastructure; see cactus_oracle.h):
 *
 *   cactus_gelu_f16                    kernel/kernel_nn.cpp:46-92 (tanh form)
 *   cactus_gelu_f16_erf                kernel/kernel_nn.cpp:94-150
 *   fast_tanh_f32x4                    kernel/kernel_utils.h:143-163
 *   compute_layernorm_node (FP16)      graph/graph_ops_nn.cpp:373-457
 *   cactus_conv1d_causal_depthwise_f16 kernel/kernel_conv.cpp:15-110
 *   cactus_conv1d_f16_k3               kernel/kernel_conv.cpp:112-236
 *
 * Operation order and contraction follow the reference as clang compiles it
 * (-ffp-contract=on): `a += b * c` and `x*s*w + b` end in one fused
 * multiply-add.  Libm boundary: tanhf (the GELU tail) and erff are
 * evaluated in double with the host libm and rounded once to float; the
 * HIP library does the same with the device math library.
 */
#include "cactus_oracle.h"

#include <math.h>
#include <stddef.h>

static float tanh_f(float x) { return (float)tanh((double)x); }
static float erf_f(float x) { return (float)erf((double)x); }

float orc_fast_tanh(float x) {
    if (x > 4.5f) return 1.0f;
    if (x < -4.5f) return -1.0f;
    const float x2 = x * x;
    const float num = 27.0f + x2;
    const float den = fmaf(9.0f, x2, 27.0f);
    return x * (num / den);
}

/* elements below (n / 8) * 8 take the vector body, the rest the scalar tail */
void orc_gelu_f16(const uint16_t* in, uint16_t* out, size_t n) {
    const float s2pi = 0.7978845608028654f, coeff = 0.044715f;
    const size_t body = (n / 8) * 8;
    for (size_t i = 0; i < n; i++) {
        const float x = orc_h2f(in[i]);
        float g;
        if (i < body) {
            const float x3 = (x * x) * x;
            const float inner = s2pi * fmaf(coeff, x3, x);
            const float t = orc_fast_tanh(inner);
            g = (0.5f * x) * (1.0f + t);
        } else {
            const float inner = s2pi * fmaf((coeff * x) * x, x, x);
            g = (0.5f * x) * (1.0f + tanh_f(inner));
        }
        out[i] = orc_f2h(g);
    }
}

void orc_gelu_erf_f16(const uint16_t* in, uint16_t* out, size_t n) {
    const float inv_sqrt2 = 0.70710678118654752440f;
    for (size_t i = 0; i < n; i++) {
        const float x = orc_h2f(in[i]);
        out[i] = orc_f2h((x * 0.5f) * (1.0f + erf_f(x * inv_sqrt2)));
    }
}

void orc_layer_norm_f16(const uint16_t* x, const uint16_t* w, const uint16_t* b, uint16_t* y, size_t rows,
                        size_t F, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const uint16_t* xr = x + r * F;
        float mean = 0.0f;
        for (size_t i = 0; i < F; i++) mean += orc_h2f(xr[i]);
        mean /= (float)F;
        float var = 0.0f;
        for (size_t i = 0; i < F; i++) {
            const float d = orc_h2f(xr[i]) - mean;
            var = fmaf(d, d, var);
        }
        var /= (float)F;
        const float inv = 1.0f / sqrtf(var + eps);
        for (size_t i = 0; i < F; i++)
            y[r * F + i] = orc_f2h(fmaf((orc_h2f(xr[i]) - mean) * inv, orc_h2f(w[i]), orc_h2f(b[i])));
    }
}

void orc_conv1d_causal_depthwise_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t N, size_t L,
                                     size_t C, size_t K, size_t dil) {
    for (size_t n = 0; n < N; n++)
        for (size_t c = 0; c < C; c++)
            for (size_t t = 0; t < L; t++) {
                /* tap k reads x[t - k*dil] with the reversed weight w[K-1-k] */
                float lane[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                size_t k = 0;
                for (; k + 8 <= K; k += 8)
                    for (int h = 0; h < 2; h++)
                        for (int j = 0; j < 4; j++) {
                            const size_t kk = k + 4 * h + j;
                            const ptrdiff_t a = (ptrdiff_t)t - (ptrdiff_t)(kk * dil);
                            const float xv = a >= 0 ? orc_h2f(x[(n * L + (size_t)a) * C + c]) : 0.0f;
                            lane[j] = fmaf(xv, orc_h2f(w[c * K + (K - 1 - kk)]), lane[j]);
                        }
                float acc = (lane[0] + lane[1]) + (lane[2] + lane[3]);
                for (; k < K; k++) {
                    const ptrdiff_t a = (ptrdiff_t)t - (ptrdiff_t)(k * dil);
                    if (a >= 0) acc = fmaf(orc_h2f(w[c * K + (K - 1 - k)]), orc_h2f(x[(n * L + (size_t)a) * C + c]), acc);
                }
                y[(n * L + t) * C + c] = orc_f2h(acc);
            }
}

void orc_conv1d_f16_k3(const uint16_t* x, const uint16_t* w, uint16_t* y, size_t N, size_t L, size_t Cin,
                       size_t Cout, size_t stride) {
    const size_t out_len = (L - 1) / stride + 1;
    for (size_t n = 0; n < N; n++)
        for (size_t oc = 0; oc < Cout; oc++)
            for (size_t o = 0; o < out_len; o++) {
                const size_t t = o * stride;
                float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                for (size_t ic = 0; ic < Cin; ic++) {
                    const uint16_t* xc = x + (n * Cin + ic) * L;
                    const uint16_t* wc = w + (oc * Cin + ic) * 3;
                    const float xm = t >= 1 ? orc_h2f(xc[t - 1]) : 0.0f;
                    const float x0 = orc_h2f(xc[t]);
                    const float xp = t + 1 < L ? orc_h2f(xc[t + 1]) : 0.0f;
                    a0 = fmaf(xm, orc_h2f(wc[0]), a0);
                    a1 = fmaf(x0, orc_h2f(wc[1]), a1);
                    a2 = fmaf(xp, orc_h2f(wc[2]), a2);
                    a3 = fmaf(0.0f, 0.0f, a3);
                }
                y[(n * Cout + oc) * out_len + o] = orc_f2h((a0 + a2) + (a1 + a3));
            }
}
