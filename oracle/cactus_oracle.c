/*
 * cactus_oracle.c -- CPU restatement of the Cactus kernel layer (test
 * infrastructure; see cactus_oracle.h).  Built with -ffp-contract=off so
 * that the only fused multiply-adds are the explicit fmaf() calls placed
 * where the reference's NEON code uses vfmaq or where clang contracts a
 * scalar `a += b * c`.
 */
#include "cactus_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 helpers                                                              */
/* ------------------------------------------------------------------------ */

/* Worker threads for the row/head loops below (1 = serial, the default).
 * Each output element is computed by the same sequential code whatever the
 * thread count, so results do not depend on it. */
int orc_nt = 1;
void orc_set_threads(int n) { orc_nt = n < 1 ? 1 : n; }

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in float */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f(sign | 0x7F800000u | (m << 13));
    return bits_f(sign | ((e + 112u) << 23) | (m << 13));
}

/* Round an arbitrary double to fp16, nearest-even, one rounding step. */
uint16_t orc_d2h(double d) {
    uint64_t b; memcpy(&b, &d, 8);
    uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    uint64_t a = b & 0x7FFFFFFFFFFFFFFFull;
    int e = (int)(a >> 52);
    if (e == 0x7FF) return sign | (a & 0xFFFFFFFFFFFFFull ? 0x7E00 : 0x7C00);
    if (a == 0) return sign;
    uint64_t mant = (a & 0xFFFFFFFFFFFFFull) | (e ? (1ull << 52) : 0);
    int exp = (e ? e : 1) - 1023;                 /* value = mant * 2^(exp-52) */
    if (exp > 15) return sign | 0x7C00;
    int shift;                                     /* bits dropped from mant */
    uint32_t base;
    if (exp >= -14) { shift = 42; base = (uint32_t)(exp + 15) << 10; }
    else {
        shift = 42 + (-14 - exp);
        if (shift > 63) return sign;               /* < 2^-25: rounds to zero */
        base = 0;
    }
    uint64_t q = mant >> shift;
    uint64_t rem = mant & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    /* for normals q holds the implicit bit (1024..2048); drop it */
    uint32_t r = (exp >= -14) ? base + (uint32_t)(q - 1024) : (uint32_t)q;
    if (r >= 0x7C00) return sign | 0x7C00;
    return sign | (uint16_t)r;
}

uint16_t orc_f2h(float f) { return orc_d2h((double)f); }

uint16_t orc_hadd(uint16_t a, uint16_t b) {
    return orc_d2h((double)orc_h2f(a) + (double)orc_h2f(b));   /* exact sum */
}
uint16_t orc_hmul(uint16_t a, uint16_t b) {
    return orc_d2h((double)orc_h2f(a) * (double)orc_h2f(b));   /* exact product */
}
uint16_t orc_hfma(uint16_t a, uint16_t b, uint16_t c) {
    return orc_d2h(fma((double)orc_h2f(a), (double)orc_h2f(b), (double)orc_h2f(c)));
}

/* NEON vcvtq_s32_f32: truncate toward zero, saturate, NaN -> 0. */
static inline int32_t cvt_trunc_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}
/* NEON vcvtnq_s32_f32: round to nearest even, saturate, NaN -> 0. */
static inline int32_t cvt_rne_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)nearbyintf(x);
}
static inline int8_t sat8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }
/* (zi + 127) << 23 reinterpreted as float, with int32 wrap-around semantics */
static inline float exp2_bits(int32_t zi) {
    return bits_f((uint32_t)((uint32_t)zi + 127u) << 23);
}

/* ------------------------------------------------------------------------ */
/* expf substitute: Cody-Waite reduction x = k*ln2 + r, |r| <= ln2/2, then    */
/* the degree-12 Taylor polynomial of e^r in double (Horner with fma), then  */
/* one rounding to float.  The HIP library evaluates the same sequence.      */
/* ------------------------------------------------------------------------ */
float orc_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 100.0f) return INFINITY;
    if (xf < -110.0f) return 0.0f;
    const double LN2_HI = 6.93147180369123816490e-01;   /* low 21 bits zero */
    const double LN2_LO = 1.90821492927058770002e-10;
    double x = (double)xf;
    double k = nearbyint(x * 1.44269504088896338700e+00);
    double r = fma(-k, LN2_HI, x);
    r = fma(-k, LN2_LO, r);
    double p = 1.0 / 479001600.0;                 /* 1/12! */
    p = fma(p, r, 1.0 / 39916800.0);
    p = fma(p, r, 1.0 / 3628800.0);
    p = fma(p, r, 1.0 / 362880.0);
    p = fma(p, r, 1.0 / 40320.0);
    p = fma(p, r, 1.0 / 5040.0);
    p = fma(p, r, 1.0 / 720.0);
    p = fma(p, r, 1.0 / 120.0);
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    uint64_t sb = (uint64_t)((int64_t)k + 1023) << 52;   /* 2^k, k in [-159,145] */
    double s; memcpy(&s, &sb, 8);
    return (float)(p * s);
}

/* fast_exp_f32x4, one lane (kernel_utils.h:108-141) */
float orc_fast_exp(float x) {
    x = fmaxf(x, -87.0f);
    x = fminf(x, 87.0f);
    float z = x * 1.4426950408889634f;
    int32_t zi = cvt_trunc_sat(z);
    float zf = z - (float)zi;
    if (zf < 0.0f) { zi -= 1; zf = zf + 1.0f; }
    float u = zf * 0.6931471805599453f;
    float p = 0.009618129842071803f;
    p = fmaf(p, u, 0.05550410866482158f);
    p = fmaf(p, u, 0.2402265069591007f);
    p = fmaf(p, u, 0.6931471805599453f);
    p = fmaf(p, u, 1.0f);
    return p * exp2_bits(zi);
}

/* Block weight of cactus_attention_f16's vector path
 * (kernel_attention.cpp:174-195): second-order 2^x polynomial. */
float orc_poly_exp_weight(float s, float bm) {
    if (s == -INFINITY) return 0.0f;
    float x = s - bm;
    x = x * 1.442695f;
    int32_t xi = cvt_trunc_sat(x);
    float xf = x - (float)xi;
    float y = fmaf(xf, 0.6931472f, 1.0f);
    float xf2 = xf * xf;
    y = fmaf(xf2, 0.2402265f, y);
    return y * exp2_bits(xi);
}

/* ------------------------------------------------------------------------ */
/* a1: activation quantization                                               */
/* ------------------------------------------------------------------------ */

/* cactus_fp16_max_abs (kernel_quants.cpp:196-221): max is order-free */
float orc_fp16_max_abs(const uint16_t* src, size_t count) {
    float m = 0.0f;
    for (size_t i = 0; i < count; i++) {
        float v = fabsf(orc_h2f(src[i]));
        if (v > m) m = v;
    }
    return m;
}

/* cactus_fp16_to_int8 (kernel_quants.cpp:158-194), single-thread chunking:
 * 8-wide body uses clamp + vcvtnq (nearest-even); the count%8 tail uses
 * clamp + std::round (ties away from zero). */
void orc_fp16_to_int8(const uint16_t* src, int8_t* dst, size_t count, float scale) {
    const float inv = 1.0f / scale;
    const size_t body = (count / 8) * 8;
    for (size_t i = 0; i < body; i++) {
        float v = orc_h2f(src[i]) * inv;
        v = fmaxf(fminf(v, 127.0f), -128.0f);
        dst[i] = sat8(cvt_rne_sat(v));
    }
    for (size_t i = body; i < count; i++) {
        float v = orc_h2f(src[i]) * inv;
        v = fmaxf(-128.0f, fminf(127.0f, v));
        dst[i] = (int8_t)roundf(v);
    }
}

/* quantize_activations_fp16_to_int8 (graph_ops_nn.cpp:35-66) */
void orc_quantize_activations(const uint16_t* x, int8_t* q, float* scales,
                              size_t M, size_t K) {
#pragma omp parallel for num_threads(orc_nt) if (orc_nt > 1 && M > 1)
    for (size_t m = 0; m < M; m++) {
        float max_abs = orc_fp16_max_abs(x + m * K, K);
        float s = max_abs / 127.0f;
        if (s < 1e-10f) s = 1e-10f;
        scales[m] = s;
        orc_fp16_to_int8(x + m * K, q + m * K, K, s);
    }
}

/* ------------------------------------------------------------------------ */
/* a2/a3: grouped integer matmul                                             */
/* ------------------------------------------------------------------------ */

/* cactus_unpack_int4_to_int8 (kernel_quants.cpp:295-351): byte i holds
 * element 2i in its low nibble and 2i+1 in its high nibble, two's
 * complement 4-bit. */
static inline int8_t nib(uint8_t byte, int hi) {
    int v = hi ? (byte >> 4) : (byte & 0x0F);
    return (int8_t)(v > 7 ? v - 16 : v);
}

void orc_unpack_int4_to_int8(const uint8_t* packed, int8_t* unpacked, size_t count) {
    for (size_t i = 0; i < count; i++) unpacked[i] = nib(packed[i / 2], (int)(i & 1));
}

void orc_group_sums_int8(const int8_t* A, const int8_t* B, int32_t* acc,
                         size_t M, size_t K, size_t N, size_t gs) {
    const size_t G = K / gs;
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++)
            for (size_t g = 0; g < G; g++) {
                int32_t s = 0;
                for (size_t k = g * gs; k < (g + 1) * gs; k++)
                    s += (int32_t)A[m * K + k] * (int32_t)B[n * K + k];
                acc[(m * N + n) * G + g] = s;
            }
}

/* Epilogue of cactus_matmul_int8/int4 (kernel_gemm.cpp:311-324):
 *   running_sum += (float)group_acc * (float)B_scale   (contracted: fma)
 * over groups in ascending order, then C = fp16(running_sum * A_scale). */
static void matmul_grouped_rows(const int8_t* A, const float* As, const int8_t* B_row,
                                const uint16_t* Bs_row, uint16_t* C, size_t M, size_t K,
                                size_t N, size_t n, size_t gs) {
    const size_t G = K / gs;
    for (size_t m = 0; m < M; m++) {
        const int8_t* a = A + m * K;
        float r = 0.0f;
        for (size_t g = 0; g < G; g++) {
            int32_t s = 0;
            for (size_t k = g * gs; k < (g + 1) * gs; k++) s += (int32_t)a[k] * (int32_t)B_row[k];
            r = fmaf((float)s, orc_h2f(Bs_row[g]), r);
        }
        C[m * N + n] = orc_f2h(r * As[m]);
    }
}

void orc_matmul_int8(const int8_t* A, const float* As, const int8_t* B, const uint16_t* Bs,
                     uint16_t* C, size_t M, size_t K, size_t N, size_t gs) {
    if (M == 0 || K == 0 || N == 0) return;
    const size_t G = K / gs;
#pragma omp parallel for schedule(dynamic, 16) num_threads(orc_nt) if (orc_nt > 1)
    for (size_t n = 0; n < N; n++)
        matmul_grouped_rows(A, As, B + n * K, Bs + n * G, C, M, K, N, n, gs);
}

/* cactus_matmul_int4 (kernel_gemm.cpp:329-529): same formula on unpacked codes */
void orc_matmul_int4(const int8_t* A, const float* As, const uint8_t* Bp, const uint16_t* Bs,
                     uint16_t* C, size_t M, size_t K, size_t N, size_t gs) {
    if (M == 0 || K == 0 || N == 0) return;
    const size_t G = K / gs;
#pragma omp parallel num_threads(orc_nt) if (orc_nt > 1)
    {
        int8_t* row = (int8_t*)malloc(K);
#pragma omp for schedule(dynamic, 16)
        for (size_t n = 0; n < N; n++) {
            orc_unpack_int4_to_int8(Bp + n * (K / 2), row, K);
            matmul_grouped_rows(A, As, row, Bs + n * G, C, M, K, N, n, gs);
        }
        free(row);
    }
}

/* Threaded CPU baseline: rows of B split over threads the way
 * CactusThreading::enqueue_n_threads splits tiles (kernel_utils.h:358-374). */
typedef struct {
    const int8_t* A; const float* As; const int8_t* B; const uint16_t* Bs; uint16_t* C;
    size_t M, K, N, gs, n0, n1;
} mm_job;

static void* mm_worker(void* p) {
    mm_job* j = (mm_job*)p;
    const size_t G = j->K / j->gs;
    for (size_t n = j->n0; n < j->n1; n++)
        matmul_grouped_rows(j->A, j->As, j->B + n * j->K, j->Bs + n * G, j->C, j->M, j->K,
                            j->N, n, j->gs);
    return NULL;
}

void orc_matmul_int8_mt(const int8_t* A, const float* As, const int8_t* B, const uint16_t* Bs,
                        uint16_t* C, size_t M, size_t K, size_t N, size_t gs, int nt) {
    if (nt <= 1) { orc_matmul_int8(A, As, B, Bs, C, M, K, N, gs); return; }
    if (nt > 64) nt = 64;
    pthread_t th[64];
    mm_job jobs[64];
    size_t per = N / (size_t)nt, rem = N % (size_t)nt;
    for (int t = 0; t < nt; t++) {
        size_t s = (size_t)t * per + ((size_t)t < rem ? (size_t)t : rem);
        size_t e = s + per + ((size_t)t < rem ? 1 : 0);
        jobs[t] = (mm_job){A, As, B, Bs, C, M, K, N, gs, s, e};
        pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* a4: cactus_matmul_f16 (kernel_gemm.cpp:17-126)                            */
/* ------------------------------------------------------------------------ */
void orc_matmul_f16(const uint16_t* a, const uint16_t* bT, uint16_t* c,
                    size_t M, size_t K, size_t N) {
    const size_t K16 = (K / 16) * 16, K8 = (K / 8) * 8;
    for (size_t m = 0; m < M; m++) {
        const uint16_t* ar = a + m * K;
#pragma omp parallel for schedule(dynamic, 256) num_threads(orc_nt) if (orc_nt > 1)
        for (size_t n = 0; n < N; n++) {
            const uint16_t* br = bT + n * K;
            uint16_t l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            /* lane j accumulates k = j (mod 8) in increasing k (:43-66) */
            for (size_t k = 0; k < K16; k += 16) {
                for (int j = 0; j < 8; j++) l[j] = orc_hfma(ar[k + j], br[k + j], l[j]);
                for (int j = 0; j < 8; j++) l[j] = orc_hfma(ar[k + 8 + j], br[k + 8 + j], l[j]);
            }
            for (size_t k = K16; k < K8; k += 8)
                for (int j = 0; j < 8; j++) l[j] = orc_hfma(ar[k + j], br[k + j], l[j]);
            /* scalar tail (:83-90): lane0 + a*b with __fp16 promoted to float
             * and contracted, then rounded back to fp16 */
            for (size_t k = K8; k < K; k++)
                l[0] = orc_f2h(fmaf(orc_h2f(ar[k]), orc_h2f(br[k]), orc_h2f(l[0])));
            /* hsum_f16x8 (:8-15) */
            uint16_t s0 = orc_hadd(l[0], l[4]), s1 = orc_hadd(l[1], l[5]);
            uint16_t s2 = orc_hadd(l[2], l[6]), s3 = orc_hadd(l[3], l[7]);
            c[m * N + n] = orc_hadd(orc_hadd(s0, s2), orc_hadd(s1, s3));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a5: cactus_attention_f16 (kernel_attention.cpp:10-255)                    */
/* ------------------------------------------------------------------------ */

/* Score of one (q, k) pair: dims 8c+j (j<4) feed low lane j, dims 8c+4+j feed
 * high lane j, both fp32 FMA chains in increasing c (:120-135); then
 * vaddvq(low + high) = (t0+t1)+(t2+t3) (:137) and dims beyond the 8-aligned
 * prefix are added with a contracted fma (:139-141). */
static float score_f16(const uint16_t* q, const uint16_t* k, size_t d) {
    float lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    const size_t da = (d / 8) * 8;
    for (size_t c = 0; c < da; c += 8)
        for (int j = 0; j < 4; j++) {
            lo[j] = fmaf(orc_h2f(q[c + j]), orc_h2f(k[c + j]), lo[j]);
            hi[j] = fmaf(orc_h2f(q[c + 4 + j]), orc_h2f(k[c + 4 + j]), hi[j]);
        }
    float t0 = lo[0] + hi[0], t1 = lo[1] + hi[1], t2 = lo[2] + hi[2], t3 = lo[3] + hi[3];
    float s = (t0 + t1) + (t2 + t3);
    for (size_t i = da; i < d; i++) s = fmaf(orc_h2f(q[i]), orc_h2f(k[i]), s);
    return s;
}

#define ATT_BLOCK 32

void orc_attention_f16(const uint16_t* Q, const uint16_t* Kt, const uint16_t* Vt, uint16_t* O,
                       size_t B, size_t S, size_t Skv, size_t Hq, size_t Hkv, size_t d,
                       float scale, const uint16_t* mask, size_t pos_off, size_t window,
                       int causal) {
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);
    const size_t da = (d / 8) * 8;
    const size_t gq = Hq / Hkv;
#pragma omp parallel num_threads(orc_nt) if (orc_nt > 1)
    {
    float* acc = (float*)malloc(sizeof(float) * (d ? d : 1));
    float bsc[ATT_BLOCK];
#pragma omp for collapse(3) schedule(dynamic, 4)
    for (size_t b = 0; b < B; b++)
    for (size_t h = 0; h < Hq; h++)
    for (size_t qp = 0; qp < S; qp++) {
        const size_t kvh = h / gq;
        const uint16_t* q = Q + ((b * S + qp) * Hq + h) * d;
        uint16_t* o = O + ((b * S + qp) * Hq + h) * d;
        const uint16_t* Mb = mask ? mask + b * S * Skv : NULL;
        float rmax = -INFINITY, rsum = 0.0f;
        for (size_t i = 0; i < d; i++) acc[i] = 0.0f;
        const int is_decode = (qp == S - 1) && S > 1;
        const size_t aq = pos_off + qp;
        size_t kv_start = 0, kv_end = Skv;
        if (window > 0 && window < Skv) {
            if (aq > window) kv_start = aq - window;
            if (causal && aq + 1 < kv_end) kv_end = aq + 1;
        } else if (causal && aq + 1 < kv_end) {
            kv_end = aq + 1;
        }
        for (size_t bs0 = kv_start; bs0 < kv_end; bs0 += ATT_BLOCK) {
            const size_t be = (bs0 + ATT_BLOCK < Skv) ? bs0 + ATT_BLOCK : Skv;
            const size_t bsz = be - bs0;
            float bmax = -INFINITY;
            if (!is_decode && causal && bs0 > aq) continue;   /* :100-105 */
            for (size_t j = 0; j < bsz; j++) {
                const size_t kp = bs0 + j;
                if (!is_decode && causal && kp > aq) { bsc[j] = -INFINITY; continue; }
                float s = score_f16(q, Kt + ((b * Skv + kp) * Hkv + kvh) * d, d);
                s = s * scale;
                if (causal && kp > aq) s = -INFINITY;
                else if (window > 0 && kp < aq && (aq - kp) > window) s = -INFINITY;
                else if (Mb && orc_h2f(Mb[qp * Skv + kp]) == 0.0f) s = -INFINITY;
                bsc[j] = s;
                bmax = fmaxf(bmax, s);
            }
            if (bmax > -INFINITY) {                       /* :160-169 */
                float corr = orc_expf(rmax - bmax);
                rsum = rsum * corr;
                for (size_t i = 0; i < da; i++) acc[i] = acc[i] * corr;
                rmax = bmax;
            }
            float bsum = 0.0f;
            const size_t vs = (bsz / 4) * 4;
            for (size_t j = 0; j < vs; j += 4) {          /* :174-195 */
                float y0 = orc_poly_exp_weight(bsc[j], bmax);
                float y1 = orc_poly_exp_weight(bsc[j + 1], bmax);
                float y2 = orc_poly_exp_weight(bsc[j + 2], bmax);
                float y3 = orc_poly_exp_weight(bsc[j + 3], bmax);
                bsc[j] = y0; bsc[j + 1] = y1; bsc[j + 2] = y2; bsc[j + 3] = y3;
                bsum = bsum + ((y0 + y1) + (y2 + y3));
            }
            for (size_t j = vs; j < bsz; j++) {           /* :197-204 */
                if (bsc[j] != -INFINITY) {
                    bsc[j] = orc_expf(bsc[j] - bmax);
                    bsum = bsum + bsc[j];
                } else {
                    bsc[j] = 0.0f;
                }
            }
            for (size_t j = 0; j < bsz; j++) {            /* :206-224 */
                const float w = bsc[j];
                if (w == 0.0f) continue;
                const uint16_t* v = Vt + ((b * Skv + bs0 + j) * Hkv + kvh) * d;
                for (size_t i = 0; i < da; i++) acc[i] = fmaf(orc_h2f(v[i]), w, acc[i]);
            }
            rsum = rsum + bsum;
        }
        if (rsum > 0.0f) {                                /* :229-252 */
            const float inv = 1.0f / rsum;
            for (size_t i = 0; i < da; i++) o[i] = orc_f2h(acc[i] * inv);
            for (size_t i = da; i < d; i++) o[i] = 0;
        } else {
            for (size_t i = 0; i < d; i++) o[i] = 0;
        }
    }
    free(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* a6: cactus_attention_hybrid_int8_fp16 (kernel_attention.cpp:257-482)      */
/* ------------------------------------------------------------------------ */

/* INT8 key: k = (float)code * scale (a rounded multiply), then the same
 * two 4-lane FMA chains as score_f16 (:351-371); the quant group is looked
 * up per 8-dim block. */
static float score_i8(const uint16_t* q, const int8_t* k, const float* ks, size_t d,
                      size_t qgs) {
    float lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    const size_t da = (d / 8) * 8;
    for (size_t c = 0; c < da; c += 8) {
        const float s = ks[c / qgs];
        for (int j = 0; j < 4; j++) {
            lo[j] = fmaf(orc_h2f(q[c + j]), (float)k[c + j] * s, lo[j]);
            hi[j] = fmaf(orc_h2f(q[c + 4 + j]), (float)k[c + 4 + j] * s, hi[j]);
        }
    }
    float t0 = lo[0] + hi[0], t1 = lo[1] + hi[1], t2 = lo[2] + hi[2], t3 = lo[3] + hi[3];
    return (t0 + t1) + (t2 + t3);
}

static float score_f16_aligned(const uint16_t* q, const uint16_t* k, size_t d) {
    float lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};
    const size_t da = (d / 8) * 8;
    for (size_t c = 0; c < da; c += 8)
        for (int j = 0; j < 4; j++) {
            lo[j] = fmaf(orc_h2f(q[c + j]), orc_h2f(k[c + j]), lo[j]);
            hi[j] = fmaf(orc_h2f(q[c + 4 + j]), orc_h2f(k[c + 4 + j]), hi[j]);
        }
    float t0 = lo[0] + hi[0], t1 = lo[1] + hi[1], t2 = lo[2] + hi[2], t3 = lo[3] + hi[3];
    return (t0 + t1) + (t2 + t3);
}

void orc_attention_hybrid_int8_fp16(const uint16_t* Q, const int8_t* Kc, const int8_t* Vc,
                                    const float* Ks, const float* Vs, const uint16_t* Kn,
                                    const uint16_t* Vn, uint16_t* O, size_t B, size_t S,
                                    size_t cache_len, size_t new_len, size_t Hq, size_t Hkv,
                                    size_t d, float scale, size_t pos_off, int causal,
                                    size_t qgs) {
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)d);
    const size_t Skv = cache_len + new_len;
    const size_t da = (d / 8) * 8;
    const size_t gq = Hq / Hkv;
    const size_t nqg = (d + qgs - 1) / qgs;
#pragma omp parallel num_threads(orc_nt) if (orc_nt > 1)
    {
    float* acc = (float*)malloc(sizeof(float) * (d ? d : 1));
    float bsc[ATT_BLOCK];
#pragma omp for collapse(3) schedule(dynamic, 4)
    for (size_t b = 0; b < B; b++)
    for (size_t h = 0; h < Hq; h++)
    for (size_t qp = 0; qp < S; qp++) {
        const size_t kvh = h / gq;
        const uint16_t* q = Q + ((b * S + qp) * Hq + h) * d;
        uint16_t* o = O + ((b * S + qp) * Hq + h) * d;
        const int8_t* Kcb = Kc + b * cache_len * Hkv * d;
        const int8_t* Vcb = Vc + b * cache_len * Hkv * d;
        const uint16_t* Knb = Kn + b * new_len * Hkv * d;
        const uint16_t* Vnb = Vn + b * new_len * Hkv * d;
        float rmax = -INFINITY, rsum = 0.0f;
        for (size_t i = 0; i < d; i++) acc[i] = 0.0f;
        const size_t aq = pos_off + qp;
        const size_t kv_end = causal ? ((aq + 1 < Skv) ? aq + 1 : Skv) : Skv;
        for (size_t bs0 = 0; bs0 < kv_end; bs0 += ATT_BLOCK) {
            const size_t be = (bs0 + ATT_BLOCK < kv_end) ? bs0 + ATT_BLOCK : kv_end;
            const size_t bsz = be - bs0;
            float bmax = -INFINITY;
            for (size_t j = 0; j < bsz; j++) {
                const size_t kp = bs0 + j;
                if (causal && kp > aq) { bsc[j] = -INFINITY; continue; }
                float s;
                if (kp < cache_len)
                    s = score_i8(q, Kcb + (kp * Hkv + kvh) * d, Ks + (kp * Hkv + kvh) * nqg, d, qgs);
                else
                    s = score_f16_aligned(q, Knb + ((kp - cache_len) * Hkv + kvh) * d, d);
                s = s * scale;
                bsc[j] = s;
                bmax = fmaxf(bmax, s);
            }
            if (bmax > -INFINITY) {
                float corr = orc_expf(rmax - bmax);
                rsum = rsum * corr;
                for (size_t i = 0; i < da; i++) acc[i] = acc[i] * corr;
                rmax = bmax;
            }
            float bsum = 0.0f;
            for (size_t j = 0; j < bsz; j++) {
                if (bsc[j] != -INFINITY) {
                    bsc[j] = orc_expf(bsc[j] - bmax);
                    bsum = bsum + bsc[j];
                } else {
                    bsc[j] = 0.0f;
                }
            }
            for (size_t j = 0; j < bsz; j++) {
                const float w = bsc[j];
                if (w == 0.0f) continue;
                const size_t kp = bs0 + j;
                if (kp < cache_len) {
                    const int8_t* v = Vcb + (kp * Hkv + kvh) * d;
                    const float* vsc = Vs + (kp * Hkv + kvh) * nqg;
                    for (size_t i = 0; i < da; i++) {
                        const float vv = (float)v[i] * vsc[(i / 8) * 8 / qgs];
                        acc[i] = fmaf(vv, w, acc[i]);
                    }
                } else {
                    const uint16_t* v = Vnb + ((kp - cache_len) * Hkv + kvh) * d;
                    for (size_t i = 0; i < da; i++) acc[i] = fmaf(orc_h2f(v[i]), w, acc[i]);
                }
            }
            rsum = rsum + bsum;
        }
        if (rsum > 0.0f) {
            const float inv = 1.0f / rsum;
            for (size_t i = 0; i < da; i++) o[i] = orc_f2h(acc[i] * inv);
            /* :472-473 leave dims beyond the 8-aligned prefix unwritten; they
             * are zeroed here so the buffer is deterministic */
            for (size_t i = da; i < d; i++) o[i] = 0;
        } else {
            for (size_t i = 0; i < d; i++) o[i] = 0;
        }
    }
    free(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* a7: cactus_quantize_kv_fp16_to_int8 (kernel_quants.cpp:223-293)           */
/* ------------------------------------------------------------------------ */
static float quantize_group(const uint16_t* src, int8_t* dst, size_t count) {
    float m = 0.0f;
    for (size_t i = 0; i < count; i++) {
        float v = fabsf(orc_h2f(src[i]));
        if (v > m) m = v;
    }
    float s = m / 127.0f;
    if (s < 1e-10f) s = 1e-10f;
    const float inv = 1.0f / s;
    const size_t body = (count / 8) * 8;
    for (size_t i = 0; i < body; i++)                /* vcvtnq + vqmovn, no clamp */
        dst[i] = sat8(cvt_rne_sat(orc_h2f(src[i]) * inv));
    for (size_t i = body; i < count; i++) {          /* roundf (ties away) + clamp */
        int32_t q = (int32_t)roundf(orc_h2f(src[i]) * inv);
        dst[i] = sat8(q);
    }
    return s;
}

void orc_quantize_kv_fp16_to_int8(const uint16_t* src, int8_t* dst, float* scales,
                                  size_t S, size_t Hkv, size_t d, size_t gs) {
    const size_t ng = (d + gs - 1) / gs;
    for (size_t idx = 0; idx < S * Hkv; idx++)
        for (size_t g = 0; g < ng; g++) {
            const size_t g0 = g * gs;
            const size_t cnt = (gs < d - g0) ? gs : d - g0;
            scales[idx * ng + g] = quantize_group(src + idx * d + g0, dst + idx * d + g0, cnt);
        }
}

/* ------------------------------------------------------------------------ */
/* a8: cactus_rms_norm_f16 (kernel_attention.cpp:484-563)                    */
/* ------------------------------------------------------------------------ */
void orc_rms_norm_f16(const uint16_t* X, const uint16_t* W, uint16_t* Y, size_t rows,
                      size_t dims, float eps) {
    const size_t tile_end = dims >= 16 ? dims - 16 + 1 : 0;
    const size_t simd_end = dims >= 8 ? dims - 8 + 1 : 0;
#pragma omp parallel for schedule(static) num_threads(orc_nt) if (orc_nt > 1 && rows > 64)
    for (size_t r = 0; r < rows; r++) {
        const uint16_t* x = X + r * dims;
        uint16_t* y = Y + r * dims;
        float v[4][4] = {{0}};
        size_t i = 0;
        for (; i < tile_end; i += 16)
            for (int u = 0; u < 4; u++)
                for (int l = 0; l < 4; l++) {
                    float a = orc_h2f(x[i + 4 * u + l]);
                    v[u][l] = fmaf(a, a, v[u][l]);
                }
        for (; i < simd_end; i += 8)
            for (int u = 0; u < 2; u++)
                for (int l = 0; l < 4; l++) {
                    float a = orc_h2f(x[i + 4 * u + l]);
                    v[u][l] = fmaf(a, a, v[u][l]);
                }
        float t[4];
        for (int l = 0; l < 4; l++) t[l] = ((v[0][l] + v[1][l]) + v[2][l]) + v[3][l];
        float ss = (t[0] + t[1]) + (t[2] + t[3]);
        for (size_t k = i; k < dims; k++) {
            float a = orc_h2f(x[k]);
            ss = fmaf(a, a, ss);
        }
        const float rms = sqrtf(ss / (float)dims + eps);
        const float inv = 1.0f / rms;
        const uint16_t hinv = orc_f2h(inv);
        size_t j = 0;
        /* elements covered by the SIMD loops use two fp16 multiplies (:541-552) */
        for (; j < i; j++) y[j] = orc_hmul(orc_hmul(x[j], hinv), W[j]);
        for (; j < dims; j++) y[j] = orc_f2h((orc_h2f(x[j]) * inv) * orc_h2f(W[j]));
    }
}

/* ------------------------------------------------------------------------ */
/* a9: cactus_rope_f16 (kernel_attention.cpp:565-676)                        */
/* ------------------------------------------------------------------------ */
void orc_rope_tables(uint16_t* cos_tab, uint16_t* sin_tab, size_t num_pos, size_t d,
                     float theta) {
    const size_t half = d / 2;
    for (size_t p = 0; p < num_pos; p++) {
        const float pf = (float)p;
        for (size_t i = 0; i < half; i++) {
            const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)d);
            const float ang = pf * freq;
            cos_tab[p * half + i] = orc_f2h(cosf(ang));
            sin_tab[p * half + i] = orc_f2h(sinf(ang));
        }
    }
}

void orc_rope_f16(const uint16_t* X, uint16_t* Y, size_t B, size_t S, size_t H, size_t d,
                  size_t start_pos, float theta) {
    const size_t half = d / 2;
    const size_t np = S + start_pos;
    uint16_t* ct = (uint16_t*)malloc(sizeof(uint16_t) * (np * half + 1));
    uint16_t* st = (uint16_t*)malloc(sizeof(uint16_t) * (np * half + 1));
    orc_rope_tables(ct, st, np, d, theta);
    const size_t vh = (half / 8) * 8;
    for (size_t b = 0; b < B; b++)
        for (size_t s = 0; s < S; s++)
            for (size_t h = 0; h < H; h++) {
                const size_t off = ((b * S + s) * H + h) * d;
                const uint16_t* c = ct + (start_pos + s) * half;
                const uint16_t* sn = st + (start_pos + s) * half;
                for (size_t i = 0; i < vh; i++) {        /* :648-660 */
                    const uint16_t x1 = X[off + i], x2 = X[off + i + half];
                    Y[off + i] = orc_hfma(x2 ^ 0x8000u, sn[i], orc_hmul(x1, c[i]));
                    Y[off + i + half] = orc_hfma(x1, sn[i], orc_hmul(x2, c[i]));
                }
                for (size_t i = vh; i < half; i++) {     /* :662-671, promoted to float */
                    const float x1 = orc_h2f(X[off + i]), x2 = orc_h2f(X[off + i + half]);
                    const float cf = orc_h2f(c[i]), sf = orc_h2f(sn[i]);
                    Y[off + i] = orc_f2h(x1 * cf - x2 * sf);
                    Y[off + i + half] = orc_f2h(x2 * cf + x1 * sf);
                }
            }
    free(ct);
    free(st);
}

/* ------------------------------------------------------------------------ */
/* a10: cactus_softmax_f16 (kernel_nn.cpp:152-251)                           */
/* ------------------------------------------------------------------------ */
void orc_softmax_f16(const uint16_t* X, uint16_t* Y, size_t rows, size_t V) {
    const size_t vv = (V / 32) * 32;
    for (size_t r = 0; r < rows; r++) {
        const uint16_t* x = X + r * V;
        uint16_t* y = Y + r * V;
        float mx = -INFINITY;
        for (size_t i = 0; i < V; i++) mx = fmaxf(mx, orc_h2f(x[i]));
        float sv[8][4] = {{0}};
        for (size_t i = 0; i < vv; i++) {
            const float e = orc_fast_exp(orc_h2f(x[i]) - mx);
            y[i] = orc_f2h(e);
            const size_t w = i % 32;
            sv[w / 4][w % 4] = sv[w / 4][w % 4] + e;
        }
        float t[4];
        for (int l = 0; l < 4; l++) {
            float a = sv[0][l];
            for (int u = 1; u < 8; u++) a = a + sv[u][l];
            t[l] = a;
        }
        float sum = (t[0] + t[1]) + (t[2] + t[3]);
        for (size_t i = vv; i < V; i++) {
            const float e = orc_expf(orc_h2f(x[i]) - mx);
            y[i] = orc_f2h(e);
            sum = sum + e;
        }
        const float inv = 1.0f / sum;
        const uint16_t hinv = orc_f2h(inv);
        for (size_t i = 0; i < vv; i++) y[i] = orc_hmul(y[i], hinv);
        for (size_t i = vv; i < V; i++) y[i] = orc_f2h(orc_h2f(y[i]) * inv);
    }
}

/* ------------------------------------------------------------------------ */
/* a11: cactus_silu_f16 (kernel_nn.cpp:12-44), single-thread chunking        */
/* ------------------------------------------------------------------------ */
void orc_silu_f16(const uint16_t* X, uint16_t* Y, size_t n) {
    const size_t body = (n / 8) * 8;
    for (size_t i = 0; i < body; i++) {
        const float x = orc_h2f(X[i]);
        const float e = orc_fast_exp(-x);
        const float sig = 1.0f / (1.0f + e);
        Y[i] = orc_f2h(x * sig);
    }
    for (size_t i = body; i < n; i++) {
        const float x = orc_h2f(X[i]);
        const float sig = 1.0f / (1.0f + orc_expf(-x));
        Y[i] = orc_f2h(x * sig);
    }
}

/* ------------------------------------------------------------------------ */
/* a12: cactus_add_f16 / cactus_multiply_f16 (kernel_blas.cpp:187-316)       */
/* ------------------------------------------------------------------------ */
void orc_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_hadd(a[i], b[i]);
}
void orc_multiply_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_hmul(a[i], b[i]);
}

/* ------------------------------------------------------------------------ */
/* a13/a14                                                                   */
/* ------------------------------------------------------------------------ */
/* compute_embedding_node, FP16 table + FP32 ids (graph_ops_tensor.cpp:301-329) */
int orc_embedding_f16(const uint16_t* table, const float* ids, uint16_t* out, size_t n,
                      size_t hidden, size_t vocab) {
    for (size_t i = 0; i < n; i++) {
        const size_t idx = (size_t)ids[i];
        if (idx >= vocab) return -1;
        memcpy(out + i * hidden, table + idx * hidden, hidden * sizeof(uint16_t));
    }
    return 0;
}

/* cactus_sample_f16 greedy branch (kernel_nn.cpp:451-466): first index wins */
uint32_t orc_argmax_f16(const uint16_t* logits, size_t V) {
    if (V == 0) return 0;
    size_t best = 0;
    float bv = orc_h2f(logits[0]);
    for (size_t i = 1; i < V; i++) {
        const float v = orc_h2f(logits[i]);
        if (v > bv) { bv = v; best = i; }
    }
    return (uint32_t)best;
}
