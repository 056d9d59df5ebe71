// decode.hip -- fused kernels of one Qwen3 decode step (batch 1, one token).
//
// Each kernel computes a run of consecutive graph nodes of
// QwenModel::forward (models/model_qwen.cpp:51-172) for one token with
// exactly the reference's arithmetic, reading the step's token, position
// and cache length from a small device "step state" so that a whole decode
// step can be captured once into a HIP graph and replayed:
//
//   state[0] token    state[1] position    state[2] cache length    state[3] step
//
//   embed       h = embedding[token]                          (graph_ops_tensor.cpp:301-329)
//   qkv         x = rms_norm(h); q|k|v = matmul(x, Wq|Wk|Wv)  (graph_ops_nn.cpp:129-251)
//   attn_prep   q/k head RMSNorm, RoPE at `position`, INT8 append of k and v
//               at `cache length` (kernel_attention.cpp:484-676, kernel_quants.cpp:223-293)
//   attention   hybrid INT8-cache attention            (attention.hip)
//   residual    h = h + matmul(x, W)                      (o-proj, MLP down)
//   mlp_up      x = rms_norm(h); m = silu(x Wg) * (x Wu)  (kernel_nn.cpp:12-44, kernel_blas.cpp:291-316)
//   lm_head     token = argmax(rms_norm(h) E^T); the last workgroup advances
//               the step state (engine_model.cpp:221-297)
#include "gemv_device.h"
#include "lm_device.h"
#include "decode_device.h"

namespace cactus_hip {

int attention_hybrid_decode(const uint16_t* q, const int8_t* kc, const int8_t* vc, const float* ks,
                            const float* vs, const uint16_t* k_new, const uint16_t* v_new,
                            uint16_t* o, int Hq, int Hkv, int d, float scale, const uint32_t* state,
                            size_t max_cache, const float* v_shadow, size_t shadow_tiles, void* stream);
int attention_hybrid_decode_prep(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                 const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                 const uint16_t* cos_t, const uint16_t* sin_t, uint32_t table_pos,
                                 int8_t* kc, int8_t* vc, float* ks, float* vs, float* v_shadow,
                                 uint16_t* o, int Hq, int Hkv, int d, float scale, const uint32_t* state,
                                 size_t max_cache, size_t shadow_tiles, void* stream);

// ----------------------------------------------------------------- embed
__global__ void dec_embed_kernel(const uint16_t* __restrict__ table, const uint32_t* __restrict__ st,
                                 uint16_t* __restrict__ h, int hidden, uint32_t vocab) {
    const uint32_t tok = st[0];
    const bool ok = tok < vocab;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x)
        h[i] = ok ? table[(size_t)tok * hidden + i] : (uint16_t)0;
}

// ----------------------------------------------------------------- GEMV
enum { PRO_PLAIN = 0, PRO_NORM = 1 };
constexpr int DEC_SCL = 2;   // group scales per thread of a decode matmul tile
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SILUMUL = 2 };

struct DecSeg {
    const uint8_t* B;        // weights [N][K] int8 or [N][K/2] packed int4
    const uint16_t* Bs;      // [N][K/gs] fp16
    uint16_t* out;           // [N]
    int N;
};

struct DecGemvArgs {
    const uint16_t* x;       // activation [K]
    const uint16_t* norm_w;  // RMSNorm weight [K] (PRO_NORM)
    const uint16_t* res;     // residual [N] (EPI_RESID); may alias seg[0].out
    float eps;
    int K, gs, rows;
    DecSeg seg[3];
};

// LDS row strides of the group sums (floats) and scales (halves): whole
// 16-byte (8-byte) vectors per row, plus 16 bytes so that consecutive rows
// start four banks apart
__host__ __device__ inline int dec_acc_stride(int G) { return ((G + 3) & ~3) + 4; }
__host__ __device__ inline int dec_scl_stride(int G) { return ((G + 3) & ~3) + 8; }

// grid.x: row tiles, grid.y: segment (EPI_SILUMUL: one tile covers `rows`
// gate rows of seg[0] and the same rows of the up projection seg[1])
template <int PRO, int EPI, bool INT4, int CH>
__global__ void __launch_bounds__(GEMV_THREADS) dec_gemv_kernel(DecGemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = a.K, gs = a.gs, G = K / gs;
    const int rows = a.rows;
    const int tid = threadIdx.x;
    const int si = EPI == EPI_SILUMUL ? 0 : (int)blockIdx.y;
    const DecSeg sg = si == 0 ? a.seg[0] : (si == 1 ? a.seg[1] : a.seg[2]);
    const int n0 = blockIdx.x * rows;
    if (n0 >= sg.N) return;
    const int nr = min(rows, sg.N - n0);
    const int vrows = EPI == EPI_SILUMUL ? 2 * rows : rows;   // virtual rows of the tile

    int8_t* actq = reinterpret_cast<int8_t*>(smem);                          // K
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem + ((K + 15) & ~15));     // K
    // group sums (as float) and scales per virtual row, rows padded so that
    // the rows' epilogue chains read distinct LDS banks
    const int AP = dec_acc_stride(G), SP = dec_scl_stride(G);
    float* accf = reinterpret_cast<float*>(xs + ((K + 7) & ~7) + 16 * RMS_T_PAD);   // vrows*AP
    uint16_t* scl = reinterpret_cast<uint16_t*>(accf + vrows * AP);          // vrows*SP
    float* red = reinterpret_cast<float*>(scl + vrows * SP);                  // 8

    const int cpr = INT4 ? K / 32 : K / 16;
    const int P = INT4 ? gs / 32 : gs / 16;
    const size_t row_bytes = INT4 ? (size_t)K / 2 : (size_t)K;
    auto row_ptr = [&](int vr) -> const uint8_t* {
        if (EPI == EPI_SILUMUL && vr >= rows) return a.seg[1].B + (size_t)(n0 + vr - rows) * row_bytes;
        return sg.B + (size_t)(n0 + vr) * row_bytes;
    };
    auto vrow_valid = [&](int vr) { return EPI == EPI_SILUMUL ? ((vr < rows ? vr : vr - rows) < nr) : vr < nr; };

    // 1. loads, in the order they are needed: the activation row (and the
    // RMSNorm weights, the residual) first -- the prologue waits for these
    // only, its loads being the oldest in flight -- then the weight tile,
    // then the group scales into registers
    constexpr int CPT = 4;    // activation chunks of 8 per thread (K <= 8192)
    const int nch = K / 8;
    uint4 xv[CPT], wv[CPT];
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int c = tid + j * GEMV_THREADS;
        xv[j] = make_uint4(0, 0, 0, 0);
        wv[j] = make_uint4(0, 0, 0, 0);
        if (c < nch) {
            xv[j] = reinterpret_cast<const uint4*>(a.x)[c];
            if (PRO == PRO_NORM) wv[j] = reinterpret_cast<const uint4*>(a.norm_w)[c];
        }
    }
    // the residual of this thread's first row (clamped row: branch-free, so
    // no wait is forced here)
    uint16_t resv = 0;
    if (EPI == EPI_RESID) resv = a.res[n0 + min(tid, nr - 1)];
    i32x4 wreg[CH];
    int crow[CH], ccol[CH];
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + i * GEMV_THREADS;
        crow[i] = c / cpr;
        ccol[i] = c - crow[i] * cpr;
        // branch-free: a chunk outside the tile reads row 0 of the tile and
        // its dot product is dropped below
        const int vr = crow[i] < vrows && vrow_valid(crow[i]) ? crow[i] : 0;
        wreg[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(row_ptr(vr) + (size_t)ccol[i] * 16));
    }
    // group scales: at most DEC_SCL per thread (checked by the launcher),
    // loaded branch-free from clamped entries and zeroed when stored, so the
    // compiler does not wait for them (nor for the weights before them) here
    uint16_t sreg[DEC_SCL];
    bool sval[DEC_SCL];
#pragma unroll
    for (int u = 0; u < DEC_SCL; u++) {
        const int i = tid + u * GEMV_THREADS;
        const int vr = i < vrows * G ? i / G : 0, g = i < vrows * G ? i % G : 0;
        sval[u] = i < vrows * G && vrow_valid(vr);
        const bool up = EPI == EPI_SILUMUL && vr >= rows;
        const int r = sval[u] ? (up ? vr - rows : vr) : 0;
        sreg[u] = (up && sval[u] ? a.seg[1].Bs : sg.Bs)[(size_t)(n0 + r) * G + g];
    }
    // 2. activation: optional RMSNorm, then per-row quantization.  Thread t
    // owns the 8-element chunks t + 256 j in registers; the LDS copy feeds
    // the RMS chains.
    auto elem = [](const uint4& v, int e) -> uint16_t {
        const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
        return (uint16_t)(e & 1 ? w >> 16 : w & 0xFFFF);
    };
    auto set_elem = [](uint4& v, int e, uint16_t h) {
        uint32_t& w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
        w = e & 1 ? (w & 0xFFFFu) | ((uint32_t)h << 16) : (w & 0xFFFF0000u) | h;
    };
    if (PRO == PRO_NORM) {
        // rows of a multiple of 128 values go chain-major into LDS (the RMS
        // chains then read 64 values per wait), others as they are
        const bool chain_major = (K & 127) == 0;
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int c = tid + j * GEMV_THREADS;
            if (c < nch) {
                if (chain_major) {
#pragma unroll
                    for (int e = 0; e < 8; e++) xs[rms_t_index(8 * c + e, K)] = elem(xv[j], e);
                } else {
                    reinterpret_cast<uint4*>(xs)[c] = xv[j];
                }
            }
        }
        __syncthreads();
        if (tid < 64) {
            float inv;
            uint16_t hinv;
            if (chain_major) rms_stats_wave_t(xs, K, a.eps, inv, hinv);
            else rms_stats_wave(xs, K, a.eps, inv, hinv);
            if (tid == 0) { red[4] = inv; red[5] = __builtin_bit_cast(float, (uint32_t)hinv); }
        }
        __syncthreads();
        const float inv = red[4];
        const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, red[5]);
        const int end8 = (K / 8) * 8;
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int c = tid + j * GEMV_THREADS;
            if (c < nch) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    set_elem(xv[j], e, rms_apply(elem(xv[j], e), elem(wv[j], e), 8 * c + e, end8, inv, hinv));
            }
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < CPT; j++)
        if (tid + j * GEMV_THREADS < nch)
#pragma unroll
            for (int e = 0; e < 8; e++) m = __builtin_fmaxf(m, __builtin_fabsf(h2f(elem(xv[j], e))));
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float mx = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float as = row_scale_from_max(mx);
    const float inv_s = 1.0f / as;
    const int body = (K / 8) * 8;
    // the 8 codes of a chunk in its own 8 bytes (INT4: its H and L dwords
    // in the row's two planes, nib_store8)
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int c = tid + j * GEMV_THREADS;
        if (c < nch) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int i = 8 * c + e;
                const uint32_t code = (uint8_t)quant_code(h2f(elem(xv[j], e)), inv_s, i >= body);
                if (e < 4) lo |= code << (8 * e);
                else hi |= code << (8 * (e - 4));
            }
            if (INT4) nib_store8(actq, K, c, nib_pack8(lo, hi));
            else *reinterpret_cast<uint2*>(actq + 8 * c) = make_uint2(lo, hi);
        }
    }
    __syncthreads();

    // 3. dot products and exact group sums; then the group scales, the last
    // loads issued, go to LDS for the epilogue (stored here rather than with
    // the codes, so that the codes barrier does not wait for the weights)
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const bool valid = crow[i] < vrows && vrow_valid(crow[i]);
        int dot = valid ? chunk_dot<INT4>(actq, ccol[i], wreg[i], K / 2) : 0;
        dot = group_lane_sum(dot, P);
        if (valid && ((tid + i * GEMV_THREADS) & (P - 1)) == 0)
            accf[crow[i] * AP + (ccol[i] * (INT4 ? 32 : 16)) / gs] = (float)dot;   // the epilogue's conversion
    }
#pragma unroll
    for (int u = 0; u < DEC_SCL; u++)
        if (tid + u * GEMV_THREADS < vrows * G) {
            const int i = tid + u * GEMV_THREADS;
            scl[(i / G) * SP + i % G] = sval[u] ? sreg[u] : (uint16_t)0;
        }
    __syncthreads();

    // 4. reference epilogue
    // one row's chain over its G groups, 4 groups per LDS read (the fp16
    // scales enter the FMAs unconverted, as mixed-precision operands); the
    // next 16 groups are read while the current 16 FMAs run
    auto chain = [&](int vr) {
        float rs = 0.0f;
        const float* ar = accf + vr * AP;
        const uint16_t* sr = scl + vr * SP;
        const int G16 = G & ~15;
        typedef float f4v __attribute__((ext_vector_type(4)));
        f4v av[2][4];
        uint2 sv[2][4];
        auto load16 = [&](int h, int gb) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                av[h][j] = *reinterpret_cast<const f4v*>(ar + gb + 4 * j);
                sv[h][j] = *reinterpret_cast<const uint2*>(sr + gb + 4 * j);
            }
        };
        if (G16 > 0) load16(0, 0);
        for (int g = 0; g < G16; g += 32) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int gb = g + 16 * h;
                if (gb < G16) {
                    load16(h ^ 1, min(gb + 16, G16 - 16));   // clamped prefetch: re-reads the last block
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t s01 = sv[h][j].x, s23 = sv[h][j].y;
                        rs = __builtin_fmaf(av[h][j][0], h2f((uint16_t)(s01 & 0xFFFFu)), rs);
                        rs = __builtin_fmaf(av[h][j][1], h2f((uint16_t)(s01 >> 16)), rs);
                        rs = __builtin_fmaf(av[h][j][2], h2f((uint16_t)(s23 & 0xFFFFu)), rs);
                        rs = __builtin_fmaf(av[h][j][3], h2f((uint16_t)(s23 >> 16)), rs);
                    }
                }
            }
        }
        for (int g = G16; g < G; g++) rs = __builtin_fmaf(ar[g], h2f(sr[g]), rs);
        return f2h(rs * as);
    };
    auto silu_mul = [&](int r, uint16_t val, uint16_t up) {
        const float gx = h2f(val);
        // silu's vector body uses fast_exp, its n % 8 tail expf (kernel_nn.cpp:12-44)
        const float e = n0 + r < (sg.N / 8) * 8 ? fast_exp(-gx) : cactus_expf(-gx);
        const float sig = 1.0f / (1.0f + e);
        sg.out[n0 + r] = hmul(f2h(gx * sig), up);
    };
    if constexpr (EPI == EPI_SILUMUL) {
        // gate rows on lanes 0..rows-1 of wave 0 and up rows on lanes
        // rows..2 rows-1: both chains in one instruction stream, then the up
        // value moves to its gate lane
        if (2 * rows <= 64) {
            if (tid < 64) {                                  // wave 0, uniform
                uint16_t val = 0;
                if (tid < 2 * rows && vrow_valid(tid)) val = chain(tid);
                const uint16_t up = (uint16_t)__shfl((int)val, tid + rows, 64);
                if (tid < nr) silu_mul(tid, val, up);
            }
            return;
        }
    }
    for (int r = tid; r < nr; r += GEMV_THREADS) {
        const uint16_t val = chain(r);
        if (EPI == EPI_STORE) {
            sg.out[n0 + r] = val;
        } else if (EPI == EPI_RESID) {
            sg.out[n0 + r] = hadd(r == tid ? resv : a.res[n0 + r], val);
        } else {
            silu_mul(r, val, chain(rows + r));
        }
    }
}

static size_t dec_gemv_smem(int K, int vrows, int G) {
    size_t s = (size_t)((K + 15) & ~15) + ((size_t)((K + 7) & ~7) + 16 * RMS_T_PAD) * 2;
    s += (size_t)vrows * dec_acc_stride(G) * 4 + (size_t)vrows * dec_scl_stride(G) * 2 + 8 * 4;
    return (s + 15) & ~(size_t)15;
}

template <int PRO, int EPI, bool INT4>
static int launch_dec_gemv(DecGemvArgs a, int nseg, hipStream_t st) {
    const int G = a.K / a.gs;
    const int cpr = INT4 ? a.K / 32 : a.K / 16;
    const int vmul = EPI == EPI_SILUMUL ? 2 : 1;
    int maxN = 0, totalN = 0;
    for (int s = 0; s < nseg; s++) { maxN = max(maxN, a.seg[s].N); totalN += a.seg[s].N; }
    // at most 2 chunks per thread; as few rows as keep >= 512 working
    // workgroups (EPI_SILUMUL: one workgroup per tile of gate rows, its up
    // rows included -- counting both had left the Qwen3 gate/up at 384
    // workgroups, 1.5 per CU: 5.92-6.34 us per launch against 5.78-5.91
    // with 768)
    int rows = (2 * GEMV_THREADS) / (cpr * vmul);
    if (rows < 1) rows = 1;
    const int work_rows = EPI == EPI_SILUMUL ? maxN : totalN;
    while (rows > 1 && (size_t)ceil_div(work_rows, rows) < 512) rows = (rows + 1) / 2;
    CH_REQUIRE(rows * cpr * vmul <= 2 * GEMV_THREADS, "decode matmul: K too large");
    CH_REQUIRE(rows * vmul * G <= DEC_SCL * GEMV_THREADS, "decode matmul: too many groups per tile");
    a.rows = rows;
    const int ch = (rows * cpr * vmul + GEMV_THREADS - 1) / GEMV_THREADS;
    const size_t smem = dec_gemv_smem(a.K, rows * vmul, G);
    CH_REQUIRE(smem <= 60 * 1024, "decode matmul: K too large for LDS");
    dim3 grid(ceil_div(maxN, rows), EPI == EPI_SILUMUL ? 1 : nseg);
    if (ch <= 1)
        hipLaunchKernelGGL((dec_gemv_kernel<PRO, EPI, INT4, 1>), grid, dim3(GEMV_THREADS), smem, st, a);
    else
        hipLaunchKernelGGL((dec_gemv_kernel<PRO, EPI, INT4, 2>), grid, dim3(GEMV_THREADS), smem, st, a);
    return check_launch("decode matmul");
}

// ----------------------------------------------------------------- attn prep
// grid: Hq + Hkv workgroups of one wave.  Workgroup h < Hq: q head h
// (RMSNorm, RoPE).  Workgroup Hq + g: k head g (RMSNorm, RoPE, INT8 append)
// and v head g (INT8 append), at the cache length of the step state.
struct PrepArgs {
    const uint16_t* q_raw; const uint16_t* k_raw; const uint16_t* v_raw;
    const uint16_t* q_norm; const uint16_t* k_norm;
    uint16_t* q_out; uint16_t* k_out;
    int8_t* kc; int8_t* vc; float* ks; float* vs;
    const uint16_t* cos_t; const uint16_t* sin_t;
    const uint32_t* st;
    float eps;
    int Hq, Hkv, d;
    uint32_t max_cache;
    uint32_t table_pos;      // positions held by the RoPE tables
    float* vsh;              // value product tiles or null
    size_t sh_ntile;
};

__global__ void __launch_bounds__(64) dec_attn_prep_kernel(PrepArgs a) {
    __shared__ uint16_t xs[256];
    __shared__ uint16_t ys[256];
    const int lane = threadIdx.x;
    const int d = a.d, half = d / 2, end8 = (d / 8) * 8;
    const uint32_t pos = a.st[1];
    const uint32_t clen = a.st[2];
    if (pos >= a.table_pos) return;   // the host keeps positions inside the table
    const bool is_q = (int)blockIdx.x < a.Hq;
    const int h = is_q ? blockIdx.x : blockIdx.x - a.Hq;
    const uint16_t* src = is_q ? a.q_raw + (size_t)h * d : a.k_raw + (size_t)h * d;
    const uint16_t* nw = is_q ? a.q_norm : a.k_norm;
    uint16_t* out = is_q ? a.q_out + (size_t)h * d : a.k_out + (size_t)h * d;
    for (int i = lane; i < d; i += 64) xs[i] = src[i];
    __syncthreads();
    float inv;
    uint16_t hinv;
    rms_stats_wave(xs, d, a.eps, inv, hinv);
    for (int i = lane; i < d; i += 64) ys[i] = rms_apply(xs[i], nw[i], i, end8, inv, hinv);
    __syncthreads();
    // RoPE at absolute position `pos`; the roped row stays in xs for the
    // cache append
    rope_row(ys, d, a.cos_t + (size_t)pos * half, a.sin_t + (size_t)pos * half, [&](int i, uint16_t v) {
        out[i] = v;
        xs[i] = v;
    });
    __syncthreads();
    if (!is_q && clen < a.max_cache) {
        const int ng = (d + 127) / 128;
        const size_t row = (size_t)clen * a.Hkv + h;
        kv_append_row(xs, a.kc + row * d, a.ks + row * ng, d);
        kv_append_row(a.v_raw + (size_t)h * d, a.vc + row * d, a.vs + row * ng, d, a.vsh, a.sh_ntile, clen, h);
    }
}

// ----------------------------------------------------------------- LM head
// RMSNorm of h in every workgroup's prologue, then the FP16-accumulation
// GEMV of kernel_gemm.cpp:17-126 against the tied embedding and the greedy
// argmax (first index wins); the last workgroup also advances the state.
struct LmDecArgs {
    const uint16_t* h; const uint16_t* norm_w; const uint16_t* b;
    float eps;
    int K, N;
    uint32_t* counter;       // scratch: counter at byte 0, argmax key at byte 8
    uint32_t* st;            // token, pos, cache_len, step
    uint32_t* tokens_out;    // [max_steps] or null
    uint32_t max_steps;
    uint16_t* logits_out;    // fp16 [N] or null
    // or null: the next step's input row, embed[token] ([N][K] fp16), is
    // written to h_next by the last workgroup (zeros for a token >= N)
    const uint16_t* embed;
    uint16_t* h_next;
};

// Greedy argmax over the rows of all workgroups and the step state's
// advance by the last workgroup to finish; every thread passes its row's
// (value, index) or index 0xFFFFFFFF for none.  The reference's argmax
// (first index wins; a NaN logit at index 0 is never beaten, any other NaN
// never wins) is a maximum over 64-bit keys: the value's bits in an
// order-preserving form, then 0xFFFFFFFF - index.  Each workgroup posts its
// best key with one atomic max, waits for that atomic to be performed, then
// counts itself done; the last one reads the maximum back with an atomic.
// Only atomics carry data between workgroups, so no cache writeback fence
// is needed (an agent-scope release per workgroup -- an L2 writeback on
// this GPU -- cost the 151936-row head ~20 us).  Scratch: the counter at
// byte 0, the key at byte 8; both are left zero.
__device__ __forceinline__ unsigned long long lm_argmax_key(float v, uint32_t idx) {
    if (idx == 0xFFFFFFFFu) return 0ull;
    if (v != v) return idx == 0 ? ~0ull : 0ull;
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xFFFFFFFFu - idx);
}

template <int THREADS>
__device__ __forceinline__ void lm_argmax_finish(const LmDecArgs& p, float best, uint32_t best_i) {
    static_assert(THREADS % 64 == 0 && THREADS <= 1024, "whole waves");
    __shared__ unsigned long long wk[THREADS / 64];
    __shared__ bool last;
    unsigned long long key = lm_argmax_key(best, best_i);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(key, off, 64);
        key = o > key ? o : key;
    }
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = key;
    __syncthreads();
    unsigned long long* kp = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(p.counter) + 8);
    if (threadIdx.x == 0) {
        unsigned long long m = wk[0];
        for (int w = 1; w < THREADS / 64; w++) m = wk[w] > m ? wk[w] : m;
        // returning atomic, then a wait that takes its result as an input:
        // the atomic has been performed before this workgroup counts
        // itself done
        const unsigned long long old = atomicMax(kp, m);
        asm volatile("s_waitcnt vmcnt(0)" ::"v"((uint32_t)old), "v"((uint32_t)(old >> 32)) : "memory");
        last = atomicAdd(p.counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last || threadIdx.x != 0) return;
    const unsigned long long m = atomicMax(kp, 0ull);     // every workgroup's key is in
    const uint32_t tok = m == 0ull ? 0u : 0xFFFFFFFFu - (uint32_t)m;
    const uint32_t step = p.st[3];
    if (p.tokens_out && step < p.max_steps) p.tokens_out[step] = tok;
    p.st[0] = tok;
    p.st[1] = p.st[1] + 1;
    p.st[2] = p.st[2] + 1;
    p.st[3] = step + 1;
    atomicExch(kp, 0ull);
    atomicExch(p.counter, 0u);
}

// The same argmax and state update for a grid whose workgroups finish
// close together (one per CU): 238 returning atomics on one address then
// queue behind each other (~14 us measured for the 151936-row head), so the
// count is two-level.  Workgroup i stores its key in slot i and, once the
// store has been performed, counts itself in group counter i % 8; the last
// of a group counts the group in the top counter; the last overall reads
// every slot, reduces them, advances the state and clears the counters.
// Scratch: top counter at byte 0, group counters at bytes 64 + 64 g, slots
// (8 bytes per workgroup) from byte 1024; counters are left zero.
constexpr int LMG_GROUPS = 8;
constexpr size_t LMG_SLOTS = 1024;
template <int THREADS>
__device__ __forceinline__ void lm_argmax_finish_groups(const LmDecArgs& p, float best, uint32_t best_i) {
    static_assert(THREADS % 64 == 0 && THREADS <= 1024, "whole waves");
    __shared__ unsigned long long wk[THREADS / 64];
    __shared__ bool last;
    auto block_max = [&](unsigned long long key) -> unsigned long long {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(key, off, 64);
            key = o > key ? o : key;
        }
        if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = key;
        __syncthreads();
        unsigned long long m = wk[0];
        for (int w = 1; w < THREADS / 64; w++) m = wk[w] > m ? wk[w] : m;
        return m;
    };
    char* base = reinterpret_cast<char*>(p.counter);
    unsigned long long* slots = reinterpret_cast<unsigned long long*>(base + LMG_SLOTS);
    const unsigned long long m = block_max(lm_argmax_key(best, best_i));
    if (threadIdx.x == 0) {
        const unsigned g = blockIdx.x % LMG_GROUPS;
        const unsigned ngroups = gridDim.x < LMG_GROUPS ? gridDim.x : LMG_GROUPS;
        const unsigned in_group = (gridDim.x - g + LMG_GROUPS - 1) / LMG_GROUPS;
        __hip_atomic_store(slots + blockIdx.x, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);              // the slot store is performed before the count
        bool l = atomicAdd(reinterpret_cast<uint32_t*>(base + 64 + 64 * g), 1u) == in_group - 1;
        if (l) l = atomicAdd(p.counter, 1u) == ngroups - 1;
        last = l;
    }
    __syncthreads();
    if (!last) return;
    unsigned long long k = 0ull;
    for (unsigned i = threadIdx.x; i < gridDim.x; i += THREADS) {
        const unsigned long long v = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        k = v > k ? v : k;
    }
    __syncthreads();                                 // wk reused
    const unsigned long long mm = block_max(k);
    const uint32_t tok = mm == 0ull ? 0u : 0xFFFFFFFFu - (uint32_t)mm;
    if (p.h_next) {
        // the next step's embedding row (every workgroup has read h by now)
        const bool ok = tok < (uint32_t)p.N;
        const uint4* src = reinterpret_cast<const uint4*>(p.embed + (size_t)(ok ? tok : 0u) * p.K);
        for (int c = threadIdx.x; c < p.K / 8; c += THREADS)
            reinterpret_cast<uint4*>(p.h_next)[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
    }
    if (threadIdx.x != 0) return;
    const uint32_t step = p.st[3];
    if (p.tokens_out && step < p.max_steps) p.tokens_out[step] = tok;
    p.st[0] = tok;
    p.st[1] = p.st[1] + 1;
    p.st[2] = p.st[2] + 1;
    p.st[3] = step + 1;
    for (int g = 0; g < LMG_GROUPS; g++) atomicExch(reinterpret_cast<uint32_t*>(base + 64 + 64 * g), 0u);
    atomicExch(p.counter, 0u);
}

// LM head + greedy argmax, streamed: each wave owns 64 vocabulary rows (one
// per lane) and moves them through its own ring of LMS_D slots by LDS DMA
// (LMS_KC k-values of 64 rows per slot), LMS_D - 1 chunks ahead, with no
// cross-wave barrier in the K loop.  Consecutive lanes fetch consecutive
// 16-byte pieces of one row; piece p of row r sits in slot position
// p ^ (r % pieces per row), so the per-lane row reads of one piece spread
// over the banks.
// Each lane's dot is the reference's 8-lane fp16 accumulation in k order.
// Ten waves per workgroup (one RMSNorm prologue) with three 4 KB slots
// each: the 151936 x 1024 Qwen3 head is 238 workgroups, at most one per CU
// (a workgroup takes ~130 KB of LDS).  Measured on MI355X, standalone: 67 us
// against 74-78 us for eight waves with two 8 KB slots (297 workgroups, so
// 41 CUs ran two in turn), 71.5 us for twelve waves, 85-106 us with 2 KB
// slots; 101 us for two waves.
constexpr int LMS_WAVES = 10, LMS_THREADS = 64 * LMS_WAVES;
constexpr int LMS_KC = 32;                              // k-values per chunk
constexpr int LMS_D = 3;                                // ring slots per wave
constexpr int LMS_SLOT = 64 * LMS_KC * 2;               // 4 KB
constexpr int LMS_NI = LMS_SLOT / 1024;                 // DMA instructions per chunk
static_assert(LMS_D >= 2 && LMS_D <= 4, "wait counts below");

__global__ void __launch_bounds__(LMS_THREADS) dec_lm_head_stream_kernel(LmDecArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = p.K, N = p.N;
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                // K
    uint16_t* as = xs + K;                                          // K (normed)
    unsigned char* ring = smem + 4 * (size_t)K + wid * LMS_D * LMS_SLOT;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)ring;
    __shared__ float stats[2];
    const int row0 = (blockIdx.x * LMS_WAVES + wid) * 64;
    const int nk = K / LMS_KC;

    // DMA sources: a row's chunk is PPR 16-byte pieces; instruction j moves
    // rows (64 / PPR) j + lane / PPR, piece (lane % PPR) ^ (row % PPR)
    constexpr int PPR = LMS_KC / 8;
    const uint16_t* src[LMS_NI];
#pragma unroll
    for (int j = 0; j < LMS_NI; j++) {
        const int r = (64 / PPR) * j + lane / PPR;
        const int pc = (lane % PPR) ^ (r % PPR);
        src[j] = p.b + (size_t)min(row0 + r, N - 1) * K + pc * 8;
    }
    auto issue = [&](int k) {
        const uint32_t slot = ring_lds + (uint32_t)((k % LMS_D) * LMS_SLOT);
#pragma unroll
        for (int j = 0; j < LMS_NI; j++) lds_dma<16>(src[j] + (size_t)k * LMS_KC, slot + j * 1024);
    };
    for (int k = 0; k < LMS_D - 1; k++)
        if (k < nk) issue(k);

    for (int i = threadIdx.x; i < K; i += LMS_THREADS) xs[i] = p.h[i];
    __syncthreads();
    if (wid == 0) {
        float inv;
        uint16_t hinv;
        rms_stats_wave(xs, K, p.eps, inv, hinv);
        if (lane == 0) { stats[0] = inv; stats[1] = __builtin_bit_cast(float, (uint32_t)hinv); }
    }
    __syncthreads();
    {
        const float inv = stats[0];
        const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, stats[1]);
        const int end8 = (K / 8) * 8;
        for (int i = threadIdx.x; i < K; i += LMS_THREADS) as[i] = rms_apply(xs[i], p.norm_w[i], i, end8, inv, hinv);
    }
    __syncthreads();

    h2v acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = (h2v){(f16)0.0f, (f16)0.0f};
    const unsigned char* rowp = ring + lane * (LMS_KC * 2);
    for (int k = 0; k < nk; k++) {
        // chunk k landed once at most the younger chunks k + 1 .. k + D - 2
        // fly (this wave's own DMA)
        {
            const int younger = min(LMS_D - 2, nk - 1 - k);
            if (younger >= 2) wait_dma<2 * LMS_NI>();
            else if (younger == 1) wait_dma<LMS_NI>();
            else wait_dma<0>();
        }
        // slot of chunk k - 1: read (into registers) during the previous step
        if (k + LMS_D - 1 < nk) issue(k + LMS_D - 1);
        const unsigned char* rp = rowp + (k % LMS_D) * LMS_SLOT;
#pragma unroll
        for (int ch = 0; ch < LMS_KC / 8; ch++) {
            const uint4 bv = *reinterpret_cast<const uint4*>(rp + ((ch ^ (lane % PPR)) * 16));
            const uint4 av = *reinterpret_cast<const uint4*>(as + k * LMS_KC + ch * 8);
            f16_step(acc, av, bv);
        }
    }
    const int my_row = row0 + lane;
    float best = -__builtin_inff();
    uint32_t best_i = 0xFFFFFFFFu;
    if (my_row < N) {
        const uint16_t logit = f16_hsum(acc);   // fp16 bits
        if (p.logits_out) p.logits_out[my_row] = logit;
        best = h2f(logit);
        best_i = (uint32_t)my_row;
    }
    lm_argmax_finish<LMS_THREADS>(p, best, best_i);
}

__global__ void __launch_bounds__(LM_THREADS) dec_lm_head_kernel(LmDecArgs p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = p.K;
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                // K
    uint16_t* as = xs + K;                                          // K (normed)
    unsigned char* stage = smem + 4 * (size_t)K + wid * LM_ROWS_PER_WAVE * LM_ROW_STRIDE;
    __shared__ float stats[2];
    for (int i = threadIdx.x; i < K; i += LM_THREADS) xs[i] = p.h[i];
    __syncthreads();
    if (wid == 0) {
        float inv;
        uint16_t hinv;
        rms_stats_wave(xs, K, p.eps, inv, hinv);
        if (lane == 0) { stats[0] = inv; stats[1] = __builtin_bit_cast(float, (uint32_t)hinv); }
    }
    __syncthreads();
    {
        const float inv = stats[0];
        const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, stats[1]);
        const int end8 = (K / 8) * 8;
        for (int i = threadIdx.x; i < K; i += LM_THREADS) as[i] = rms_apply(xs[i], p.norm_w[i], i, end8, inv, hinv);
    }
    __syncthreads();

    const int row0 = (blockIdx.x * (LM_THREADS / 64) + wid) * LM_ROWS_PER_WAVE;
    const int my_row = row0 + lane;
    h2v acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = (h2v){(f16)0.0f, (f16)0.0f};
    for (int k0 = 0; k0 < K; k0 += LM_KC) {
        const int kc = min(LM_KC, K - k0);
        const int cpr = kc / 8;
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
            const uint4 av = *reinterpret_cast<const uint4*>(as + k0 + ch * 8);
            f16_step(acc, av, bv);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    float best = -__builtin_inff();
    uint32_t best_i = 0xFFFFFFFFu;
    if (my_row < p.N) {
        const uint16_t logit = f16_hsum(acc);   // fp16 bits
        if (p.logits_out) p.logits_out[my_row] = logit;
        best = h2f(logit);
        best_i = (uint32_t)my_row;
    }
    lm_argmax_finish<LM_THREADS>(p, best, best_i);
}

// LM head over the tiled embedding (cactus_hip_lm_tiles_build), laid out
// [K/8][N rounded up to 64][8 values]: wave w's 16-byte load of step q
// (lane = row) reads the 1 KB at (q * Npad + 64 w) * 8 values -- one
// contiguous read per wave instruction, straight into registers, no LDS
// staging -- and the waves of a step read one contiguous band, so that the
// whole grid sweeps memory in order (a row-block-major layout, where the
// waves stream regions 128 KB apart, measured 87-91 us against 72 us for
// this head).  Rows are step-major for that reason only.  LMT_D loads per
// lane in flight (issued before the RMSNorm prologue, which they overlap);
// the normalized row is read from LDS by broadcast.  Each lane's dot is the
// reference's 8-lane fp16 accumulation in k order (kernel_gemm.cpp:17-126).
// Ten waves per workgroup: the 151936 x 1024 head is 238 workgroups, at most
// one per CU, so every CU streams the same ten 64-row blocks.  With four
// waves (594 workgroups) CUs ran two or three workgroups and the CUs with
// three finished ~1.5x later (per-workgroup timestamps: loop ends 26-54 us,
// the head 57-58 us in the step); with ten it takes 50.9-51.4 us.  Measured
// with four waves: 62.2 us with 8 loads in flight, 57.3-58.6 with 12, 58-59
// with 14 or 16; 8 waves per workgroup 65.0, 2 waves 67.5.
constexpr int LMT_WAVES = 10, LMT_THREADS = 64 * LMT_WAVES, LMT_D = 12;

__global__ void __launch_bounds__(LMT_THREADS) dec_lm_head_tiled_kernel(LmDecArgs p) {
    __shared__ __align__(16) uint16_t xs[4096 + 16 * RMS_T_PAD];
    __shared__ __align__(16) uint16_t as[4096];
    __shared__ float stats[2];
    const int K = p.K, N = p.N, nq = K / 8;
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int blk = (int)blockIdx.x * LMT_WAVES + wid;              // this wave's 64-row block
    const bool live = blk * 64 < N;                                  // wave-uniform
    // the row and the RMSNorm weights first: the prologue then waits for
    // them alone, while the first LMT_D steps of weights are in flight
    const int nch = K / 8;
    uint4 hv[2], wv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int c = min((int)threadIdx.x + j * LMT_THREADS, nch - 1);
        hv[j] = reinterpret_cast<const uint4*>(p.h)[c];
        wv[j] = reinterpret_cast<const uint4*>(p.norm_w)[c];
    }
    const size_t npad = ((size_t)N + 63) / 64 * 64;
    const i32x4* tp = reinterpret_cast<const i32x4*>(p.b) + (size_t)(live ? blk : 0) * 64 + lane;
    i32x4 ring[LMT_D];
#pragma unroll
    for (int u = 0; u < LMT_D; u++) ring[u] = __builtin_nontemporal_load(tp + (size_t)min(u, nq - 1) * npad);

    // RMSNorm: the row chain-major in LDS when K % 128 == 0 (16 reads per
    // chain of 64 values), as it is otherwise
    auto elem = [](const uint4& v, int e) -> uint16_t {
        const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
        return (uint16_t)(e & 1 ? w >> 16 : w & 0xFFFF);
    };
    const bool chain_major = (K & 127) == 0;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int c = (int)threadIdx.x + j * LMT_THREADS;
        if (c < nch) {
            if (chain_major) {
#pragma unroll
                for (int e = 0; e < 8; e++) xs[rms_t_index(8 * c + e, K)] = elem(hv[j], e);
            } else {
                reinterpret_cast<uint4*>(xs)[c] = hv[j];
            }
        }
    }
    __syncthreads();
    if (wid == 0) {
        float inv;
        uint16_t hinv;
        if (chain_major) rms_stats_wave_t(xs, K, p.eps, inv, hinv);
        else rms_stats_wave(xs, K, p.eps, inv, hinv);
        if (lane == 0) { stats[0] = inv; stats[1] = __builtin_bit_cast(float, (uint32_t)hinv); }
    }
    __syncthreads();
    {
        const float inv = stats[0];
        const uint16_t hinv = (uint16_t)__builtin_bit_cast(uint32_t, stats[1]);
        const int end8 = (K / 8) * 8;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int c = (int)threadIdx.x + j * LMT_THREADS;
            if (c < nch) {
#pragma unroll
                for (int e = 0; e < 8; e++) as[8 * c + e] = rms_apply(elem(hv[j], e), elem(wv[j], e), 8 * c + e, end8, inv, hinv);
            }
        }
    }
    __syncthreads();

    h2v acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = (h2v){(f16)0.0f, (f16)0.0f};
    const uint4* av4 = reinterpret_cast<const uint4*>(as);
    // whole groups of D steps (branch-free, so the compiler's wait before
    // each step is for that step's load only), then the remaining steps
    int q0 = 0;
    for (; q0 + LMT_D <= nq; q0 += LMT_D) {
#pragma unroll
        for (int u = 0; u < LMT_D; u++) {
            const int q = q0 + u;
            // the slot is used before it is refilled (with step q + D, clamped:
            // the last steps re-read step nq - 1), so each step waits for its
            // own load only and the refill takes the slot's registers.  (The
            // refill first kept the old value live past it: the compiler
            // then copied all D slots, waiting for every load, before
            // issuing any refill, and the ring drained every D steps.)
            f16_step(acc, av4[q], __builtin_bit_cast(uint4, ring[u]));
            ring[u] = __builtin_nontemporal_load(tp + (size_t)min(q + LMT_D, nq - 1) * npad);
            // keep the refill here: the scheduler would otherwise gather the
            // D refills at the end of the unrolled group
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < LMT_D; u++)
        if (q0 + u < nq) f16_step(acc, av4[q0 + u], __builtin_bit_cast(uint4, ring[u]));
    const int my_row = blk * 64 + lane;
    float best = -__builtin_inff();
    uint32_t best_i = 0xFFFFFFFFu;
    if (live && my_row < N) {
        const uint16_t logit = f16_hsum(acc);   // fp16 bits
        if (p.logits_out) p.logits_out[my_row] = logit;
        best = h2f(logit);
        best_i = (uint32_t)my_row;
    }
    lm_argmax_finish_groups<LMT_THREADS>(p, best, best_i);
}

// tiles[(q * Npad + row) * 8 + e] = embedding[row][8 q + e], 0 past N
__global__ void lm_tiles_build_kernel(const uint16_t* __restrict__ emb, uint4* __restrict__ tiles, int K, int N,
                                      size_t total) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // one 16-byte piece
    if (i >= total) return;
    const size_t npad = ((size_t)N + 63) / 64 * 64;
    const size_t row = i % npad;
    const int q = (int)(i / npad);
    tiles[i] = row < (size_t)N ? *reinterpret_cast<const uint4*>(emb + row * K + 8 * (size_t)q)
                               : make_uint4(0, 0, 0, 0);
}

}  // namespace cactus_hip

using namespace cactus_hip;

extern "C" {

int cactus_hip_decode_embed(const uint16_t* table, const uint32_t* state, uint16_t* h, size_t hidden,
                            size_t vocab, void* stream) {
    CH_REQUIRE(table && state && h && hidden > 0 && vocab > 0, "decode_embed: bad argument");
    hipLaunchKernelGGL(dec_embed_kernel, dim3(1), dim3(256), 0, as_stream(stream), table, state, h,
                       (int)hidden, (uint32_t)vocab);
    return check_launch("decode_embed");
}

int cactus_hip_decode_qkv(const uint16_t* h, const uint16_t* norm_w, float eps, size_t K,
                          size_t group_size, const int8_t* wq, const uint16_t* sq, uint16_t* q,
                          size_t nq, const int8_t* wk, const uint16_t* sk, uint16_t* k, size_t nk,
                          const int8_t* wv, const uint16_t* sv, uint16_t* v, size_t nv, void* stream) {
    CH_REQUIRE(h && norm_w && wq && sq && q && wk && sk && k && wv && sv && v, "decode_qkv: null pointer");
    CH_REQUIRE(((uintptr_t)h | (uintptr_t)norm_w) % 16 == 0, "decode_qkv: h and norm_w must be 16-byte aligned");
    CH_REQUIRE(group_size >= 16 && K % group_size == 0 && (group_size & (group_size - 1)) == 0 &&
               group_size <= 1024 && K <= 8192, "decode_qkv: bad K / group_size");
    DecGemvArgs a{};
    a.x = h; a.norm_w = norm_w; a.eps = eps; a.K = (int)K; a.gs = (int)group_size;
    a.seg[0] = {reinterpret_cast<const uint8_t*>(wq), sq, q, (int)nq};
    a.seg[1] = {reinterpret_cast<const uint8_t*>(wk), sk, k, (int)nk};
    a.seg[2] = {reinterpret_cast<const uint8_t*>(wv), sv, v, (int)nv};
    return launch_dec_gemv<PRO_NORM, EPI_STORE, false>(a, 3, as_stream(stream));
}

int cactus_hip_decode_matmul_residual(const uint16_t* x, size_t K, size_t group_size, const void* w,
                                      const uint16_t* s, size_t N, int int4, uint16_t* h,
                                      void* stream) {
    CH_REQUIRE(x && w && s && h, "decode_matmul_residual: null pointer");
    CH_REQUIRE((uintptr_t)x % 16 == 0, "decode_matmul_residual: x must be 16-byte aligned");
    CH_REQUIRE(group_size >= (int4 ? 32u : 16u) && K % group_size == 0 &&
               (group_size & (group_size - 1)) == 0 && group_size <= 1024 && K <= 8192,
               "decode_matmul_residual: bad K / group_size");
    DecGemvArgs a{};
    a.x = x; a.res = h; a.K = (int)K; a.gs = (int)group_size;
    a.seg[0] = {static_cast<const uint8_t*>(w), s, h, (int)N};
    if (int4) return launch_dec_gemv<PRO_PLAIN, EPI_RESID, true>(a, 1, as_stream(stream));
    return launch_dec_gemv<PRO_PLAIN, EPI_RESID, false>(a, 1, as_stream(stream));
}

int cactus_hip_decode_mlp_up(const uint16_t* h, const uint16_t* norm_w, float eps, size_t K,
                             size_t group_size, const uint8_t* wg, const uint16_t* sg,
                             const uint8_t* wu, const uint16_t* su, size_t N, uint16_t* m,
                             void* stream) {
    CH_REQUIRE(h && norm_w && wg && sg && wu && su && m, "decode_mlp_up: null pointer");
    CH_REQUIRE(((uintptr_t)h | (uintptr_t)norm_w) % 16 == 0, "decode_mlp_up: h and norm_w must be 16-byte aligned");
    CH_REQUIRE(group_size >= 32 && K % group_size == 0 && (group_size & (group_size - 1)) == 0 &&
               group_size <= 1024 && K <= 8192, "decode_mlp_up: bad K / group_size");
    DecGemvArgs a{};
    a.x = h; a.norm_w = norm_w; a.eps = eps; a.K = (int)K; a.gs = (int)group_size;
    a.seg[0] = {wg, sg, m, (int)N};
    a.seg[1] = {wu, su, nullptr, (int)N};
    return launch_dec_gemv<PRO_NORM, EPI_SILUMUL, true>(a, 2, as_stream(stream));
}

int cactus_hip_decode_attn_prep(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float theta,
                                const uint32_t* state, uint16_t* q_out, uint16_t* k_out,
                                int8_t* k_cache, int8_t* v_cache, float* k_scales, float* v_scales,
                                size_t max_cache, float* v_shadow, void* stream) {
    CH_REQUIRE(q_raw && k_raw && v_raw && q_norm && k_norm && state && q_out && k_out && k_cache &&
               v_cache && k_scales && v_scales, "decode_attn_prep: null pointer");
    CH_REQUIRE(head_dim >= 8 && head_dim <= 256 && head_dim % 2 == 0, "decode_attn_prep: head_dim");
    RopeTable t;
    int rc = rope_table(max_cache + 1, head_dim, theta, &t);
    if (rc) return rc;
    PrepArgs a{};
    a.q_raw = q_raw; a.k_raw = k_raw; a.v_raw = v_raw; a.q_norm = q_norm; a.k_norm = k_norm;
    a.q_out = q_out; a.k_out = k_out; a.kc = k_cache; a.vc = v_cache; a.ks = k_scales; a.vs = v_scales;
    a.cos_t = t.cos_d; a.sin_t = t.sin_d; a.st = state; a.eps = eps;
    a.Hq = (int)num_q_heads; a.Hkv = (int)num_kv_heads; a.d = (int)head_dim;
    a.max_cache = (uint32_t)max_cache;
    a.table_pos = (uint32_t)t.npos;
    a.vsh = v_shadow;
    a.sh_ntile = (max_cache + 63) / 64;
    hipLaunchKernelGGL(dec_attn_prep_kernel, dim3((unsigned)(num_q_heads + num_kv_heads)), dim3(64), 0,
                       as_stream(stream), a);
    return check_launch("decode_attn_prep");
}

int cactus_hip_decode_attention(const uint16_t* q, const int8_t* k_cache, const int8_t* v_cache,
                                const float* k_scales, const float* v_scales, const uint16_t* k_new,
                                const uint16_t* v_new, uint16_t* o, size_t num_q_heads,
                                size_t num_kv_heads, size_t head_dim, float scale,
                                const uint32_t* state, size_t max_cache, const float* v_shadow,
                                void* stream) {
    CH_REQUIRE(q && k_cache && v_cache && k_scales && v_scales && k_new && v_new && o && state,
               "decode_attention: null pointer");
    CH_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 8,
               "decode_attention: bad head counts");
    CH_REQUIRE(head_dim % 8 == 0 && head_dim <= 256, "decode_attention: head_dim");
    return attention_hybrid_decode(q, k_cache, v_cache, k_scales, v_scales, k_new, v_new, o,
                                   (int)num_q_heads, (int)num_kv_heads, (int)head_dim, scale, state,
                                   max_cache, v_shadow, (max_cache + 63) / 64, stream);
}

int cactus_hip_decode_prep_attention(const uint16_t* q_raw, const uint16_t* k_raw, const uint16_t* v_raw,
                                     const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                     size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float theta,
                                     const uint32_t* state, int8_t* k_cache, int8_t* v_cache,
                                     float* k_scales, float* v_scales, size_t max_cache, float* v_shadow,
                                     float scale, uint16_t* o, void* stream) {
    CH_REQUIRE(q_raw && k_raw && v_raw && q_norm && k_norm && state && k_cache && v_cache && k_scales &&
               v_scales && o, "decode_prep_attention: null pointer");
    CH_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, "decode_prep_attention: bad head counts");
    CH_REQUIRE(head_dim == 64 || head_dim == 128, "decode_prep_attention: head_dim must be 64 or 128");
    RopeTable t;
    int rc = rope_table(max_cache + 1, head_dim, theta, &t);
    if (rc) return rc;
    return attention_hybrid_decode_prep(q_raw, k_raw, v_raw, q_norm, k_norm, eps, t.cos_d, t.sin_d,
                                        (uint32_t)t.npos, k_cache, v_cache, k_scales, v_scales, v_shadow, o,
                                        (int)num_q_heads, (int)num_kv_heads, (int)head_dim, scale, state,
                                        max_cache, (max_cache + 63) / 64, stream);
}

int cactus_hip_decode_lm_head(const uint16_t* h, const uint16_t* norm_w, float eps,
                              const uint16_t* embedding, size_t K, size_t N, uint32_t* state,
                              uint32_t* tokens_out, size_t max_steps, uint16_t* logits_out,
                              void* scratch, size_t scratch_bytes, void* stream) {
    CH_REQUIRE(h && norm_w && embedding && state && scratch, "decode_lm_head: null pointer");
    CH_REQUIRE(K % 8 == 0 && K <= 4096 && ((uintptr_t)embedding & 15) == 0, "decode_lm_head: bad K");
    const bool streamed = K % LMS_KC == 0;
    const unsigned blocks = streamed ? ceil_div(N, LMS_WAVES * 64) : ceil_div(N, (LM_THREADS / 64) * LM_ROWS_PER_WAVE);
    CH_REQUIRE(scratch_bytes >= 256, "decode_lm_head: scratch too small");
    LmDecArgs p{};
    p.h = h; p.norm_w = norm_w; p.b = embedding; p.eps = eps; p.K = (int)K; p.N = (int)N;
    p.counter = static_cast<uint32_t*>(scratch);
    p.st = state; p.tokens_out = tokens_out; p.max_steps = (uint32_t)max_steps; p.logits_out = logits_out;
    if (streamed) {
        const size_t smem = 4 * K + (size_t)LMS_WAVES * LMS_D * LMS_SLOT;
        // dynamic LDS for the largest K accepted here (4096); the kernel's
        // static reduction arrays take the rest of the CU's 160 KB
        constexpr size_t kMaxSmem = 4 * 4096 + (size_t)LMS_WAVES * LMS_D * LMS_SLOT;
        static const hipError_t attr = hipFuncSetAttribute(
            (const void*)dec_lm_head_stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxSmem);
        if (attr != hipSuccess) {
            (void)hipGetLastError();
            return fail(CACTUS_HIP_ERUNTIME, std::string("decode_lm_head: LDS attribute: ") + hipGetErrorString(attr));
        }
        hipLaunchKernelGGL(dec_lm_head_stream_kernel, dim3(blocks), dim3(LMS_THREADS), smem, as_stream(stream), p);
        return check_launch("decode_lm_head");
    }
    const size_t smem = 4 * K + (size_t)(LM_THREADS / 64) * LM_ROWS_PER_WAVE * LM_ROW_STRIDE;
    hipLaunchKernelGGL(dec_lm_head_kernel, dim3(blocks), dim3(LM_THREADS), smem, as_stream(stream), p);
    return check_launch("decode_lm_head");
}


int cactus_hip_lm_tiles_bytes(size_t K, size_t N, size_t* bytes) {
    CH_REQUIRE(bytes && K % 8 == 0 && K > 0 && K <= 4096 && N > 0 && N < (1u << 30), "lm_tiles_bytes: bad shape");
    *bytes = (N + 63) / 64 * 64 * K * 2;
    return CACTUS_HIP_OK;
}

int cactus_hip_lm_tiles_build(const uint16_t* embedding, size_t K, size_t N, uint16_t* tiles, void* stream) {
    CH_REQUIRE(embedding && tiles, "lm_tiles_build: null pointer");
    CH_REQUIRE(K % 8 == 0 && K > 0 && K <= 4096 && N > 0 && N < (1u << 30), "lm_tiles_build: bad shape");
    CH_REQUIRE(((uintptr_t)embedding | (uintptr_t)tiles) % 16 == 0, "lm_tiles_build: pointers must be 16-byte aligned");
    const size_t total = (N + 63) / 64 * 64 * (K / 8);
    hipLaunchKernelGGL(lm_tiles_build_kernel, dim3((unsigned)ceil_div(total, (size_t)256)), dim3(256), 0,
                       as_stream(stream), embedding, reinterpret_cast<uint4*>(tiles), (int)K, (int)N, total);
    return check_launch("lm_tiles_build");
}

int cactus_hip_decode_lm_head_tiled(const uint16_t* h, const uint16_t* norm_w, float eps, const uint16_t* tiles,
                                    size_t K, size_t N, uint32_t* state, uint32_t* tokens_out, size_t max_steps,
                                    uint16_t* logits_out, void* scratch, size_t scratch_bytes, void* stream) {
    CH_REQUIRE(h && norm_w && tiles && state && scratch, "decode_lm_head_tiled: null pointer");
    CH_REQUIRE(K % 8 == 0 && K > 0 && K <= 4096 && N > 0 && N < (1u << 30), "decode_lm_head_tiled: bad K / N");
    CH_REQUIRE(((uintptr_t)tiles | (uintptr_t)h | (uintptr_t)norm_w) % 16 == 0,
               "decode_lm_head_tiled: tiles, h and norm_w must be 16-byte aligned");
    const unsigned blocks = (unsigned)ceil_div(N, (size_t)LMT_WAVES * 64);
    CH_REQUIRE(scratch_bytes >= LMG_SLOTS + 8 * (size_t)blocks, "decode_lm_head_tiled: scratch too small");
    LmDecArgs p{};
    p.h = h; p.norm_w = norm_w; p.b = tiles; p.eps = eps; p.K = (int)K; p.N = (int)N;
    p.counter = static_cast<uint32_t*>(scratch);
    p.st = state; p.tokens_out = tokens_out; p.max_steps = (uint32_t)max_steps; p.logits_out = logits_out;
    hipLaunchKernelGGL(dec_lm_head_tiled_kernel, dim3(blocks), dim3(LMT_THREADS), 0, as_stream(stream), p);
    return check_launch("decode_lm_head_tiled");
}

int cactus_hip_decode_lm_head_tiled_embed(const uint16_t* h, const uint16_t* norm_w, float eps,
                                          const uint16_t* tiles, const uint16_t* embedding, size_t K, size_t N,
                                          uint32_t* state, uint32_t* tokens_out, size_t max_steps,
                                          uint16_t* logits_out, uint16_t* h_next, void* scratch,
                                          size_t scratch_bytes, void* stream) {
    CH_REQUIRE(h && norm_w && tiles && embedding && h_next && state && scratch,
               "decode_lm_head_tiled_embed: null pointer");
    CH_REQUIRE(K % 8 == 0 && K > 0 && K <= 4096 && N > 0 && N < (1u << 30), "decode_lm_head_tiled_embed: bad K / N");
    CH_REQUIRE(((uintptr_t)tiles | (uintptr_t)h | (uintptr_t)norm_w | (uintptr_t)embedding | (uintptr_t)h_next) % 16 == 0,
               "decode_lm_head_tiled_embed: tiles, h, norm_w, embedding and h_next must be 16-byte aligned");
    const unsigned blocks = (unsigned)ceil_div(N, (size_t)LMT_WAVES * 64);
    CH_REQUIRE(scratch_bytes >= LMG_SLOTS + 8 * (size_t)blocks, "decode_lm_head_tiled_embed: scratch too small");
    LmDecArgs p{};
    p.h = h; p.norm_w = norm_w; p.b = tiles; p.eps = eps; p.K = (int)K; p.N = (int)N;
    p.counter = static_cast<uint32_t*>(scratch);
    p.st = state; p.tokens_out = tokens_out; p.max_steps = (uint32_t)max_steps; p.logits_out = logits_out;
    p.embed = embedding; p.h_next = h_next;
    hipLaunchKernelGGL(dec_lm_head_tiled_kernel, dim3(blocks), dim3(LMT_THREADS), 0, as_stream(stream), p);
    return check_launch("decode_lm_head_tiled_embed");
}

}  // extern "C"
