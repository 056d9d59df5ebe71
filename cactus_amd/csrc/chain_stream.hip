// chain_stream.hip -- the exact decode value chains over the value product
// tiles (a6 value accumulation, kernel_attention.cpp:395-482), in a file of
// its own: it is compiled without machine sinking, which would otherwise
// move the loop-invariant scalar address arithmetic of the hand-placed
// loads into the chain's issue stream.
#include "hip_common.h"
#include "attention_args.h"

namespace cactus_hip {

// ------------------------------------------------ kernel B, decode form
// Decode value chains (one batch, at most two query rows, the INT8 cache
// with its value product tiles).  A workgroup owns one query head and one
// 64-dim slice of one row; wave 0 runs the slice's 64 chains, lane = dim.
// A dependent FMA chain is bound by the chain wave's own instruction issue
// (about one instruction per 4.7 cycles), so every operand reaches the
// chain wave's registers with as few instructions as possible and without
// LDS: a key quad of products by one global_load_dwordx4 per lane from the
// [key / 4][64 dims][4 keys] tiles, the same key quad's weights by one
// global_load_dwordx4 that every lane makes from the same address (a ring
// of CS_R 32-key blocks, CS_R - 1 blocks in flight), and the block's
// rescale factor by one v_readlane.  Wave 1 turns the row's block maxima
// into the rescale factors, the per-block fast-path mask and the running sum
// (the reference's sequential order) while wave 0 chains.  The tiles and
// weights stream from this XCD's L2: kv head h's chain workgroups run on
// XCD h % 8, where the score kernel before this one wrote the head's
// weights and this kernel's prefetch workgroups fetch its product tiles
// ahead of the chains (an L2 hit costs the chain ~7 cycles per key, an
// Infinity Cache hit ~16, HBM ~25).
constexpr int CS_R = 3;          // ring depth in 32-key blocks (CS_R - 1 blocks ahead)
constexpr int CS_P = CS_R;       // blocks per unrolled step: the ring's period
// s_waitcnt immediate (gfx9 encoding): vmcnt VM (6 bits, split), expcnt
// unconstrained, lgkmcnt LGKM
template <int VM, int LGKM>
constexpr int waitcnt_imm() {
    static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "waitcnt range");
    return (VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8);
}
constexpr int CS_THREADS = 128;  // chain wave + block-data wave

// Workgroup -> (row, kv head, head in group, slice): the kv head's
// workgroups sit on XCD kvh % 8 (workgroup i runs on XCD i % 8).
// s_waitcnt vmcnt(N) whose wait the compiler sees as producing the eight
// registers of a ring slot (their loads are then complete: vector memory
// loads return in order, and the N younger loads are the look-ahead blocks')
template <int N, typename V>
__device__ __forceinline__ void wait_vm_tie(V* p) {
    asm volatile("s_waitcnt vmcnt(%8)"
                 : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(p[4]), "+v"(p[5]), "+v"(p[6]), "+v"(p[7])
                 : "n"(N));
}
// the same for two slots' registers at once (one s_waitcnt)
template <int N, typename V>
__device__ __forceinline__ void wait_vm_tie2(V* p, V* w) {
    asm volatile("s_waitcnt vmcnt(%16)"
                 : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(p[4]), "+v"(p[5]), "+v"(p[6]), "+v"(p[7]),
                   "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7])
                 : "n"(N));
}

// inclusive max-scan over the wave's lanes (identity -1): row_shr 1, 2, 4,
// 8 within each 16-lane row, then row_bcast:15 and row_bcast:31 across rows
__device__ __forceinline__ int wave_scan_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x111, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x112, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x114, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x118, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x142, 0xA, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x143, 0xC, 0xF, false));
    return v;
}

struct CsMap {
    int row, kvh, hj, sl;
    bool valid;
};
__device__ __forceinline__ CsMap cs_map(const AttnArgs& a, int nsl) {
    const int L = blockIdx.x;
    int j = L >> 3;
    CsMap m;
    m.sl = j % nsl;
    j /= nsl;
    m.hj = j % a.gq;
    j /= a.gq;
    m.row = j % a.S;
    m.kvh = (L & 7) + 8 * (j / a.S);
    m.valid = m.kvh < a.Hkv;
    return m;
}
__host__ __device__ inline unsigned cs_grid(int S, int Hkv, int gq, int nsl) {
    return 8u * (unsigned)((Hkv + 7) / 8) * (unsigned)S * (unsigned)gq * (unsigned)nsl;
}
// Workgroups after the chain workgroups fetch the cached keys' product
// tiles into the L2 of the chains' XCD, lowest blocks first, while the
// chains start.  The chains' own few CUs cannot do it: each CU's
// outstanding misses cap its fetch rate near 50 GB/s, and the fetch would
// queue ahead of the chains' loads.  CS_PF_WGS per XCD, on CUs beside the
// chains (8 per XCD fetch the 16 MB of a 4096-key layer ~3x faster than
// the chains consume it).
constexpr int CS_PF_WGS = 8;
__device__ void chain_tile_prefetch(const AttnArgs& a, int j, int nj, int nsl) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int x = j & 7;                                     // this workgroup's XCD = kv heads x, x + 8, ...
    const int k = j >> 3, K = nj >> 3;
    const int nkx = x < a.Hkv ? (a.Hkv - x + 7) / 8 : 0;
    const int per = nkx * nsl;                               // tile slices of this XCD
    const int nbc = (int)((a.cache_len + ATT_BLOCK - 1) / ATT_BLOCK);
    const int total = nbc * per;
    const unsigned off = (unsigned)lane * 128u;             // one dword per 128-byte line
    int sink = 0;
    // lowest blocks first; one 8 KB block slice per wave load, at most 32
    // in flight; the register stays live until the last has landed
    for (int it = __builtin_amdgcn_readfirstlane(2 * k + wv); it < total; it += 2 * K) {
        const int b = it / per, r = it % per;
        const char* p = reinterpret_cast<const char*>(
            a.vsh + sh_index(x + 8 * (r / nsl), nsl, r % nsl, a.sh_ntile, (size_t)b * ATT_BLOCK, 0));
        asm volatile("s_waitcnt vmcnt(31)\n\tglobal_load_dword %0, %1, %2" : "+v"(sink) : "v"(off), "s"(p));
    }
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(sink));
}

// wts: the weights a_in.w (rows of wstride floats, padded by one block)
__global__ void __launch_bounds__(CS_THREADS) attn_chain_stream_kernel(AttnArgs a_in, int nbmax,
                                                                      const float* __restrict__ wts) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const AttnArgs a = resolve(a_in);
    extern __shared__ __align__(16) unsigned char smem[];
    const int nch = (nbmax + 63) / 64;
    float* corr_s = reinterpret_cast<float*>(smem);                                   // [nch * 64]
    float* bsum_s = corr_s + (size_t)nch * 64;                                        // [nch * 64]
    uint64_t* fast_s = reinterpret_cast<uint64_t*>(bsum_s + (size_t)nch * 64);        // [nch]
    float* rs_s = reinterpret_cast<float*>(fast_s + nch);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int d = a.d, da = (d / 8) * 8, nsl = (d + 63) / 64;
    const unsigned nchain = cs_grid(a.S, a.Hkv, a.gq, nsl);
    if (blockIdx.x >= nchain) {                              // whole workgroup, before any barrier
        chain_tile_prefetch(a, (int)(blockIdx.x - nchain), (int)(gridDim.x - nchain), nsl);
        return;
    }
    const CsMap m = cs_map(a, nsl);
    if (!m.valid) return;                                    // whole workgroup, before any barrier
    const int qp = m.row;
    const size_t row = (size_t)qp * a.Hq + (size_t)m.kvh * a.gq + m.hj;
    const int dim = m.sl * 64 + lane;
    const float NEG_INF = -__builtin_inff();

    size_t rks, rke, rbl;
    kv_range<true>(a, (size_t)qp, rks, rke, rbl);           // hybrid: rks = 0, rbl = rke
    const int nb = rke > 0 ? (int)((rke + ATT_BLOCK - 1) / ATT_BLOCK) : 0;
    const size_t kfull = rke < a.cache_len ? rke : a.cache_len;   // keys of full cached blocks

    if (wv == 1) {
        // ---- block data: rescale factors (the running max is the last
        // finite block max; a block without one keeps the factor 1, which
        // leaves every value unchanged) and the fast-path mask; then the
        // running sum.  Barrier 1: chunk 0 ready; barrier 2: every chunk;
        // barrier 3: the running sum.
        const float* bm = a.bmax + row * a.nbstride;
        const float* bsm = a.bsum + row * a.nbstride;
        float carry = NEG_INF;
        const int nchu = (nb + 63) / 64;                    // chunks the chains use
        for (int c = 0; c < nchu; c++) {
            const int i = c * 64 + lane;
            const float mx = i < nb ? bm[i] : NEG_INF;
            const float bs = i < nb ? bsm[i] : 0.0f;
            const bool fin = mx > NEG_INF;
            const int idx = wave_scan_max(fin ? lane : -1);        // last finite block at or before this one
            const int ex = __builtin_amdgcn_update_dpp(-1, idx, 0x138, 0xF, 0xF, false);   // wave_shr:1
            const float pm = __shfl(mx, ex < 0 ? 0 : ex, 64);
            const float prev = ex >= 0 ? pm : carry;
            const float corr = fin ? cactus_expf(prev - mx) : 1.0f;
            const int last = __builtin_amdgcn_readlane(idx, 63);
            if (last >= 0) carry = lane_f(mx, last);
            const bool full = (size_t)(i + 1) * ATT_BLOCK <= kfull;
            const bool fast = i < nb && full && fin && !__builtin_signbit(bs);
            const uint64_t fastm = __ballot(fast);
            corr_s[i] = corr;
            bsum_s[i] = __builtin_fabsf(bs);
            if (lane == 0) fast_s[c] = fastm;
            if (c == 0) __syncthreads();                     // barrier 1
        }
        if (nchu == 0) __syncthreads();
        __syncthreads();                                     // barrier 2
        // running sum in the reference's order, one block at a time:
        // rs = rs * corr, then rs = rs + block sum (two roundings)
        float rs = 0.0f;
        for (int c = 0; c < nchu; c++) {
            const float cj = corr_s[c * 64 + lane], bj = bsum_s[c * 64 + lane];
            const int nin = min(64, nb - c * 64);
            int j = 0;
            for (; j + 4 <= nin; j += 4) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    rs = rs * lane_f(cj, j + u);
                    rs = rs + lane_f(bj, j + u);
                }
            }
            for (; j < nin; j++) {
                rs = rs * lane_f(cj, j);
                rs = rs + lane_f(bj, j);
            }
        }
        if (lane == 0) *rs_s = rs;
        __syncthreads();                                     // barrier 3
        return;
    }

    // ---- chain wave
    constexpr int BLK_BYTES = ATT_BLOCK * 64 * 4;           // a block's products in one slice
    const char* pbase = reinterpret_cast<const char*>(a.vsh + sh_index(m.kvh, nsl, m.sl, a.sh_ntile, 0, 0));
    const char* wbase = reinterpret_cast<const char*>(wts + row * a.wstride);
    unsigned voff[8];
#pragma unroll
    for (int q = 0; q < 8; q++) voff[q] = lane * 16 + q * 1024;
    const unsigned vzero = 0u;
    f4v pr[CS_R][8];     // products: lane = dim, 4 consecutive keys per register quad
    f4v wr[CS_R][8];     // weights: the same 4 keys' weights in every lane
    // Hand-placed loads (global_load with a scalar base and a lane offset):
    // the compiler neither waits for them early nor counts them;
    // wait_vm_tie waits for a slot before its use, and every slot is waited
    // for before the loop ends.  Block indices are clamped to the row's last
    // block, and a weight row has room for one block past its last (the
    // weight stride is padded by 64).
    auto issue_p = [&](f4v* dst, int blk) {
        const char* b = pbase + (size_t)blk * BLK_BYTES;
#pragma unroll
        for (int q = 0; q < 8; q++)
            asm volatile("global_load_dwordx4 %0, %1, %2" : "=&v"(dst[q]) : "v"(voff[q]), "s"(b));
    };
    auto issue_w = [&](f4v* dst, int blk) {
        const char* b = wbase + (size_t)blk * ATT_BLOCK * 4;
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:0" : "=&v"(dst[0]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:16" : "=&v"(dst[1]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:32" : "=&v"(dst[2]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:48" : "=&v"(dst[3]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:64" : "=&v"(dst[4]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:80" : "=&v"(dst[5]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:96" : "=&v"(dst[6]) : "v"(vzero), "s"(b));
        asm volatile("global_load_dwordx4 %0, %1, %2 offset:112" : "=&v"(dst[7]) : "v"(vzero), "s"(b));
    };
    // the step's new rows (fp16 values past the cache), loaded and waited
    // for before any hand-placed load is issued
    float pnew[2] = {0.0f, 0.0f};
    const int dimc = dim < d ? dim : d - 1;
    for (int t = 0; t < 2 && (size_t)t < a.new_len; t++)
        pnew[t] = h2f(a.v[((size_t)t * a.Hkv + m.kvh) * (size_t)d + dimc]);
    asm volatile("" ::"v"(pnew[0]), "v"(pnew[1]));
    const int nbl = nb > 0 ? nb - 1 : 0;
    // ring slot of a block: its weights, then its products; CS_R - 1 blocks
    // in flight ahead of the one being chained
    auto issue = [&](int slot, int blk) {
        issue_w(wr[slot], blk);
        issue_p(pr[slot], blk);
    };
    if (nb > 0) {
#pragma unroll
        for (int r = 0; r < CS_R - 1; r++) issue(r, min(r, nbl));
    }
    __syncthreads();                                         // barrier 1
    float acc = 0.0f;
    float cv = 0.0f;
    uint64_t fastm = 0;
    const uint32_t clen = (uint32_t)a.cache_len, kend = (uint32_t)rke;

    // block at ring position r: wait for its slot (all but the 16 loads of
    // the CS_R - 2 = 1 younger block), then fill the slot freed a block ago
    // with the block CS_R - 1 ahead (its index clamped to the last block)
    auto step_in = [&](int r, int blk_ahead) {
        static_assert(CS_R == 3, "wait count below assumes one younger block");
        wait_vm_tie2<16>(pr[r % CS_R], wr[r % CS_R]);
        __builtin_amdgcn_sched_barrier(0);
        issue((r + CS_R - 1) % CS_R, blk_ahead);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto corr_of = [&](int bl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cv), bl));
    };
    // block at ring position r: the common case -- a full cached block with
    // a finite max and no zero weight -- is 32 plain FMAs, computed for every
    // block; any other block (zero weights skipped, kernel_attention.cpp:
    // 200-201, since an FMA with one could turn an accumulator of -0 into
    // +0; keys past the cache from the new rows; keys past the row's end
    // skipped) then recomputes its result from the block's starting value
    // with selects, out of the straight-line path
    auto chain_block = [&](int r, int blk, bool fast) {
        const int bl = blk & 63;
        const float cb = corr_of(bl);
        const float a0 = acc;
        float af = a0 * cb;
#pragma unroll
        for (int q = 0; q < 8; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) af = __builtin_fmaf(pr[r % CS_R][q][e], wr[r % CS_R][q][e], af);
        acc = af;
        if (__builtin_expect(!fast, 0)) {
            float as = a0 * cb;
            const uint32_t bs0 = (uint32_t)blk * ATT_BLOCK;
            const uint32_t ncache = clen > bs0 ? clen - bs0 : 0u;     // keys of the block in the cache
            const uint32_t nlive = kend > bs0 ? kend - bs0 : 0u;      // keys of the block in the row
#pragma unroll
            for (int k = 0; k < ATT_BLOCK; k++) {
                const float pv = (uint32_t)k < ncache ? pr[r % CS_R][k / 4][k % 4] : pnew[(k - (int)ncache) & 1];
                const float w = (uint32_t)k < nlive ? wr[r % CS_R][k / 4][k % 4] : 0.0f;
                const float f = __builtin_fmaf(pv, w, as);
                as = w != 0.0f ? f : as;
            }
            acc = as;
        }
    };

    // block data of the 64-block chunk c (its rescale factors in cv, one
    // per lane; its fast-path mask); wave 1 has written chunk 0 by barrier 1 and
    // the others by barrier 2
    auto load_chunk = [&](int c) {
        if (c == 1) __syncthreads();                         // barrier 2
        cv = corr_s[c * 64 + lane];
        const uint64_t fw = fast_s[c];
        __builtin_amdgcn_s_waitcnt(waitcnt_imm<63, 0>());   // the chunk's block data is in registers
        fastm = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(fw >> 32)) << 32) |
                (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)fw);
    };
    const int nchu = (nb + 63) / 64;
    if (nb > 0) load_chunk(0);
    // CS_P consecutive blocks per step, block g + r in ring slot r: g steps
    // over the whole row by the ring's period, so the slot of every block is
    // its index mod CS_R.  A step inside one chunk whose look-ahead blocks
    // all lie inside the row needs no clamp and no chunk change; a step at a
    // chunk edge (64 is no multiple of CS_P) or at the row's end takes the
    // checked form.
    int g = 0;
    while (g < nb) {
        // the run of plain steps from g: inside g's chunk, look-ahead inside
        // the row, and not at a chunk's first block (whose data is loaded
        // by the checked form)
        int lim = min(((g >> 6) + 1) * 64 - CS_P, nbl - (CS_P + CS_R - 2));
        if (g > 0 && (g & 63) == 0) lim = -1;
        for (; g <= lim; g += CS_P) {
            const uint32_t gm = (uint32_t)(fastm >> (g & 63));
#pragma unroll
            for (int r = 0; r < CS_P; r++) {
                step_in(r, g + r + CS_R - 1);
                chain_block(r, g + r, (gm >> r) & 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (g >= nb) break;
        // one checked step
#pragma unroll
        for (int r = 0; r < CS_P; r++) {
            const int blk = g + r;
            if (blk >= nb) break;
            if (blk > 0 && (blk & 63) == 0) load_chunk(blk >> 6);
            step_in(r, min(blk + CS_R - 1, nbl));
            chain_block(r, blk, (fastm >> (blk & 63)) & 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        g += CS_P;
    }
    // the look-ahead loads still in flight land before their registers can
    // be reused
#pragma unroll
    for (int r = 0; r < CS_R; r++) {
        wait_vm_tie<0>(pr[r]);
        wait_vm_tie<0>(wr[r]);
    }
    if (nchu < 2) __syncthreads();                           // barrier 2 (rows of one chunk)
    __syncthreads();                                         // barrier 3
    const float rs = *rs_s;
    if (dim < d) {
        uint16_t* ov = a.o + row * (size_t)d;
        if (!(rs > 0.0f) || dim >= da) ov[dim] = 0;
        else ov[dim] = f2h(acc * (1.0f / rs));
    }
}

int launch_chain_stream(const AttnArgs& a, int nbmax, void* stream) {
    CH_REQUIRE(a.B == 1 && a.S <= 2 && a.new_len <= 2 && a.d <= 256 && nbmax <= 1024,
               "attention: value product tiles serve one batch, at most two query rows and head_dim <= 256");
    const int nsl = (a.d + 63) / 64;
    const int nch = (nbmax + 63) / 64;
    const size_t smem = 2 * (size_t)nch * 64 * sizeof(float) + (size_t)nch * sizeof(uint64_t) + 16;
    const unsigned npf = a.cache_len > 0 ? 8u * CS_PF_WGS : 0u;
    hipLaunchKernelGGL(attn_chain_stream_kernel, dim3(cs_grid(a.S, a.Hkv, a.gq, nsl) + npf), dim3(CS_THREADS), smem,
                       as_stream(stream), a, nbmax, (const float*)a.w);
    return check_launch("attention values (decode)");
}

}  // namespace cactus_hip
