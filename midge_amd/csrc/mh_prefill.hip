// mh_prefill.hip — expert-major prefill of one MoE layer with CDNA4 scaled
// MFMA: forward_batch()'s route + expert-major block (engine/midge.c:591-611)
// with expert_apply (engine/midge.c:437-467) as one grouped GEMM per routed
// expert over the tokens routed to it.
//
//   lists      assignments (token t, slot i) grouped by expert: counts,
//              offsets, token of each list position, slot of each position
//   quantize   xb (per token) -> kTerms planes of fp6 e2m3 with an e8m0
//              scale per 32-element block: x = sum_t q_t * 2^e_t, each term
//              the rounding residual of the previous one (each shrinks the
//              block's largest residual by >= 2^-4). fp4 x fp6 runs the
//              instruction at twice the rate of fp4 x fp8 (measured 8.1
//              against 4.3 PFLOP/s), and an e2m3 term reduces a block's
//              residual as much as an e4m3 one.
//   gate/up    per (expert, 32-row tile): A = the fp4 gate and up rows
//              verbatim (e2m1 nibbles) with e8m0 scales taken exactly from
//              the f16 powers of two; B = the quantized tokens of the
//              expert; V_MFMA_SCALE_F32_32X32X64_F8F6F4 accumulates all
//              terms in f32; epilogue bias + clamped SwiGLU -> h
//   quantize   h -> kTerms planes, as for x
//   down       per (expert, 32-row tile) over h; epilogue + bias -> y of the
//              assignment's slot; the existing prefill combine then adds
//              w * y to each token in ascending expert order.
//
// Operand layout of the 32x32x64 instruction with fp4 A and fp6 B
// (measured on gfx950 with one-hot operands): lane l holds A row l % 32 and
// B column l % 32; with g = l / 32, A's 16 bytes (32 e2m1 values) and B's 24
// bytes (32 e2m3 values, 6 bits each from the lowest bit up) are columns
// 32 g .. 32 g + 31 of the step, in order, and each lane's scale covers its
// own 32 columns. So for K step s (weight columns 64s .. 64s+63) A lane
// (m, g) loads 16-byte chunk 2s+g of row m (one MXFP4 block and its scale)
// and B lane (n, g) block 2s+g of token n with its scale: activations are
// quantized in natural 32-column blocks, like the weights. Output lane l:
// column l % 32, rows 8(i/4) + 4g + i%4 for accumulator i.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "mh_internal.h"

namespace mh {

namespace {

constexpr int kTerms = 3;      // fp6 terms per activation
constexpr int kNT = 4;         // 32-token tiles per pass (weights loaded once per pass)
constexpr int kWaves = 4;      // 32-row tiles per block (one per wave)

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v6i __attribute__((ext_vector_type(6)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

// ---------------------------------------------------------------- lists

// The lists in one block (E <= kPlistMaxE): ranks by LDS atomics, an
// exclusive scan of the counts, then the scatter. Positions within an
// expert's list follow the atomics' order; every output is per assignment,
// so the order does not change any result.
constexpr int kPlistMaxE = 4096;
__global__ void __launch_bounds__(1024)
k_plist_one(const int32_t *sel, int N, int E, int k, int *rank, int *offs, int *list_tok, int *slot_of) {
    __shared__ int cnt[kPlistMaxE];
    __shared__ int wsum[16];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    for (int i = t; i < E; i += 1024) cnt[i] = 0;
    __syncthreads();
    for (int a = t; a < N; a += 1024) {
        const int e = sel[a];
        rank[a] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
    }
    __syncthreads();
    // thread t owns counters [t * ch, t * ch + ch): local sum, block scan
    const int ch = (E + 1023) / 1024;
    int own = 0;
    for (int i = 0; i < ch; ++i) {
        const int e = t * ch + i;
        if (e < E) own += cnt[e];
    }
    int v = own;
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    if (lane == 63) wsum[wv] = v;
    __syncthreads();
    int run = v - own, total = 0;
    for (int i = 0; i < 16; ++i) {
        if (i < wv) run += wsum[i];
        total += wsum[i];
    }
    for (int i = 0; i < ch; ++i) {
        const int e = t * ch + i;
        if (e < E) {
            const int c = cnt[e];
            cnt[e] = run;
            offs[e] = run;
            run += c;
        }
    }
    if (t == 0) offs[E] = total;
    __syncthreads();
    for (int a = t; a < N; a += 1024) {
        const int r = rank[a];
        if (r >= 0) {
            const int p = cnt[sel[a]] + r;
            list_tok[p] = a / k;
            slot_of[p] = a;
        }
    }
}


// ---------------------------------------------------------------- quantize

// e such that m * 2^-e <= 7.5 (the largest e2m3 value), as small as possible.
__device__ __forceinline__ int fp6_block_exp(float m) {
    int km;
    const float fm = frexpf(m, &km);   // m = fm * 2^km, fm in [0.5, 1)
    return fm <= 0.9375f ? km - 3 : km - 2;
}

// Rows of K f32 (row r of the input = in[(map ? map[r] : r) * K ...]) ->
// kTerms planes q[t][r][K] and sc[t][r][scs] (e8m0, scs >= K / 32: rows
// padded to 16 bytes), one scale 2^e per 32-column block b (thread = (row,
// block)). Block b of a plane is 32 bytes at 32 b: its 32 e2m3 codes, 6 bits
// each from the lowest bit up in column order (24 bytes), then 8 zero bytes.
// Each term is the previous residual divided by 2^e and rounded by the
// hardware converter, which interleaves its two 16-value inputs (even
// columns, odd columns); its values come back exactly from the inverse
// converter, so the residuals are exact. A zero block keeps e = 0.
__global__ void __launch_bounds__(256)
k_quant_terms(const float *__restrict__ in, const int *__restrict__ map, int rows, int K,
              uint8_t *__restrict__ q, uint8_t *__restrict__ sc, int scs) {
    const int nb = K / 32;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (int64_t)rows * nb) return;
    const int r = (int)(id / nb), b = (int)(id - (int64_t)r * nb);
    const int src = map ? map[r] : r;
    const float *p0 = in + (int64_t)src * K + 32 * b;
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 a = ((const float4 *)p0)[j];
        v[4 * j + 0] = a.x; v[4 * j + 1] = a.y; v[4 * j + 2] = a.z; v[4 * j + 3] = a.w;
    }
    for (int t = 0; t < kTerms; ++t) {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) m = fmaxf(m, fabsf(v[j]));
        const int e = m > 0.f ? max(-126, min(127, fp6_block_exp(m))) : 0;
        const float scl = ldexpf(1.0f, e);
        v16f ev, od;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            ev[j] = v[2 * j];
            od[j] = v[2 * j + 1];
        }
        const v6i w = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(ev, od, scl);
        const v32f back = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(w, scl);
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] -= back[j];
        uint8_t *qr = q + ((int64_t)t * rows + r) * K + 32 * b;
        *(uint4 *)qr = make_uint4((uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]);
        *(uint4 *)(qr + 16) = make_uint4((uint32_t)w[4], (uint32_t)w[5], 0u, 0u);
        sc[((int64_t)t * rows + r) * scs + b] = (uint8_t)(e + 127);
    }
}

// ---------------------------------------------------------------- GEMM

struct GemmArgs {
    const uint8_t *experts;
    uint64_t stride;
    uint64_t off[9];
    int E, H, F;
    float alpha, limit;
    int act_plain;
    const int *offs;       // [E + 1]
    const int *list_tok;   // [N]
    const int *slot_of;    // [N]
    const uint8_t *bq;     // [kTerms][b_rows][K]
    const uint8_t *bs;     // [kTerms][b_rows][K / 32]
    int b_rows;
    float *hbuf;           // [N][F]  (gate/up output, list order)
    float *ye;             // [n * k][H] (down output, slot order)
    unsigned *err;         // set if a weight scale is not a power of two
};

// f16 power of two -> e8m0 (exact); flags anything else.
__device__ __forceinline__ int e8m0_of_f16(uint32_t h, unsigned *bad) {
    const uint32_t f = __float_as_uint(mh_f16((uint16_t)h));
    if (f & 0x807FFFFFu) *bad = 1u;   // sign or mantissa bits: not a positive power of two
    return (int)((f >> 23) & 0xFFu);  // a zero scale (an e8m0 below f16's range) becomes 2^-127
}

// LDS of the GEMM block, for K columns and nmat weight matrices:
//   bbuf   two buffers of one K step's B operands for every (term, token
//          tile, half, lane) as 16-byte pieces
//   tiles  one 32 x 33 f32 transpose tile per wave
//   asc    the f16 scales of each wave's 32 weight rows, all of K (loaded
//          once per block: [wave][matrix][row][K / 32])
//   bsc    the e8m0 scales of the pass's tokens, all of K ([term][token]
//          rows of bss bytes: 8-aligned, +8 so that 32 lanes reading one
//          column fall in distinct banks)
constexpr int kBPieces = kTerms * kNT * 2 * 64;              // 16-byte pieces per K step
static_assert(kTerms * 128 == 64 * kWaves + 128, "a tile's B pieces: one per thread, two in waves 0-1");
constexpr size_t kLdsMax = 160 * 1024;                       // LDS per workgroup on gfx950

// e8m0 scale row stride of the quantized activations in memory (16-byte rows)
__host__ __device__ inline int bscale_stride(int K) { return ((K / 32) + 15) & ~15; }

struct GemmLds {
    size_t tiles, asc, bsc, total;
    int bss;
};
__host__ __device__ inline GemmLds gemm_lds(int K, int nmat) {
    const int nsc = K / 32;
    GemmLds L;
    L.bss = ((nsc + 7) & ~7) + 8;
    L.tiles = 2 * (size_t)kBPieces * 16;
    L.asc = L.tiles + sizeof(float) * kWaves * 32 * 33;
    L.bsc = L.asc + (size_t)kWaves * nmat * 32 * nsc * 2;
    L.total = L.bsc + (size_t)kTerms * kNT * 32 * L.bss;
    return L;
}

// MODE 0: gate/up (K = H, rows = F, B rows = tokens through list_tok);
// MODE 1: down (K = F, rows = H, B rows = list positions).
// Block = (expert, 4 row tiles of 32), one wave per row tile; the expert's
// tokens in passes of up to kNT 32-token tiles. Per K step the block stages
// B (all terms and tiles) in LDS, double-buffered: step s+1 is loaded from
// memory while step s's MFMAs run; each wave keeps its A (weight) chunks two
// steps ahead in registers.
template <int MODE>
__global__ void __launch_bounds__(64 * kWaves) k_moe_gemm(GemmArgs A) {
    constexpr int NM = MODE == 0 ? 2 : 1;   // weight matrices: gate and up, or down
    extern __shared__ __attribute__((aligned(16))) uint8_t glds[];
    const int K = MODE == 0 ? A.H : A.F;
    const GemmLds LL = gemm_lds(K, NM);
    mh_u4 *bbuf = (mh_u4 *)glds;                                    // [2][kBPieces]
    float(*tiles)[32][33] = (float(*)[32][33])(glds + LL.tiles);
    uint16_t *asc = (uint16_t *)(glds + LL.asc);
    uint8_t *bsc = glds + LL.bsc;
    const int bss = LL.bss, scs = bscale_stride(K);
    const int R = MODE == 0 ? A.F : A.H;
    const int RT = R / 32;
    const int groups = (RT + kWaves - 1) / kWaves;
    // XCD-aware order: the dispatcher deals blocks to the 8 XCDs round
    // robin (block b to XCD b % 8), so logical block lin = (b % 8) * (nb / 8)
    // + b / 8 puts an expert's row groups on one XCD, where its tokens' B
    // operands stay in that XCD's L2 (the grid is a multiple of 8)
    const int lin = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);
    if (lin >= A.E * groups) return;   // block-uniform: padding to a multiple of 8
    const int e = lin / groups, rgrp = lin - e * groups;
    const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
    const int rt = rgrp * kWaves + wave;
    const bool wact = rt < RT;                 // inactive waves still stage B
    const int base = A.offs[e], T = A.offs[e + 1] - base;
    if (T == 0) return;                        // block-uniform
    const int m = l & 31, g = l >> 5;
    const int row = (wact ? rt : 0) * 32 + m;
    const uint8_t *ex = A.experts + (uint64_t)e * A.stride;
    const int rowbytes = K / 2, nsc = K / 32, steps = K / 64;
    const uint8_t *a0 = ex + A.off[MODE == 0 ? 0 : 6] + (size_t)row * rowbytes;
    const uint8_t *a1 = ex + A.off[3] + (size_t)row * rowbytes;
    unsigned bad = 0;
    float(*tl)[33] = tiles[wave];
    // the wave's weight scales, all of K, as contiguous dwords (the 32 rows'
    // scales are one run: 32 * nsc u16, nsc even); read by this wave only
    // (loads in batches of 16 per lane, then the stores: one memory latency
    // per batch instead of one per dword)
    uint16_t *wsc = asc + (size_t)wave * NM * 32 * nsc;
    if (wact) {
        const int nd = 16 * nsc;   // dwords per matrix
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
            const uint32_t *src = (const uint32_t *)((const uint16_t *)(ex + A.off[MODE == 0 ? 1 + 3 * mt : 7]) +
                                                     (size_t)rt * 32 * nsc);
            uint32_t *dst = (uint32_t *)(wsc + (size_t)mt * 32 * nsc);
            for (int k0 = 0; k0 < nd; k0 += 64 * 16) {
                uint32_t v[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) v[u] = src[min(k0 + 64 * u + l, nd - 1)];
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    if (k0 + 64 * u + l < nd) dst[k0 + 64 * u + l] = v[u];
            }
        }
    }
    for (int p0 = 0; p0 < T; p0 += 32 * kNT) {
        const int nt = min(kNT, (T - p0 + 31) / 32);
        // B pieces of tile j: 384 (term t, token n, quarter c), c fastest,
        // so one load instruction reads 64 contiguous bytes (a K step) of
        // each of 16 tokens. Thread tid loads piece tid (t = tid / 128) and,
        // in waves 0-1, piece tid + 256 (t = 2), both of token n = (tid / 4)
        // % 32 and quarter c = tid % 4; the store puts quarter c = 2 g + half
        // (block 2s + g, its bytes 16 half .. 16 half + 15) into the operand
        // slot (t, j, half) lane 32 g + n. Only the pass's
        // nt tiles are loaded; list positions past T read position T - 1
        // (their columns are not stored).
        const int bc = tid & 3, bn = (tid >> 2) & 31, bt = tid >> 7;
        const bool two = tid < 128;   // wave-uniform
        const size_t tstride = (size_t)A.b_rows * K;
        const uint8_t *bsrc[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int p = min(p0 + 32 * min(j, nt - 1) + bn, T - 1);
            const int br = MODE == 0 ? A.list_tok[base + p] : base + p;
            bsrc[j] = A.bq + (size_t)br * K + 16 * bc;
        }
        auto bdst = [&](int t, int j) { return ((t * kNT + j) * 2 + (bc & 1)) * 64 + 32 * (bc >> 1) + bn; };
        // the pass's activation scales, all of K: rows (term, token) of scs
        // bytes in memory (16-byte pieces) into LDS rows of bss bytes; the
        // previous pass ended with a barrier, so bsc is free
        {
            const int pr = scs / 16, total = kTerms * kNT * 32 * pr;
            constexpr int kB = 9;   // 16-byte pieces per thread per batch
            for (int q0 = 0; q0 < total; q0 += 64 * kWaves * kB) {
                mh_u4 v[kB];
#pragma unroll
                for (int u = 0; u < kB; ++u) {
                    const int q = min(q0 + 64 * kWaves * u + tid, total - 1);
                    const int ri = q / pr, pc = q - ri * pr;
                    const int t = ri / (kNT * 32), tok = ri - t * (kNT * 32);
                    const int p = min(p0 + tok, T - 1);
                    const int br = MODE == 0 ? A.list_tok[base + p] : base + p;
                    v[u] = mh_load16_cached(mh_global(A.bs + ((size_t)t * A.b_rows + br) * scs + 16 * pc));
                }
#pragma unroll
                for (int u = 0; u < kB; ++u) {
                    const int q = q0 + 64 * kWaves * u + tid;
                    if (q < total) {
                        const int ri = q / pr, pc = q - ri * pr;
                        uint2 *d = (uint2 *)(bsc + (size_t)ri * bss + 16 * pc);
                        d[0] = make_uint2(v[u].x, v[u].y);
                        d[1] = make_uint2(v[u].z, v[u].w);
                    }
                }
            }
        }
        v16f acc0[kNT], acc1[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            acc0[j] = v16f{};
            acc1[j] = v16f{};
        }
        // Register sets are indexed at compile time (a runtime index turns
        // every load into a wait and an indexed move): A (weights) in three
        // sets and B in two, both loaded two steps ahead, B then staged into
        // two LDS buffers. Steps run in groups of 6 = lcm(3, 2).
        // (loads through the caches: a weight load takes 32 bytes of each
        // of 32 rows, so four K steps share every 128-byte line, and a B
        // load 64 bytes of each token; non-temporal lines were fetched again
        // by the later instructions: 259 -> 221 us gate/up, 164 -> 150 us
        // down at 512 tokens of gpt-oss-20b)
        mh_u4 wa0[3], wa1[3];
        mh_u4 rb[2][2 * kNT];
        auto load_a = [&](int set, int st) {
            const int c = 2 * min(st, steps - 1) + g;
            wa0[set] = mh_load16_cached(mh_global(a0 + c * 16));
            if constexpr (MODE == 0) wa1[set] = mh_load16_cached(mh_global(a1 + c * 16));
        };
        auto load_b = [&](auto ntc, int set, int st) {
            constexpr int NTT = decltype(ntc)::value;
            const int sc = min(st, steps - 1);
#pragma unroll
            for (int j = 0; j < NTT; ++j) {
                rb[set][2 * j] = mh_load16_cached(mh_global(bsrc[j] + (size_t)bt * tstride + 64 * sc));
                if (two) rb[set][2 * j + 1] = mh_load16_cached(mh_global(bsrc[j] + 2 * tstride + 64 * sc));
            }
        };
        auto store_b = [&](auto ntc, int set, int buf) {
            constexpr int NTT = decltype(ntc)::value;
            mh_u4 *nb = bbuf + (size_t)buf * kBPieces;
#pragma unroll
            for (int j = 0; j < NTT; ++j) {
                nb[bdst(bt, j)] = rb[set][2 * j];
                if (two) nb[bdst(2, j)] = rb[set][2 * j + 1];
            }
        };
        // the MFMAs of step st over NTT token tiles (NTT = nt as a compile-time
        // instantiation: no per-tile guards), reading tile j + 1's B operands
        // from LDS while tile j's MFMAs run
        auto math = [&](auto ntc, int u, int buf, int st) {
            constexpr int NTT = decltype(ntc)::value;
            const int blk = 2 * st + g;   // this lane's scale block
            v8i qa0 = {}, qa1 = {};
            qa0[0] = (int)wa0[u].x; qa0[1] = (int)wa0[u].y; qa0[2] = (int)wa0[u].z; qa0[3] = (int)wa0[u].w;
            const int sa0 = e8m0_of_f16(wsc[(size_t)m * nsc + blk], &bad);
            int sa1 = 127;
            if constexpr (MODE == 0) {
                qa1[0] = (int)wa1[u].x; qa1[1] = (int)wa1[u].y; qa1[2] = (int)wa1[u].z; qa1[3] = (int)wa1[u].w;
                sa1 = e8m0_of_f16(wsc[(size_t)(32 + m) * nsc + blk], &bad);
            }
            const mh_u4 *bb = bbuf + (size_t)buf * kBPieces;
            v8i qb[2][kTerms];
            int sbv[2][kTerms];
            auto rd = [&](int j, int slot) {
#pragma unroll
                for (int t = 0; t < kTerms; ++t) {
                    const mh_u4 lo = bb[((t * kNT + j) * 2 + 0) * 64 + l];
                    const uint2 hi = *(const uint2 *)&bb[((t * kNT + j) * 2 + 1) * 64 + l];   // bytes 16-23 (fp6: 24 bytes)
                    qb[slot][t] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, 0, 0};
                    sbv[slot][t] = bsc[(size_t)((t * kNT + j) * 32 + m) * bss + blk];
                }
            };
            rd(0, 0);
#pragma unroll
            for (int j = 0; j < NTT; ++j) {
                if (j + 1 < NTT) rd(j + 1, (j + 1) & 1);
#pragma unroll
                for (int t = 0; t < kTerms; ++t) {
                    acc0[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa0, qb[j & 1][t], acc0[j], 4, 2, 0, sa0,
                                                                             0, sbv[j & 1][t]);
                    if constexpr (MODE == 0)
                        acc1[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa1, qb[j & 1][t], acc1[j], 4, 2, 0,
                                                                                 sa1, 0, sbv[j & 1][t]);
                }
            }
            // pin that order for the scheduler (left alone, it reuses one
            // operand set and waits for every read): the weight scales and
            // tile 0's reads, then per tile the next tile's reads (9 DS
            // reads) ahead of this tile's MFMAs
            constexpr int kDsRead = 0x100, kMfma = 0x008, kPerTile = kTerms * NM;
            __builtin_amdgcn_sched_group_barrier(kDsRead, 3 * kTerms + NM, 0);
#pragma unroll
            for (int j = 0; j + 1 < NTT; ++j) {
                __builtin_amdgcn_sched_group_barrier(kDsRead, 3 * kTerms, 0);
                __builtin_amdgcn_sched_group_barrier(kMfma, kPerTile, 0);
            }
            __builtin_amdgcn_sched_group_barrier(kMfma, kPerTile, 0);
        };
        // step st at position j of its group: B and A of st + 2 issued, the
        // MFMAs of st, then B of st + 1 (loaded a step ago) into the other
        // LDS buffer: each load has two steps of MFMAs to arrive
        auto run_steps = [&](auto ntc) {
            load_b(ntc, 0, 0);
            store_b(ntc, 0, 0);
            load_b(ntc, 1, 1);
            load_a(0, 0);
            load_a(1, 1);
            __syncthreads();
            auto step = [&](int j, int st) {
                load_b(ntc, j % 2, st + 2);
                load_a((j + 2) % 3, st + 2);
                __builtin_amdgcn_sched_barrier(0);
                if (wact) math(ntc, j % 3, j % 2, st);
                store_b(ntc, (j + 1) % 2, (j + 1) % 2);
                __syncthreads();
            };
            int st = 0;
            for (; st + 6 <= steps; st += 6) {
#pragma unroll
                for (int j = 0; j < 6; ++j) step(j, st + j);
            }
#pragma unroll
            for (int j = 0; j < 5; ++j)
                if (st + j < steps) step(j, st + j);
        };
        static_assert(kNT == 4, "one instantiation per tile count");
        switch (nt) {   // block-uniform
        case 1: run_steps(std::integral_constant<int, 1>{}); break;
        case 2: run_steps(std::integral_constant<int, 2>{}); break;
        case 3: run_steps(std::integral_constant<int, 3>{}); break;
        default: run_steps(std::integral_constant<int, 4>{}); break;
        }
        if (wact) {
            // epilogue through the wave's LDS tile: lane (m, g) owns column m
            // (token p0 + 32 j + m) and rows 8 (i / 4) + 4 g + i % 4; after the
            // transpose lane l writes row 32 rt + m of tokens 2 q + g. The
            // lane's 16 rows' biases are loaded once, together, before any
            // store (stores may alias them, so they are not reloaded per tile)
            float bias0[16], bias1[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const size_t grow4 = (size_t)(rt * 32 + 8 * (i / 4) + 4 * g + (i % 4)) * 4;
                bias0[i] = *(const float *)(ex + A.off[MODE == 0 ? 2 : 8] + grow4);
                if constexpr (MODE == 0) bias1[i] = *(const float *)(ex + A.off[5] + grow4);
            }
#pragma unroll
            for (int j = 0; j < kNT; ++j) {
                if (j >= nt) break;
                int dst[16];   // MODE 1: the slot of each token this lane writes
                if constexpr (MODE == 1) {
#pragma unroll
                    for (int q = 0; q < 16; ++q) dst[q] = A.slot_of[base + min(p0 + 32 * j + 2 * q + g, T - 1)];
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rr = 8 * (i / 4) + 4 * g + (i % 4);
                    float v;
                    if constexpr (MODE == 0) {
                        float gg = acc0[j][i] + bias0[i];
                        float uu = acc1[j][i] + bias1[i];
                        if (A.act_plain) {
                            v = gg / (1.0f + expf(-gg)) * uu;
                        } else {
                            if (gg > A.limit) gg = A.limit;
                            if (uu > A.limit) uu = A.limit;
                            if (uu < -A.limit) uu = -A.limit;
                            v = gg / (1.0f + expf(-A.alpha * gg)) * (uu + 1.0f);
                        }
                    } else {
                        v = acc0[j][i] + bias0[i];
                    }
                    tl[m][rr] = v;   // [token][row]
                }
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int tok = 2 * q + g, p = p0 + 32 * j + tok;
                    if (p < T) {
                        const float v = tl[tok][m];
                        if constexpr (MODE == 0) A.hbuf[(size_t)(base + p) * A.F + rt * 32 + m] = v;
                        else A.ye[(size_t)dst[q] * A.H + rt * 32 + m] = v;
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    if (bad) atomicOr(A.err, 1u);
}

}  // namespace

// Assignments grouped by expert (offsets[E + 1], token and slot of each list
// position) in the S_LIST scratch; E <= 4096.
int launch_expert_lists(const int32_t *sel, int N, int E, int k, ExpertLists *out, hipStream_t s) {
    if (E > kPlistMaxE) return fail(MH_E_UNSUPPORTED, "expert lists: %d experts > %d", E, kPlistMaxE);
    void *pl;
    MH_TRY(scratch(S_LIST, sizeof(int) * ((size_t)E + 1 + 3 * (size_t)N), &pl));
    int *offs = (int *)pl, *rank = offs + E + 1;
    out->offs = offs;
    out->list_tok = rank + N;
    out->slot_of = rank + 2 * (size_t)N;
    MH_LAUNCH("plist", k_plist_one, dim3(1), dim3(1024), 0, s, sel, N, E, k, rank, offs, out->list_tok, out->slot_of);
    return hip_check(hipGetLastError(), "expert lists launch");
}

// True when the scaled-MFMA path handles this layer (MXFP4 experts, shapes
// that tile by 64 along K and 32 along rows, whose scales fit the GEMM's LDS).
bool prefill_mfma_ok(const DevLayer &L) {
    if (sw(SW_NO_MFMA)) return false;
    return L.expert_dt == MH_DT_MXFP4 && L.hidden % 64 == 0 && L.ffn % 64 == 0 && L.top_k >= 1 &&
           L.n_experts <= kPlistMaxE && L.hidden <= INT32_MAX && L.ffn <= INT32_MAX &&
           gemm_lds((int)L.hidden, 2).total <= kLdsMax && gemm_lds((int)L.ffn, 1).total <= kLdsMax;
}

// Expert-major MoE of n tokens: x[t] += sum over t's slots, in ascending
// expert order, of w * expert(xb[t]); ye is [n * k][H] scratch read by the
// prefill combine (launched by the caller), written for routed slots only.
int run_expert_major_mfma(const DevLayer &L, int n, const float *xb, const int32_t *sel, float *ye,
                          hipStream_t s) {
    const int k = L.top_k, E = L.n_experts, N = n * k;
    const int H = (int)L.hidden, F = (int)L.ffn;
    if (!prefill_mfma_ok(L)) return fail(MH_E_UNSUPPORTED, "prefill: layer shape not handled by the MFMA path");
    const size_t lds_gu = gemm_lds(H, 2).total, lds_dn = gemm_lds(F, 1).total;
    static uint64_t lds_epoch = 0;   // the initialisation the LDS attribute was set under
    if (lds_epoch != init_epoch()) {
        MH_HIP(hipFuncSetAttribute((const void *)k_moe_gemm<0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax));
        MH_HIP(hipFuncSetAttribute((const void *)k_moe_gemm<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax));
        lds_epoch = init_epoch();
    }
    unsigned *scale_err_dev = nullptr;
    MH_TRY(async_flag(F_PREFILL_SCALE, "prefill: an MXFP4 scale is not a positive power of two (e8m0 cannot hold it)",
                      &scale_err_dev));
    ExpertLists lists;
    MH_TRY(launch_expert_lists(sel, N, E, k, &lists, s));
    const int *offs = lists.offs, *list_tok = lists.list_tok, *slot_of = lists.slot_of;
    // quantized activations: the larger of x (n rows of H) and h (N rows of F)
    const size_t qx = (size_t)kTerms * n * H, qh = (size_t)kTerms * N * F;
    const size_t qbytes = std::max(qx + (size_t)kTerms * n * bscale_stride(H), qh + (size_t)kTerms * N * bscale_stride(F));
    void *pq, *ph;
    MH_TRY(scratch(S_Q, qbytes, &pq));
    MH_TRY(scratch(S_H, sizeof(float) * (size_t)N * F, &ph));
    uint8_t *q = (uint8_t *)pq;
    float *hbuf = (float *)ph;

    // ye rows of unroutable slots are not written: the combine skips them

    GemmArgs A;
    A.experts = L.experts;
    A.stride = L.expert_stride;
    for (int i = 0; i < 9; i++) A.off[i] = L.off[i];
    A.E = E;
    A.H = H;
    A.F = F;
    A.alpha = L.alpha;
    A.limit = L.limit;
    A.act_plain = L.act_plain;
    A.offs = offs;
    A.list_tok = list_tok;
    A.slot_of = slot_of;
    A.hbuf = hbuf;
    A.ye = ye;
    A.err = scale_err_dev;

    // gate/up over the quantized tokens
    {
        const int64_t thr = (int64_t)n * (H / 32);
        A.bq = q;
        A.bs = q + (size_t)kTerms * n * H;
        A.b_rows = n;
        MH_LAUNCH("quant_x", k_quant_terms, dim3((unsigned)((thr + 255) / 256)), dim3(256), 0, s, xb, nullptr, n, H,
                  q, q + (size_t)kTerms * n * H, bscale_stride(H));
        const int groups = (F / 32 + kWaves - 1) / kWaves;
        MH_LAUNCH("moe_gu_mfma", k_moe_gemm<0>, dim3((unsigned)((E * groups + 7) / 8 * 8)), dim3(64 * kWaves), lds_gu,
                  s, A);
    }
    // down over the quantized h (list order)
    {
        const int64_t thr = (int64_t)N * (F / 32);
        A.bq = q;
        A.bs = q + (size_t)kTerms * N * F;
        A.b_rows = N;
        MH_LAUNCH("quant_h", k_quant_terms, dim3((unsigned)((thr + 255) / 256)), dim3(256), 0, s, hbuf, nullptr, N,
                  F, q, q + (size_t)kTerms * N * F, bscale_stride(F));
        const int groups = (H / 32 + kWaves - 1) / kWaves;
        MH_LAUNCH("moe_down_mfma", k_moe_gemm<1>, dim3((unsigned)((E * groups + 7) / 8 * 8)), dim3(64 * kWaves),
                  lds_dn, s, A);
    }
    return hip_check(hipGetLastError(), "prefill MFMA launches");
}

}  // namespace mh
