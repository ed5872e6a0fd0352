// mh_fewtok.hip — the expert FFN of a decode step of a few tokens (2 to 16,
// at most 64 assignments) on the f16 matrix cores: moe()'s per-slot expert
// work (engine/midge.c:514-541: gate and up matvecs + biases, the clamped
// SwiGLU, the down matvec + bias) with the assignments grouped by expert, so
// that each routed expert's weights are read and converted once for all the
// tokens routed to it instead of once per assignment.
//
//   groups    the top-k kernel's expert-sorted order (order[r] = assignment,
//             order[N + r] = its expert, unroutable ones last as -1) split
//             into runs of one expert and the runs into groups of up to kFM
//             assignments; every block derives the same table in its first
//             wave.
//   work      (group, chunk): a chunk is one tile per wave. Gate/up tiles are
//             8 pairs (gate rows p0 .. p0 + 7 over up rows p0 .. p0 + 7: one
//             16-row matrix-core tile, so a pair's gate and up land in one
//             wave), down tiles 16 rows. Block b takes the contiguous range
//             [W b / NB, W (b + 1) / NB) of the W = groups x chunks items.
//   A         the tile's rows, two 8-row ranges, each contiguous in memory,
//             loaded whole (1 KB per wave instruction) into registers and
//             stored to the wave's LDS region; the next item's loads are
//             issued before this item's math, so one item's transfer runs
//             under the previous one's matrix-core work. e2m1 times the
//             chunk's f16 scale is converted to f16 exactly (the stack's plan
//             admits only scales that are zero or powers of two in [2^-23,
//             2^13]).
//   B         the group's inputs (xb of each assignment's token, or h of each
//             assignment) as two f16 terms in columns 2j and 2j + 1: v' = v
//             2^-s, hi = v' rounded, lo = v' - hi rounded (v' within 2^-22
//             |v'|), with s >= 0 the smallest power that keeps the column
//             below 2^15; staged in LDS whenever the block's group changes.
//   output    the f32 accumulators of columns 2j and 2j + 1 are added and
//             scaled by 2^s; gate/up: + biases, activation -> h[a][p]; down:
//             + bias -> ye[a][r]. The products and sums run in another order
//             than the reference's row dots, like every matrix-core path here.
#include <algorithm>

#include "mh_gemv.cuh"
#include "mh_mfma16.cuh"

namespace mh {

namespace {

constexpr int kFWaves = 4;
constexpr int kFThreads = 64 * kFWaves;
constexpr int kFM = 4;          // assignments per group (B columns 2 kFM)
constexpr int kFMaxN = 64;      // assignments per call (one wave builds the table)
constexpr int kFMaxK = 3072;    // hidden and ffn
constexpr int kFLoads = 12;     // 1 KB loads per 8-row range (8 x kFMaxK / 2 bytes)
constexpr int kFScLoads = 2;    // 1 KB loads per 8-row scale window (<= 15 + 8 x kFMaxK / 16 bytes)
constexpr int kFE = kFMaxK / kFThreads;   // B elements per thread and column
static_assert(kFLoads * 1024 >= 8 * kFMaxK / 2, "an 8-row range per kFLoads wave loads");
static_assert(kFScLoads * 1024 >= 15 + 8 * (kFMaxK / 32) * 2, "an 8-row scale window per kFScLoads wave loads");

struct FewArgs {
    const uint8_t *experts;   // the layer's expert table
    uint32_t layer_bytes;     // E x stride (< 4 GiB)
    uint32_t stride;
    uint32_t off[9];          // wt_expert_layout offsets (engine/mten.h:136-150)
    int H, F, N, k;           // hidden, ffn, assignments (n k), slots per token
    float alpha, limit;
    int act_plain;
    const int32_t *order;     // [2 N]
    const float *in;          // gate/up: xb [n][H]; down: h [N][F]
    float *out;               // gate/up: h [N][F]; down: ye [N][H]
};

// LDS of a block for K input columns (bytes, all 16-aligned).
struct FewLds {
    size_t b, a, s, r, g, bias, total;
    int rsp, kp, sw;
};
__host__ __device__ inline FewLds few_lds(int K) {
    FewLds L;
    L.kp = (K + 127) / 128 * 128 + 8;   // f16 per B column: zeros to whole 128-column steps, + 8 (banks)
    L.rsp = K / 2 + 16;            // bytes per staged row
    L.sw = (K / 32) * 16 + 16;     // bytes per 8-row scale window
    L.b = 0;
    L.a = L.b + (size_t)2 * kFM * L.kp * 2;
    L.s = L.a + (size_t)kFWaves * 16 * L.rsp;
    L.r = L.s + (size_t)kFWaves * 2 * L.sw;
    L.g = L.r + (size_t)kFWaves * 16 * kFM * 4;
    L.total = L.g + (size_t)(4 * kFMaxN + 8 + 2 * kFM) * 4;
    L.bias = L.total;              // [kFWaves][16] f32: the staged item's biases
    L.total += (size_t)kFWaves * 16 * 4;
    return L;
}

__device__ __forceinline__ mh_u4 few_ld16(mh_rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kGemvNT);
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float few_act(float g, float u, float alpha, float limit, int plain) {
    if (plain) return g / (1.0f + expf(-g)) * u;
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    if (u < -limit) u = -limit;
    const float a = g / (1.0f + expf(-alpha * g));
    return a * (u + 1.0f);
}

// MODE 0: gate/up (K = H, tiles of 8 pairs); MODE 1: down (K = F, tiles of
// 16 rows).
template <int MODE>
__global__ void __launch_bounds__(kFThreads) k_fewtok(FewArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int K = MODE == 0 ? A.H : A.F;
    const int RB = K / 2, CH = K / 32;
    const FewLds Ld = few_lds(K);
    _Float16 *sB = (_Float16 *)(lds + Ld.b);
    uint8_t *sA = lds + Ld.a;
    uint8_t *sS = lds + Ld.s;
    float *sR = (float *)(lds + Ld.r);
    int *sG = (int *)(lds + Ld.g);   // [kFMaxN] start, [kFMaxN] count, [kFMaxN] expert, groups, valid
    int *sGa = sG + 3 * kFMaxN + 8;  // [kFM] the staged group's assignments (-1 past its count)
    float *sGs = (float *)(sGa + kFM);   // [kFM] their columns' output scales 2^s
    float *sBias = (float *)(lds + Ld.bias);
    int *sOrd = (int *)(sGs + kFM);      // [kFMaxN] order[0 .. N): the assignment at each sorted position
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int N = A.N;

    // ---------------------------------------------------------- groups
    if (wave == 0) {
        const int r = lane;
        const int e = r < N ? A.order[N + r] : -1;
        sOrd[r] = r < N ? A.order[r] : 0;
        const int ep = __shfl_up(e, 1);
        const bool valid = e >= 0;
        const uint64_t vmask = __ballot(valid);   // a prefix: unroutable assignments sort last
        const bool rstart = valid && (r == 0 || e != ep);
        const uint64_t rs_mask = __ballot(rstart);
        const uint64_t upto = r == 63 ? ~0ull : ((2ull << r) - 1);
        const uint64_t below = rs_mask & upto;
        const int rs = below ? 63 - __clzll((long long)below) : 0;
        const int gsq = rs + ((r - rs) / kFM) * kFM;
        const bool gstart = valid && r == gsq;
        const uint64_t gs_mask = __ballot(gstart);
        const int vend = __popcll(vmask);
        if (gstart) {
            const uint64_t above = rs_mask & ~upto;
            const int nx = above ? __ffsll((long long)above) - 1 : 64;
            const int gi = __popcll(gs_mask & ((1ull << r) - 1));
            sG[gi] = r;
            sG[kFMaxN + gi] = min(kFM, min(nx, vend) - r);
            sG[2 * kFMaxN + gi] = e;
        }
        if (lane == 0) {
            sG[3 * kFMaxN] = __popcll(gs_mask);
            sG[3 * kFMaxN + 1] = vend;
        }
    }
    __syncthreads();
    const int NG = sG[3 * kFMaxN], vend = sG[3 * kFMaxN + 1];
    const int NB = (int)gridDim.x, b = (int)blockIdx.x;
    if (MODE == 1 && vend < N) {   // unroutable assignments contribute y = 0
        const int nz = (N - vend) * A.H;
        for (int i = b * kFThreads + t; i < nz; i += NB * kFThreads) {
            const int r = vend + i / A.H;
            A.out[(size_t)sOrd[r] * A.H + (i - (r - vend) * A.H)] = 0.f;
        }
    }
    const int TPG = MODE == 0 ? A.F / 8 : A.H / 16;   // tiles per group
    const int CPG = (TPG + kFWaves - 1) / kFWaves;    // chunks per group
    const int64_t W = (int64_t)NG * CPG;
    const int w0 = (int)(W * b / NB), w1 = (int)(W * (b + 1) / NB);
    if (w0 >= w1) return;   // block-uniform

    const mh_rsrc rex = gemv_rsrc(A.experts, A.layer_bytes);
    const uint32_t rng = 8u * (uint32_t)RB;          // bytes of an 8-row range
    const uint32_t srng = 8u * (uint32_t)CH * 2u;    // bytes of its scales
    // this lane's place in a range for load i: offset i 1024 + 16 lane ->
    // (row, column), stepped by 1024 bytes
    int row0 = (16 * lane) / RB, col0 = 16 * lane - row0 * RB;

    // Two items in flight per wave, each in its own register set (the loop
    // below alternates them, so every index is static): an item's rows,
    // scale windows, its 16 biases (lanes 0-3, 16 bytes each: gate/up bg of
    // the 8 pairs then bu; down bd of the 16 rows) and its scale ranges'
    // offsets in their windows. Everything loaded goes to LDS whole, so no
    // loaded register is copied (a copy would wait for every load in
    // flight).
    struct Set {
        mh_u4 qa[2][kFLoads], qs[2][kFScLoads], qb;
        uint32_t nmis[2];
    };
    Set s0, s1;
    uint32_t mis[2] = {0u, 0u};   // of the staged item
    auto item = [&](int w, int &g, int &tile) {
        g = w / CPG;
        tile = (w - g * CPG) * kFWaves + wave;
    };
    auto issue = [&](int w, Set &S) __attribute__((always_inline)) {
        mh_u4(&qa)[2][kFLoads] = S.qa;
        mh_u4(&qs)[2][kFScLoads] = S.qs;
        uint32_t(&nmis)[2] = S.nmis;
        int g, tile;
        item(w, g, tile);
        tile = min(tile, TPG - 1);   // past the group's tiles: a repeat that is not used
        const uint32_t eo = (uint32_t)sG[2 * kFMaxN + g] * A.stride;
        uint32_t base[2], sbase[2];
        if constexpr (MODE == 0) {
            const uint32_t p0 = 8u * (uint32_t)tile;
            base[0] = eo + A.off[0] + p0 * RB;
            base[1] = eo + A.off[3] + p0 * RB;
            sbase[0] = eo + A.off[1] + p0 * CH * 2u;
            sbase[1] = eo + A.off[4] + p0 * CH * 2u;
        } else {
            const uint32_t r0 = 16u * (uint32_t)tile;
            base[0] = eo + A.off[6] + r0 * RB;
            base[1] = base[0] + rng;
            sbase[0] = eo + A.off[7] + r0 * CH * 2u;
            sbase[1] = sbase[0] + srng;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < kFLoads; ++i) {
                const uint32_t o = (uint32_t)(i * 1024 + 16 * lane);
                qa[h][i] = few_ld16(rex, base[h] + min(o, rng - 16u));
            }
            nmis[h] = sbase[h] & 15u;
            const uint32_t win = nmis[h] + srng;
#pragma unroll
            for (int i = 0; i < kFScLoads; ++i) {
                const uint32_t o = (uint32_t)(i * 1024 + 16 * lane);
                qs[h][i] = few_ld16(rex, (sbase[h] & ~15u) + min(o, ((win + 15u) & ~15u) - 16u));
            }
        }
        const int lb = lane & 3;
        if constexpr (MODE == 0)
            S.qb = few_ld16(rex, eo + (lb < 2 ? A.off[2] : A.off[5]) + (8u * (uint32_t)tile + 4u * (lb & 1)) * 4u);
        else
            S.qb = few_ld16(rex, eo + A.off[8] + (16u * (uint32_t)tile + 4u * lb) * 4u);
    };
    // the oldest item in flight into this wave's LDS region
    auto stage = [&](const Set &S) __attribute__((always_inline)) {
        const mh_u4(&qa)[2][kFLoads] = S.qa;
        const mh_u4(&qs)[2][kFScLoads] = S.qs;
        const uint32_t(&nmis)[2] = S.nmis;
        uint8_t *a = sA + (size_t)wave * 16 * Ld.rsp;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int row = row0, col = col0;
#pragma unroll
            for (int i = 0; i < kFLoads; ++i) {
                if (row < 8) *(mh_u4 *)(a + (size_t)(8 * h + row) * Ld.rsp + col) = qa[h][i];
                col += 1024;
                while (col >= RB) {
                    col -= RB;
                    ++row;
                }
            }
            uint8_t *sc = sS + (size_t)(2 * wave + h) * Ld.sw;
#pragma unroll
            for (int i = 0; i < kFScLoads; ++i) {
                const int o = i * 1024 + 16 * lane;
                if (o < Ld.sw) *(mh_u4 *)(sc + o) = qs[h][i];
            }
            mis[h] = nmis[h];
        }
        if (lane < 4) *(mh_u4 *)(sBias + wave * 16 + 4 * lane) = S.qb;
    };
    // The group's B columns in two steps (block-wide): load_b issues every
    // load of the group's inputs at once (a wave's loads complete in issue
    // order, so the conversion waits one round trip, behind the weight
    // loads already in flight); store_b finds each column's scale (one
    // barrier), converts and stores the terms. Callers put a barrier before
    // (the previous group's B is no longer read) and after.
    float bv[kFM][kFE];
    auto load_b = [&](int g) __attribute__((always_inline)) {
        const int gs = sG[g], cnt = sG[kFMaxN + g];
#pragma unroll
        for (int j = 0; j < kFM; ++j) {
            const int a = sOrd[gs + min(j, cnt - 1)];
            const float *src = MODE == 0 ? A.in + (size_t)(a / A.k) * A.H : A.in + (size_t)a * A.F;
#pragma unroll
            for (int e = 0; e < kFE; ++e) bv[j][e] = src[min(t + e * kFThreads, K - 1)];
        }
    };
    auto store_b = [&](int g) __attribute__((always_inline)) {
        const int gs = sG[g], cnt = sG[kFMaxN + g];
        // each column's scale: 2^-s with s >= 0 the smallest that keeps
        // max |v| 2^-s below 2^15 (f16 holds the hi term)
#pragma unroll
        for (int j = 0; j < kFM; ++j) {
            float mx = 0.f;
#pragma unroll
            for (int e = 0; e < kFE; ++e) mx = fmaxf(mx, fabsf(bv[j][e]));
            mx = wave_max_f(mx);
            if (lane == 0) sR[wave * kFM + j] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kFM; ++j) {
            if (j >= cnt) break;   // block-uniform
            const float mx = fmaxf(fmaxf(sR[j], sR[kFM + j]), fmaxf(sR[2 * kFM + j], sR[3 * kFM + j]));
            int sh = 0;
            if (mx >= 32768.f && mx <= 3.0e38f) sh = (int)ceilf(log2f(mx / 32768.f)) + 1;
            const float down = ldexpf(1.0f, -sh);
            _Float16 *hi = sB + (size_t)(2 * j) * Ld.kp, *lo = hi + Ld.kp;
#pragma unroll
            for (int e = 0; e < kFE; ++e) {
                const int i = t + e * kFThreads;
                if (i < K) {
                    const float v = bv[j][e] * down;
                    const _Float16 h = (_Float16)v;
                    hi[i] = h;
                    lo[i] = (_Float16)(v - (float)h);
                }
            }
            for (int i = K + t; i < Ld.kp; i += kFThreads) hi[i] = lo[i] = (_Float16)0.f;
            if (t == 0) {
                sGa[j] = sOrd[gs + j];
                sGs[j] = ldexpf(1.0f, sh);
            }
        }
        if (t < kFM && t >= cnt) sGa[t] = -1;
    };

    const int m = lane & 15, gq = lane >> 4;
    int cur = -1;
    // item w from S, then item wn's loads into S
    auto body = [&](int w, Set &S, int wn) __attribute__((always_inline)) {
        int g, tile;
        item(w, g, tile);
        stage(S);
        const float *bias = sBias + wave * 16;
        if (g != cur) {   // block-uniform: the block's range enters the next group
            __syncthreads();   // every wave is done with the previous group's B
            load_b(g);
            store_b(g);
            __syncthreads();
            cur = g;
        }
        issue(wn, S);
        const int cnt = sG[kFMaxN + g];
        const int ncol = 2 * cnt;
        // ---- the tile's products: 16 rows x the group's columns over K, two
        // accumulators (instructions j even / odd) so that consecutive
        // matrix-core instructions do not wait on each other
        const uint8_t *ar = sA + (size_t)wave * 16 * Ld.rsp + (size_t)m * Ld.rsp;
        const uint8_t *sr = sS + (size_t)(2 * wave + (m >> 3)) * Ld.sw + mis[m >> 3] + (size_t)(m & 7) * CH * 2;
        const _Float16 *bc = sB + (size_t)m * Ld.kp;
        // Every lane reads B: a column past the group's (stale LDS) only
        // feeds an output column that is not used, and the chunks past K
        // (clamped A) meet the columns' zero padding. The next step's
        // operands are read before this step's math; four accumulators keep
        // the matrix-core instructions independent.
        v4f acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
        const int NQ = (CH + 3) >> 2;
        auto rd = [&](int q, mh_u4 &w4, float &sc, v8h (&hb)[4]) __attribute__((always_inline)) {
            const int cc = min(4 * q + gq, CH - 1);
            w4 = *(const mh_u4 *)(ar + (size_t)cc * 16);
            sc = mh_f16(*(const uint16_t *)(sr + (size_t)cc * 2));
#pragma unroll
            for (int j = 0; j < 4; ++j) hb[j] = *(const v8h *)(bc + 128 * q + 32 * gq + 8 * j);
        };
        mh_u4 w4n;
        float scn;
        v8h hbn[4];
        rd(0, w4n, scn, hbn);
        for (int q = 0; q < NQ; ++q) {
            const mh_u4 w4 = w4n;
            const float sc = scn;
            v8h hb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) hb[j] = hbn[j];
            rd(min(q + 1, NQ - 1), w4n, scn, hbn);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp4x8_f16(dword_of(w4, j), sc), hb[j], acc[j], 0, 0, 0);
        }
        const v4f accs = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        // ---- epilogue: column pairs summed and scaled
        const bool live = tile < TPG;
        float *rr = sR + (size_t)wave * 16 * kFM;
        if constexpr (MODE == 0) {
            // rows 4 gq + i of column m; pair results through the wave's LDS
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = accs[i] + dpp_shl<1>(accs[i]);
                if ((m & 1) == 0 && m < ncol) rr[(4 * gq + i) * kFM + (m >> 1)] = v * sGs[m >> 1];
            }
            __builtin_amdgcn_wave_barrier();
            const int p = lane >> 2, j = lane & 3;   // lanes 0-31: pair p, assignment j
            if (live && lane < 32 && j < cnt) {
                const float gv = rr[p * kFM + j] + bias[p];
                const float uv = rr[(8 + p) * kFM + j] + bias[8 + p];
                A.out[(size_t)sGa[j] * A.F + 8 * tile + p] = few_act(gv, uv, A.alpha, A.limit, A.act_plain);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = accs[i] + dpp_shl<1>(accs[i]);
                if (live && (m & 1) == 0 && m < ncol)
                    A.out[(size_t)sGa[m >> 1] * A.H + 16 * tile + 4 * gq + i] = v * sGs[m >> 1] + bias[4 * gq + i];
            }
        }
        __builtin_amdgcn_wave_barrier();   // rr is rewritten by the next item
    };
    {   // the first group's inputs, then the first two items' weights
        int g, tile;
        item(w0, g, tile);
        load_b(g);
        issue(w0, s0);
        issue(min(w0 + 1, w1 - 1), s1);
        store_b(g);
        __syncthreads();
        cur = g;
    }
    // Two items per pass with no condition on either (a condition would make
    // the compiler copy the register sets at the loop edge, which waits for
    // every load in flight): past the range's end the last item is loaded
    // again, and for an odd count recomputed, rewriting the same outputs.
    for (int w = w0; w < w1; w += 2) {
        body(w, s0, min(w + 2, w1 - 1));
        body(min(w + 1, w1 - 1), s1, min(w + 3, w1 - 1));
    }
}

}  // namespace

bool fewtok_ok(const DevLayer &L, int n) {
    const int64_t N = (int64_t)n * L.top_k;
    return L.expert_dt == MH_DT_MXFP4 && n >= 2 && N <= kFMaxN && L.hidden % 32 == 0 && L.ffn % 32 == 0 &&
           L.hidden <= kFMaxK && L.ffn <= kFMaxK && L.expert_stride % 16 == 0 &&
           L.expert_stride * (uint64_t)L.n_experts < (1ull << 32) && (uintptr_t)L.experts % 16 == 0 &&
           L.off[0] % 16 == 0 && L.off[3] % 16 == 0 && L.off[6] % 16 == 0 &&
           few_lds((int)std::max(L.hidden, L.ffn)).total <= 160 * 1024;
}

// The expert FFN of n tokens (fewtok_ok) from the top-k kernel's expert-
// sorted order: h (scratch [N][F]) from xb, then ye [N][H].
int launch_fewtok(const DevLayer &L, int n, const int32_t *order, const float *xb, float *h, float *ye,
                  hipStream_t s) {
    if (!fewtok_ok(L, n)) return fail(MH_E_UNSUPPORTED, "few-token expert path: shape not handled");
    FewArgs A;
    A.experts = L.experts;
    A.layer_bytes = (uint32_t)(L.expert_stride * (uint64_t)L.n_experts);
    A.stride = (uint32_t)L.expert_stride;
    for (int i = 0; i < 9; i++) A.off[i] = (uint32_t)L.off[i];
    A.H = (int)L.hidden;
    A.F = (int)L.ffn;
    A.N = n * L.top_k;
    A.k = L.top_k;
    A.alpha = L.alpha;
    A.limit = L.limit;
    A.act_plain = L.act_plain;
    A.order = order;
    static int ready_dev = -1;
    int dev = 0;
    MH_HIP(hipGetDevice(&dev));
    if (ready_dev != dev) {
        MH_HIP(hipFuncSetAttribute((const void *)k_fewtok<0>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        MH_HIP(hipFuncSetAttribute((const void *)k_fewtok<1>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        ready_dev = dev;
    }
    const int nb = device_cus();
    A.in = xb;
    A.out = h;
    MH_LAUNCH("fewtok_gu", k_fewtok<0>, dim3((unsigned)nb), dim3(kFThreads), few_lds(A.H).total, s, A);
    MH_TRY(hip_check(hipGetLastError(), "few-token gate/up launch"));
    A.in = h;
    A.out = ye;
    MH_LAUNCH("fewtok_down", k_fewtok<1>, dim3((unsigned)nb), dim3(kFThreads), few_lds(A.F).total, s, A);
    return hip_check(hipGetLastError(), "few-token down launch");
}

}  // namespace mh
