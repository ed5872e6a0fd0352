// mh_grouped.hip — the expert FFN of a decode step of 2-16 tokens (at most
// 64 assignments) with each routed expert's weights read once for all the
// tokens routed to it: moe()'s per-slot expert work (engine/midge.c:514-541:
// gate and up matvecs + biases, the clamped SwiGLU, the down matvec + bias)
// regrouped by expert, as the reference's expert-major prefill groups tokens
// (engine/midge.c:591-611), on the f16 matrix cores.
//
//   groups  the top-k kernel's expert-sorted order (order[r] = assignment,
//           order[N + r] = its expert, unroutable ones last as -1) split into
//           runs of one expert and the runs into groups of up to kGT
//           assignments; every block derives the same table in its first
//           wave.
//   tiles   8 weight rows: a gate/up tile is 4 pairs (gate rows p0 .. p0 + 3
//           and up rows p0 .. p0 + 3), a down tile 8 rows. Block (x, g) takes
//           tiles [kTB x, +kTB) of group g, kTW per wave; blocks past the
//           groups exit, and the hardware's dispatch balances the rest.
//   A       a K step is 256 elements: one load instruction reads the tile's
//           8 rows x 128 contiguous bytes (whole cache lines), lane (m, g)
//           the 16-byte MXFP4 chunk 8 s + 2 g + (m >> 3) of row m & 7, kPD
//           steps ahead in a ring of registers that runs on across tiles;
//           e2m1 times the chunk's f16 scale converts to f16 exactly (the
//           stack's plan admits only scales that are zero or powers of two
//           in [2^-23, 2^13]). Matrix-core rows m and m + 8 then hold the
//           even and the odd chunks of the same weight row.
//   scales  a tile's f16 scales (8 rows x K / 32) are one or two contiguous
//           runs of whole 16-byte pieces: two loads per lane bring them into
//           the wave's LDS (double-buffered: the next tile's arrive while
//           this one's steps run), and each step reads its lane's scale
//           there. One 16-bit load per lane and step cost as much address
//           work as the step's weight load (92 vs 84 us per gate/up launch
//           at 16 tokens of gpt-oss-120b).
//   B       the group's inputs (xb of each assignment's token, or h of each
//           assignment) as two f16 terms, in columns 2j and 2j + 1 for the
//           even chunks and 8 + 2j, 9 + 2j for the odd ones (two LDS regions
//           placed so that a step's reads fall in distinct banks):
//           v' = v 2^-s, hi = RN(v'), lo = RN(v' - hi), with 2^s the power of
//           two that brings the column's max |v'| into [2^14, 2^15) (|v' - hi
//           - lo| <= 2^-22 |v'| + 2^-25); staged once per block, with the
//           biases of its tiles, while the first weight loads fly.
//   cost    the e2m1 -> f16 conversion (one instruction per two codes) on
//           the vector ALU bounds the kernel with the weight stream: at 16
//           tokens of gpt-oss-120b a gate/up launch converts ~40 experts'
//           weights in ~53 us with its loads served from cache, against ~65
//           us of HBM time.
//   output  C[r][n] + C[r + 8][n + 8] (even plus odd chunks) for n = 2j and
//           2j + 1 added and scaled by 2^s; gate/up: + biases, activation ->
//           h[a][p]; down: + bias -> ye[a][r]. The products and sums run in
//           another order than the reference's row dots, like every
//           matrix-core path here.
#include <algorithm>

#include "mh_gemv.cuh"
#include "mh_mfma16.cuh"

namespace mh {

namespace {

constexpr int kGW = 8;                     // waves per block
constexpr int kGThreads = 64 * kGW;
constexpr int kGT = 4;                     // assignments per group
constexpr int kGCols = 2 * kGT;            // B columns (hi, lo per assignment)
constexpr int kGMaxN = 64;                 // assignments per call (one wave builds the table)
constexpr int kGMaxK = 3072;               // hidden and ffn
constexpr int kGE = kGMaxK / kGThreads;    // staged B elements per thread and column
constexpr int kPD = 4;                     // K steps in flight per wave (a tile's steps: a multiple)
constexpr int kTW = 4;                     // tiles per wave
constexpr int kTB = kTW * kGW;             // tiles per block
constexpr int kGLdsMax = 80 * 1024;        // LDS per block (two blocks per CU)

struct GrpArgs {
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

// K steps of 256 per tile (rounded up to a multiple of kPD: the steps past
// K read zeros in B), and the f16 per B column of a region: the even (or
// odd) chunks of those steps, + 8, so that a column starts 4 banks after the
// previous one; the odd region starts 32 banks after the even one.
__host__ __device__ inline int grp_nq(int K) { return ((K / 32 + 7) / 8 + kPD - 1) / kPD * kPD; }
__host__ __device__ inline int grp_kh(int K) { return grp_nq(K) * 128 + 8; }

// LDS of a block (bytes, 16-aligned parts): B (two regions of kGCols
// columns), the staged biases (8 per tile), the group table, and per wave
// two tiles' weight scales (16 K / 32 bytes each).
struct GrpLds {
    size_t b, bias, tab, sc, total;
};
__host__ __device__ inline GrpLds grp_lds(int K) {
    GrpLds L;
    L.b = 0;
    L.bias = L.b + (size_t)2 * kGCols * grp_kh(K) * 2;
    L.tab = L.bias + (size_t)kTB * 8 * 4;
    L.sc = (L.tab + (size_t)(5 * kGMaxN + 8 + 2 * kGT) * 4 + 15) & ~(size_t)15;
    L.total = L.sc + (size_t)kGW * 2 * 16 * (K / 32);
    return L;
}

__device__ __forceinline__ float grp_act(float g, float u, float alpha, float limit, int plain) {
    if (plain) return g / (1.0f + expf(-g)) * u;
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    if (u < -limit) u = -limit;
    const float a = g / (1.0f + expf(-alpha * g));
    return a * (u + 1.0f);
}

// MODE 0: gate/up (K = H, tiles of 4 pairs); MODE 1: down (K = F, tiles of
// 8 rows).
// Two blocks per CU (their LDS fits twice) at four waves per SIMD (the
// launch bound's second argument, the minimum waves per SIMD, caps the
// registers at 128): the conversion work of some waves runs under the memory
// waits of others (at 3 waves per SIMD, 101 vs 92 us per gate/up launch at
// 16 tokens of gpt-oss-120b).
template <int MODE>
__global__ void __launch_bounds__(kGThreads, 4) k_grouped(GrpArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int K = MODE == 0 ? A.H : A.F;
    const int C = K / 32;   // 16-byte chunks per row
    const int NQ = grp_nq(K);   // K steps of 256 per tile (a multiple of kPD)
    const int kh = grp_kh(K);
    const GrpLds Ld = grp_lds(K);
    _Float16 *sB = (_Float16 *)(lds + Ld.b);
    float *sBias = (float *)(lds + Ld.bias);
    int *sGst = (int *)(lds + Ld.tab);   // [kGMaxN] group start (sorted position)
    int *sGcnt = sGst + kGMaxN;          // [kGMaxN] assignments in the group
    int *sGexp = sGcnt + kGMaxN;         // [kGMaxN] its expert
    int *sOrd = sGexp + kGMaxN;          // [kGMaxN] order[0 .. N): assignment at each sorted position
    int *sMisc = sOrd + kGMaxN;          // [8] groups, routed assignments
    int *sGa = sMisc + 8;                // [kGT] the staged group's assignments
    float *sGs = (float *)(sGa + kGT);   // [kGT] their columns' output scales 2^s
    float *sMax = (float *)(sGs + kGT);  // [kGMaxN] staging: per-wave column maxima
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
        const uint64_t rmask = __ballot(rstart);
        const uint64_t upto = r == 63 ? ~0ull : ((2ull << r) - 1);
        const uint64_t below = rmask & upto;
        const int rs = below ? 63 - __clzll((long long)below) : 0;   // this run's start
        const bool gstart = valid && (r - rs) % kGT == 0;
        const uint64_t gmask = __ballot(gstart);
        const int vend = __popcll(vmask);
        if (gstart) {
            const uint64_t above = rmask & ~upto;
            const int next_run = above ? __ffsll((long long)above) - 1 : 64;
            const int gi = __popcll(gmask & ((1ull << r) - 1));
            sGst[gi] = r;
            sGcnt[gi] = min(kGT, min(next_run, vend) - r);
            sGexp[gi] = e;
        }
        if (lane == 0) {
            sMisc[0] = __popcll(gmask);
            sMisc[1] = vend;
        }
    }
    __syncthreads();
    const int NG = sMisc[0], vend = sMisc[1];
    if (MODE == 1 && vend < N && blockIdx.y == 0) {   // unroutable assignments contribute y = 0
        const int nz = (N - vend) * A.H;
        for (int i = (int)blockIdx.x * kGThreads + t; i < nz; i += (int)gridDim.x * kGThreads) {
            const int r = vend + i / A.H;
            A.out[(size_t)sOrd[r] * A.H + (i - (r - vend) * A.H)] = 0.f;
        }
    }
    const int TPG = MODE == 0 ? A.F / 4 : A.H / 8;   // tiles per group
    const int g = (int)blockIdx.y;
    const int tb0 = (int)blockIdx.x * kTB, tb1 = min(tb0 + kTB, TPG);   // this block's tiles
    if (g >= NG || tb0 >= TPG) return;   // block-uniform

    const mh_rsrc rex = gemv_rsrc(A.experts, A.layer_bytes);
    const int m = lane & 15, gq = lane >> 4;
    const int r8 = m & 7, par = m >> 3;   // this lane's weight row in the tile, chunk parity
    const uint32_t rowbytes = (uint32_t)C * 16u;
    const uint32_t eo = (uint32_t)sGexp[g] * A.stride;
    // this wave's tiles [tw0, tw1) (none past the block's last)
    const int tw0 = min(tb0 + wave * kTW, tb1), tw1 = min(tw0 + kTW, tb1);
    const int nt = tw1 - tw0;

    // this lane's row of a tile: the byte offset of its data
    auto tile_row = [&](int tile) -> uint32_t {
        uint32_t row, od;
        if constexpr (MODE == 0) {
            row = 4u * (uint32_t)tile + (uint32_t)(r8 & 3);
            od = r8 < 4 ? A.off[0] : A.off[3];
        } else {
            row = 8u * (uint32_t)tile + (uint32_t)r8;
            od = A.off[6];
        }
        return eo + od + row * rowbytes;
    };
    // a tile's scales: C 16-byte pieces (gate/up: the 4 gate rows' run, then
    // the 4 up rows'; down: the 8 rows' run; 16-aligned since C is even),
    // kept in LDS with row r8 at byte 2 C r8
    uint8_t *sScW = lds + Ld.sc + (size_t)wave * 2 * 16 * C;   // this wave's two buffers
    auto sc_load = [&](int tile, mh_u4 (&v)[2]) __attribute__((always_inline)) {
        const uint32_t ut = (uint32_t)tile, uc = (uint32_t)C;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t p = (uint32_t)min(lane + 64 * u, C - 1);
            uint32_t a;
            if constexpr (MODE == 0)
                a = p < uc / 2 ? eo + A.off[1] + ut * 8u * uc + 16u * p : eo + A.off[4] + ut * 8u * uc + 16u * (p - uc / 2);
            else
                a = eo + A.off[7] + ut * 16u * uc + 16u * p;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rex, a, 0, 0);
        }
    };
    auto sc_store = [&](int buf, const mh_u4 (&v)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (lane + 64 * u < C) *(mh_u4 *)(sScW + (size_t)buf * 16 * C + 16 * (lane + 64 * u)) = v[u];
    };

    // the ring: step s's chunk in slot s % kPD (the cursors advance by
    // selects: stores to one of two counters under a condition would be
    // merged into a store through a chosen pointer, which keeps the counters
    // in scratch memory)
    mh_u4 qa[kPD];
    int t_p = min(max(tw0, tb0), tb1 - 1), q_p = 0;   // (a wave with no tiles reads one, unused)
    uint32_t rd_p = tile_row(t_p);
    auto issue = [&](int j) __attribute__((always_inline)) {
        const uint32_t cc = (uint32_t)min(8 * q_p + 2 * gq + par, C - 1);   // past K: a repeat (B is zero there)
        // (cached loads: non-temporal ones were slower here, 117 vs 102 us per
        // gate/up launch at 16 tokens of gpt-oss-120b)
        qa[j] = __builtin_amdgcn_raw_buffer_load_b128(rex, rd_p + 16u * cc, 0, 0);
        const bool wrap = q_p == NQ - 1;
        const bool adv = wrap && t_p + 1 < tw1;   // past the wave's tiles: the last again
        q_p = wrap ? 0 : q_p + 1;
        t_p = adv ? t_p + 1 : t_p;
        rd_p = tile_row(t_p);
    };

    // ---------------------------------------------------------- B
    // The group's inputs and the biases of the block's tiles (8 per tile:
    // gate/up bg of the 4 pairs then bu; down bd of the 8 rows) are loaded
    // first, then the ring's first steps, so that staging waits for its own
    // loads only (loads complete in issue order). Then each column's scale
    // from its max |v| (one barrier), and the terms, zeros past K.
    {
        const int gs = sGst[g], cnt = sGcnt[g];
        float bv[kGT][kGE];
#pragma unroll
        for (int j = 0; j < kGT; ++j) {
            if (j < cnt) {   // block-uniform
                const int a = sOrd[gs + j];
                const float *src = MODE == 0 ? A.in + (size_t)(a / A.k) * A.H : A.in + (size_t)a * A.F;
#pragma unroll
                for (int e = 0; e < kGE; ++e) bv[j][e] = src[min(t + e * kGThreads, K - 1)];
            }
        }
        const uint8_t *eb = A.experts + (size_t)eo;
        constexpr int kBP = (kTB * 8 + kGThreads - 1) / kGThreads;   // biases per thread
        float biasv[kBP];
#pragma unroll
        for (int u = 0; u < kBP; ++u) {
            const int i = t + u * kGThreads;
            const int btile = min(tb0 + (i >> 3), tb1 - 1), br = i & 7;
            if constexpr (MODE == 0)
                biasv[u] = ((const float *)(eb + (br < 4 ? A.off[2] : A.off[5])))[4 * btile + (br & 3)];
            else
                biasv[u] = ((const float *)(eb + A.off[8]))[8 * btile + br];
        }
        mh_u4 sc0[2];   // the wave's first tile's scales
        sc_load(t_p, sc0);
        for (int j = 0; j < kPD; ++j) issue(j);
        sc_store(0, sc0);
#pragma unroll
        for (int u = 0; u < kBP; ++u)
            if (t + u * kGThreads < kTB * 8) sBias[t + u * kGThreads] = biasv[u];
#pragma unroll
        for (int j = 0; j < kGT; ++j) {
            if (j >= cnt) break;   // block-uniform
            float mx = 0.f;
#pragma unroll
            for (int e = 0; e < kGE; ++e)
                if (t + e * kGThreads < K) mx = fmaxf(mx, fabsf(bv[j][e]));
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            if (lane == 0) sMax[wave * kGT + j] = mx;
        }
        __syncthreads();
        // element k: chunk c = k / 32 in region c & 1 at (c >> 1) 32 + k % 32
        // of its column; k < NQ 256 covers every step (zeros past K). The
        // columns past the group's are not written: a matrix-core output
        // column reads only its own B column, and theirs are not used.
#pragma unroll
        for (int j = 0; j < kGT; ++j) {
            if (j >= cnt) {   // block-uniform
                if (t == 0) sGa[j] = -1;
                continue;
            }
            float down;
            {
                float mx = 0.f;
                for (int w = 0; w < kGW; ++w) mx = fmaxf(mx, sMax[w * kGT + j]);
                // 2^s with max |v| 2^-s in [2^14, 2^15): s = e - 15 for
                // max = f 2^e, f in [0.5, 1) (s = 0 for a zero, subnormal or
                // non-finite max)
                const int be = (int)((__float_as_uint(mx) >> 23) & 255u);   // mx in [2^(be-127), 2^(be-126))
                const int sh = (be > 0 && mx <= 3.0e38f) ? be - 126 - 15 : 0;
                down = ldexpf(1.0f, -sh);
                if (t == 0) {
                    sGa[j] = sOrd[gs + j];
                    sGs[j] = ldexpf(1.0f, sh);
                }
            }
#pragma unroll
            for (int e = 0; e < kGE; ++e) {
                const int k = t + e * kGThreads;
                if (k < NQ * 256) {
                    const float v = k < K ? bv[j][e] * down : 0.f;
                    const _Float16 h = (_Float16)v;
                    const int c = k >> 5;
                    _Float16 *col = sB + ((size_t)(c & 1) * kGCols + 2 * j) * kh + (c >> 1) * 32 + (k & 31);
                    col[0] = h;                                // hi
                    col[kh] = (_Float16)(v - (float)h);        // lo (the next column)
                }
            }
        }
        __syncthreads();
    }
    if (nt <= 0) return;   // wave-uniform; no barrier follows

    const int cnt = sGcnt[g];
    // B lane (n, g): region n >> 3, column n & 7, local chunk 4 s + g
    const _Float16 *bcol = sB + ((size_t)par * kGCols + r8) * kh + 32 * gq;
    // A tile's steps run in groups of kPD (ring slot j = step % kPD, a
    // constant), the accumulators live in the matrix-core registers across
    // them, and the outputs follow the tile's last group.
    for (int tile = tw0; tile < tw1; ++tile) {
        const int buf = (tile - tw0) & 1;
        mh_u4 scn[2];   // the next tile's scales (the wave's last tile re-reads its own, unused)
        sc_load(min(tile + 1, tw1 - 1), scn);
        const uint16_t *scr = (const uint16_t *)(sScW + (size_t)buf * 16 * C) + r8 * C;   // this lane's row
        v4f acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
        for (int q0 = 0; q0 < NQ; q0 += kPD) {
            uint16_t scq[kPD];
#pragma unroll
            for (int j = 0; j < kPD; ++j) scq[j] = scr[min(8 * (q0 + j) + 2 * gq + par, C - 1)];
#pragma unroll
            for (int j = 0; j < kPD; ++j) {
                const float sc = mh_f16(scq[j]);
                const _Float16 *bp = bcol + 128 * (q0 + j);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const v8h hb = *(const v8h *)(bp + 8 * i);
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp4x8_f16(dword_of(qa[j], i), sc), hb, acc[i], 0,
                                                                    0, 0);
                }
                issue(j);
            }
        }
        sc_store(buf ^ 1, scn);   // the wave reads its own LDS in order: no barrier
        // ---- the tile's outputs
        const int tl = tile - tb0;   // the tile's place in the staged biases
        const v4f accs = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        // lane (n < 8, gq < 2) holds C[4 gq + i][n]; lane + 40 holds
        // C[4 gq + i + 8][n + 8]: even plus odd chunks, then the column pair
        // (hi, lo) of assignment n / 2
        float w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = accs[i] + __shfl(accs[i], (lane + 40) & 63);
            w[i] = v + dpp_shl<1>(v);
        }
        const int a = m >> 1;
        const bool mine = m < 2 * cnt && (m & 1) == 0;
        if constexpr (MODE == 0) {
            // gate rows 0-3 (gq 0), up rows 4-7 (gq 1): up from lane + 16
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float u = __shfl(w[i], (lane + 16) & 63);
                if (mine && gq == 0) {
                    const float gv = w[i] * sGs[a] + sBias[tl * 8 + i];
                    const float uv = u * sGs[a] + sBias[tl * 8 + 4 + i];
                    A.out[(size_t)sGa[a] * A.F + 4 * tile + i] = grp_act(gv, uv, A.alpha, A.limit, A.act_plain);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (mine && gq < 2)
                    A.out[(size_t)sGa[a] * A.H + 8 * tile + 4 * gq + i] = w[i] * sGs[a] + sBias[tl * 8 + 4 * gq + i];
        }
    }
}

}  // namespace

bool grouped_ok(const DevLayer &L, int n) {
    const int64_t N = (int64_t)n * L.top_k;
    return L.expert_dt == MH_DT_MXFP4 && n >= 2 && N <= kGMaxN && L.hidden % 64 == 0 && L.ffn % 64 == 0 &&
           L.hidden <= kGMaxK && L.ffn <= kGMaxK &&
           L.expert_stride % 16 == 0 && L.expert_stride * (uint64_t)L.n_experts < (1ull << 32) &&
           (uintptr_t)L.experts % 16 == 0 && L.off[0] % 16 == 0 && L.off[3] % 16 == 0 && L.off[6] % 16 == 0 &&
           L.off[1] % 16 == 0 && L.off[4] % 16 == 0 && L.off[7] % 16 == 0 &&
           L.off[2] % 4 == 0 && L.off[5] % 4 == 0 && L.off[8] % 4 == 0;
}

// The expert FFN of n tokens (grouped_ok) from the top-k kernel's expert-
// sorted order: h (scratch [N][F]) from xb, then ye [N][H].
int launch_grouped(const DevLayer &L, int n, const int32_t *order, const float *xb, float *h, float *ye,
                   hipStream_t s) {
    if (!grouped_ok(L, n)) return fail(MH_E_UNSUPPORTED, "grouped expert path: shape not handled");
    GrpArgs A;
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
    const GrpLds l0 = grp_lds(A.H), l1 = grp_lds(A.F);
    if (l0.total > kGLdsMax || l1.total > kGLdsMax)
        return fail(MH_E_UNSUPPORTED, "grouped expert path: LDS of %zu / %zu bytes per block", l0.total, l1.total);
    static int ready_dev = -1;
    int dev = 0;
    MH_HIP(hipGetDevice(&dev));
    if (ready_dev != dev) {
        MH_HIP(hipFuncSetAttribute((const void *)k_grouped<0>, hipFuncAttributeMaxDynamicSharedMemorySize, kGLdsMax));
        MH_HIP(hipFuncSetAttribute((const void *)k_grouped<1>, hipFuncAttributeMaxDynamicSharedMemorySize, kGLdsMax));
        ready_dev = dev;
    }
    // groups <= assignments: blocks (x, g) for g past the groups exit
    const unsigned ny = (unsigned)A.N;
    A.in = xb;
    A.out = h;
    MH_LAUNCH("grouped_gu", k_grouped<0>, dim3((unsigned)((A.F / 4 + kTB - 1) / kTB), ny), dim3(kGThreads), l0.total, s,
              A);
    MH_TRY(hip_check(hipGetLastError(), "grouped gate/up launch"));
    A.in = h;
    A.out = ye;
    MH_LAUNCH("grouped_down", k_grouped<1>, dim3((unsigned)((A.H / 8 + kTB - 1) / kTB), ny), dim3(kGThreads),
              l1.total, s, A);
    return hip_check(hipGetLastError(), "grouped down launch");
}

}  // namespace mh
