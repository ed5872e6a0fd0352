// mh_prefill.hip — expert-major prefill of one MoE layer with CDNA4 scaled
// MFMA: forward_batch()'s route + expert-major block (engine/midge.c:591-611)
// with expert_apply (engine/midge.c:437-467) as one grouped GEMM per routed
// expert over the tokens routed to it.
//
//   lists      assignments (token t, slot i) grouped by expert: counts,
//              offsets, token of each list position, slot of each position
//   quantize   xb (per token) -> kTerms planes of fp8 e4m3 with an e8m0
//              scale per 32-element block: x = sum_t q_t * 2^e_t, each term
//              the rounding residual of the previous one (3 terms keep the
//              f32 GEMM's accuracy to ~1.5e-5 relative)
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
// Operand layout of the 32x32x64 instruction (measured on gfx950): lane l
// holds A row l % 32 and B column l % 32; with g = l / 32, A's 16 bytes (32
// e2m1 values) and B's 32 bytes (32 e4m3 values) pair as
//   K  0-15: A group 0 nibbles  0-15,  B group 0 bytes  0-15
//   K 16-31: A group 1 nibbles  0-15,  B group 0 bytes 16-31
//   K 32-47: A group 0 nibbles 16-31,  B group 1 bytes  0-15
//   K 48-63: A group 1 nibbles 16-31,  B group 1 bytes 16-31
// and the scale blocks of both operands follow A: lane (., g)'s scale covers
// K 0-15 + 32-47 (g = 0) or K 16-31 + 48-63 (g = 1). So for K step s (weight
// columns 64s .. 64s+63) A lane (m, g) loads 16-byte chunk 2s+g of row m (one
// MXFP4 block and its scale); B lane (n, g) loads columns 64s+16g+[0,16) and
// 64s+32+16g+[0,16) of token n with the scale of column block 2s+g. The
// activations are therefore quantized in natural 32-column blocks, like the
// weights. Output lane l: column l % 32, rows 8(i/4) + 4g + i%4 for
// accumulator i.
#include <stdlib.h>

#include <algorithm>

#include "mh_internal.h"

namespace mh {

namespace {

constexpr int kTerms = 3;      // fp8 terms per activation
constexpr int kNT = 4;         // 32-token tiles per pass (weights loaded once per pass)
constexpr int kWaves = 4;      // 32-row tiles per block (one per wave)

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- lists

__global__ void k_plist_count(const int32_t *sel, int N, int E, int *cnt, int *rank) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= N) return;
    const int e = sel[a];
    rank[a] = (e >= 0 && e < E) ? atomicAdd(&cnt[e], 1) : -1;
}

__global__ void k_plist_offsets(const int *cnt, int E, int *offs) {
    if (threadIdx.x == 0) {
        int s = 0;
        for (int e = 0; e < E; ++e) {
            offs[e] = s;
            s += cnt[e];
        }
        offs[E] = s;
    }
}

__global__ void k_plist_scatter(const int32_t *sel, const int *rank, const int *offs, int N, int k, int *list_tok,
                                int *slot_of) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= N || rank[a] < 0) return;
    const int p = offs[sel[a]] + rank[a];
    list_tok[p] = a / k;
    slot_of[p] = a;
}

__global__ void k_fill_i32(int *p, int n, int v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// ---------------------------------------------------------------- quantize

// e such that m * 2^-e <= 448 (the largest e4m3 value), as small as possible.
__device__ __forceinline__ int fp8_block_exp(float m) {
    int km;
    const float fm = frexpf(m, &km);   // m = fm * 2^km, fm in [0.5, 1)
    return fm <= 0.875f ? km - 9 : km - 8;
}

// Rows of K f32 (row r of the input = in[(map ? map[r] : r) * K ...]) ->
// kTerms planes q[t][r][K] (e4m3) and sc[t][r][K / 32] (e8m0), one scale per
// 32-column block b (thread = (row, block)).
__global__ void __launch_bounds__(256)
k_quant_terms(const float *__restrict__ in, const int *__restrict__ map, int rows, int K,
              uint8_t *__restrict__ q, uint8_t *__restrict__ sc) {
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
        int e = m > 0.f ? fp8_block_exp(m) : -127;
        e = max(-127, min(127, e));
        const float inv = ldexpf(1.0f, -e), scl = ldexpf(1.0f, e);
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * j] * inv, v[4 * j + 1] * inv, 0, false);
            word = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * j + 2] * inv, v[4 * j + 3] * inv, word, true);
            w[j] = (uint32_t)word;
            // the term's values back in f32 (exact), and the residuals (exact)
            v[4 * j + 0] = v[4 * j + 0] - __builtin_amdgcn_cvt_f32_fp8(word, 0) * scl;
            v[4 * j + 1] = v[4 * j + 1] - __builtin_amdgcn_cvt_f32_fp8(word, 1) * scl;
            v[4 * j + 2] = v[4 * j + 2] - __builtin_amdgcn_cvt_f32_fp8(word, 2) * scl;
            v[4 * j + 3] = v[4 * j + 3] - __builtin_amdgcn_cvt_f32_fp8(word, 3) * scl;
        }
        uint8_t *qr = q + ((int64_t)t * rows + r) * K + 32 * b;
        *(uint4 *)qr = make_uint4(w[0], w[1], w[2], w[3]);
        *(uint4 *)(qr + 16) = make_uint4(w[4], w[5], w[6], w[7]);
        sc[((int64_t)t * rows + r) * nb + b] = (uint8_t)(e + 127);
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

// LDS of the GEMM block: two buffers of one K step's B operands for every
// (term, token tile, half, lane) as 16-byte pieces, their scales, and one
// 32 x 33 transpose tile per wave.
constexpr int kBPieces = kTerms * kNT * 2 * 64;              // 16-byte pieces per K step
constexpr int kBScales = kTerms * kNT * 64;                  // scale bytes per K step
constexpr int kPiecesPerThread = kBPieces / (64 * kWaves);   // 6
constexpr int kScalesPerThread = (kBScales + 64 * kWaves - 1) / (64 * kWaves);
constexpr size_t kGemmLds = 2 * (size_t)kBPieces * 16 + 2 * (size_t)kBScales + sizeof(float) * kWaves * 32 * 33;
static_assert(kBPieces % (64 * kWaves) == 0, "B pieces must split evenly over the block");

// MODE 0: gate/up (K = H, rows = F, B rows = tokens through list_tok);
// MODE 1: down (K = F, rows = H, B rows = list positions).
// Block = (expert, 4 row tiles of 32), one wave per row tile; the expert's
// tokens in passes of up to kNT 32-token tiles. Per K step the block stages
// B (all terms and tiles) in LDS, double-buffered: step s+1 is loaded from
// memory while step s's MFMAs run; each wave keeps its A (weight) chunks two
// steps ahead in registers.
template <int MODE>
__global__ void __launch_bounds__(64 * kWaves) k_moe_gemm(GemmArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t glds[];
    mh_u4 *bbuf = (mh_u4 *)glds;                                    // [2][kBPieces]
    uint8_t *sbuf = glds + 2 * (size_t)kBPieces * 16;                // [2][kBScales]
    float(*tiles)[32][33] = (float(*)[32][33])(sbuf + 2 * kBScales);
    const int K = MODE == 0 ? A.H : A.F;
    const int R = MODE == 0 ? A.F : A.H;
    const int RT = R / 32;
    const int groups = (RT + kWaves - 1) / kWaves;
    const int e = blockIdx.x / groups, rgrp = blockIdx.x - e * groups;
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
    const uint16_t *s0 = (const uint16_t *)(ex + A.off[MODE == 0 ? 1 : 7]) + (size_t)row * nsc;
    const uint8_t *a1 = ex + A.off[3] + (size_t)row * rowbytes;
    const uint16_t *s1 = (const uint16_t *)(ex + A.off[4]) + (size_t)row * nsc;
    unsigned bad = 0;
    float(*tl)[33] = tiles[wave];
    for (int p0 = 0; p0 < T; p0 += 32 * kNT) {
        const int nt = min(kNT, (T - p0 + 31) / 32);
        // this thread's B pieces: q = tid + 256 i -> (term, tile, half, lane)
        const uint8_t *bsrc[kPiecesPerThread];
#pragma unroll
        for (int i = 0; i < kPiecesPerThread; ++i) {
            const int q = tid + 64 * kWaves * i;
            const int lane = q & 63, half = (q >> 6) & 1, j = (q >> 7) % kNT, t = q / (128 * kNT);
            const int p = p0 + 32 * j + (lane & 31);
            int br = -1;
            if (j < nt && p < T) br = MODE == 0 ? A.list_tok[base + p] : base + p;
            bsrc[i] = br < 0 ? nullptr
                             : A.bq + ((size_t)t * A.b_rows + br) * K + 16 * (lane >> 5) + 32 * half;
        }
        const uint8_t *ssrc[kScalesPerThread];
#pragma unroll
        for (int i = 0; i < kScalesPerThread; ++i) {
            const int q = tid + 64 * kWaves * i;
            ssrc[i] = nullptr;
            if (q < kBScales) {
                const int lane = q & 63, j = (q >> 6) % kNT, t = q / (64 * kNT);
                const int p = p0 + 32 * j + (lane & 31);
                if (j < nt && p < T) {
                    const int br = MODE == 0 ? A.list_tok[base + p] : base + p;
                    ssrc[i] = A.bs + ((size_t)t * A.b_rows + br) * nsc + (lane >> 5);
                }
            }
        }
        v16f acc0[kNT], acc1[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            acc0[j] = v16f{};
            acc1[j] = v16f{};
        }
        // stage step 0
        {
            mh_u4 rb[kPiecesPerThread];
            uint32_t rs[kScalesPerThread];
#pragma unroll
            for (int i = 0; i < kPiecesPerThread; ++i)
                rb[i] = bsrc[i] ? *(const mh_u4 *)bsrc[i] : mh_u4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < kScalesPerThread; ++i) rs[i] = ssrc[i] ? *ssrc[i] : 0u;
#pragma unroll
            for (int i = 0; i < kPiecesPerThread; ++i) bbuf[tid + 64 * kWaves * i] = rb[i];
#pragma unroll
            for (int i = 0; i < kScalesPerThread; ++i)
                if (tid + 64 * kWaves * i < kBScales) sbuf[tid + 64 * kWaves * i] = (uint8_t)rs[i];
        }
        // A for steps 0 and 1
        mh_u4 wa0[3], wa1[3];
        uint32_t ws0[3], ws1[3];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = 2 * min(u, steps - 1) + g;
            wa0[u] = mh_load16(mh_global(a0 + c * 16));
            ws0[u] = mh_load_u16(mh_global(s0 + c));
            if constexpr (MODE == 0) {
                wa1[u] = mh_load16(mh_global(a1 + c * 16));
                ws1[u] = mh_load_u16(mh_global(s1 + c));
            }
        }
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            const int cur = s & 1;
            // memory for step s+1 (B pieces, into registers) and step s+2 (A)
            mh_u4 rb[kPiecesPerThread];
            uint32_t rs[kScalesPerThread];
            const bool more = s + 1 < steps;
#pragma unroll
            for (int i = 0; i < kPiecesPerThread; ++i)
                rb[i] = (more && bsrc[i]) ? *(const mh_u4 *)(bsrc[i] + 64 * (s + 1)) : mh_u4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < kScalesPerThread; ++i) rs[i] = (more && ssrc[i]) ? ssrc[i][2 * (s + 1)] : 0u;
            {
                const int c = 2 * min(s + 2, steps - 1) + g;
                wa0[(s + 2) % 3] = mh_load16(mh_global(a0 + c * 16));
                ws0[(s + 2) % 3] = mh_load_u16(mh_global(s0 + c));
                if constexpr (MODE == 0) {
                    wa1[(s + 2) % 3] = mh_load16(mh_global(a1 + c * 16));
                    ws1[(s + 2) % 3] = mh_load_u16(mh_global(s1 + c));
                }
            }
            if (wact) {
                const int u = s % 3;
                v8i qa0 = {}, qa1 = {};
                qa0[0] = (int)wa0[u].x; qa0[1] = (int)wa0[u].y; qa0[2] = (int)wa0[u].z; qa0[3] = (int)wa0[u].w;
                const int sa0 = e8m0_of_f16(ws0[u], &bad);
                int sa1 = 127;
                if constexpr (MODE == 0) {
                    qa1[0] = (int)wa1[u].x; qa1[1] = (int)wa1[u].y; qa1[2] = (int)wa1[u].z; qa1[3] = (int)wa1[u].w;
                    sa1 = e8m0_of_f16(ws1[u], &bad);
                }
                const mh_u4 *bb = bbuf + (size_t)cur * kBPieces;
                const uint8_t *sb8 = sbuf + (size_t)cur * kBScales;
#pragma unroll
                for (int t = 0; t < kTerms; ++t) {
#pragma unroll
                    for (int j = 0; j < kNT; ++j) {
                        if (j >= nt) break;
                        const mh_u4 lo = bb[((t * kNT + j) * 2 + 0) * 64 + l];
                        const mh_u4 hi = bb[((t * kNT + j) * 2 + 1) * 64 + l];
                        const v8i qb = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                        (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                        const int sbv = sb8[(t * kNT + j) * 64 + l];
                        acc0[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa0, qb, acc0[j], 4, 0, 0, sa0, 0, sbv);
                        if constexpr (MODE == 0)
                            acc1[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa1, qb, acc1[j], 4, 0, 0, sa1, 0, sbv);
                    }
                }
            }
            if (more) {
                mh_u4 *nb = bbuf + (size_t)(cur ^ 1) * kBPieces;
#pragma unroll
                for (int i = 0; i < kPiecesPerThread; ++i) nb[tid + 64 * kWaves * i] = rb[i];
                uint8_t *ns = sbuf + (size_t)(cur ^ 1) * kBScales;
#pragma unroll
                for (int i = 0; i < kScalesPerThread; ++i)
                    if (tid + 64 * kWaves * i < kBScales) ns[tid + 64 * kWaves * i] = (uint8_t)rs[i];
            }
            __syncthreads();
        }
        if (wact) {
            // epilogue through the wave's LDS tile: lane (m, g) owns column m
            // (token p0 + 32 j + m) and rows 8 (i / 4) + 4 g + i % 4; after the
            // transpose lane l writes row 32 rt + m of tokens 2 q + g
#pragma unroll
            for (int j = 0; j < kNT; ++j) {
                if (j >= nt) break;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rr = 8 * (i / 4) + 4 * g + (i % 4);
                    const size_t grow4 = (size_t)(rt * 32 + rr) * 4;
                    float v;
                    if constexpr (MODE == 0) {
                        float gg = acc0[j][i] + *(const float *)(ex + A.off[2] + grow4);
                        float uu = acc1[j][i] + *(const float *)(ex + A.off[5] + grow4);
                        if (A.act_plain) {
                            v = gg / (1.0f + expf(-gg)) * uu;
                        } else {
                            if (gg > A.limit) gg = A.limit;
                            if (uu > A.limit) uu = A.limit;
                            if (uu < -A.limit) uu = -A.limit;
                            v = gg / (1.0f + expf(-A.alpha * gg)) * (uu + 1.0f);
                        }
                    } else {
                        v = acc0[j][i] + *(const float *)(ex + A.off[8] + grow4);
                    }
                    tl[m][rr] = v;   // [token][row]
                }
                __builtin_amdgcn_wave_barrier();
                for (int q = 0; q < 16; ++q) {
                    const int tok = 2 * q + g, p = p0 + 32 * j + tok;
                    if (p < T) {
                        const float v = tl[tok][m];
                        if constexpr (MODE == 0) A.hbuf[(size_t)(base + p) * A.F + rt * 32 + m] = v;
                        else A.ye[(size_t)A.slot_of[base + p] * A.H + rt * 32 + m] = v;
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    if (bad) atomicOr(A.err, 1u);
}

unsigned *g_scale_err = nullptr;       // host-mapped flag
unsigned *g_scale_err_dev = nullptr;

}  // namespace

// True when the scaled-MFMA path handles this layer (MXFP4 experts, shapes
// that tile by 64 along K and 32 along rows).
bool prefill_mfma_ok(const DevLayer &L) {
    const char *off = getenv("MIDGE_HIP_NO_MFMA");
    if (off && off[0] && off[0] != '0') return false;
    return L.expert_dt == MH_DT_MXFP4 && L.hidden % 64 == 0 && L.ffn % 64 == 0 && L.top_k >= 1 &&
           L.n_experts <= 65535;
}

// Expert-major MoE of n tokens: x[t] += sum over t's slots, in ascending
// expert order, of w * expert(xb[t]); ye is [n * k][H] scratch read by the
// prefill combine (launched by the caller).
int run_expert_major_mfma(const DevLayer &L, int n, const float *xb, const int32_t *sel, float *ye,
                          hipStream_t s) {
    const int k = L.top_k, E = L.n_experts, N = n * k;
    const int H = (int)L.hidden, F = (int)L.ffn;
    static bool lds_set = false;
    if (!lds_set) {
        MH_HIP(hipFuncSetAttribute((const void *)k_moe_gemm<0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds));
        MH_HIP(hipFuncSetAttribute((const void *)k_moe_gemm<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds));
        lds_set = true;
    }
    if (!g_scale_err) {
        MH_HIP(hipHostMalloc((void **)&g_scale_err, sizeof(unsigned), hipHostMallocMapped));
        *g_scale_err = 0;
        MH_HIP(hipHostGetDevicePointer((void **)&g_scale_err_dev, g_scale_err, 0));
        watch_async_error(g_scale_err, "prefill: an MXFP4 scale is not a positive power of two (e8m0 cannot hold it)");
    }
    // lists: cnt[E], offs[E + 1], rank[N], list_tok[N], slot_of[N]
    void *pl;
    MH_TRY(scratch(S_LIST, sizeof(int) * ((size_t)2 * E + 1 + 3 * (size_t)N), &pl));
    int *cnt = (int *)pl, *offs = cnt + E, *rank = offs + E + 1, *list_tok = rank + N, *slot_of = list_tok + N;
    // quantized activations: the larger of x (n rows of H) and h (N rows of F)
    const size_t qx = (size_t)kTerms * n * H, qh = (size_t)kTerms * N * F;
    const size_t qbytes = std::max(qx + qx / 32, qh + qh / 32);
    void *pq, *ph;
    MH_TRY(scratch(S_Q, qbytes, &pq));
    MH_TRY(scratch(S_H, sizeof(float) * (size_t)N * F, &ph));
    uint8_t *q = (uint8_t *)pq;
    float *hbuf = (float *)ph;

    MH_LAUNCH("plist", k_fill_i32, dim3(1), dim3(256), 0, s, cnt, E, 0);
    MH_LAUNCH("plist", k_plist_count, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, s, sel, N, E, cnt, rank);
    MH_LAUNCH("plist", k_plist_offsets, dim3(1), dim3(64), 0, s, cnt, E, offs);
    MH_LAUNCH("plist", k_plist_scatter, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, s, sel, rank, offs, N, k,
              list_tok, slot_of);
    // ye rows of unfilled slots stay zero (a fill kernel: callers may capture this in a graph)
    MH_LAUNCH("plist", k_fill_i32, dim3(1024), dim3(256), 0, s, (int *)ye, N * H, 0);

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
    A.err = g_scale_err_dev;

    // gate/up over the quantized tokens
    {
        const int64_t thr = (int64_t)n * (H / 32);
        A.bq = q;
        A.bs = q + (size_t)kTerms * n * H;
        A.b_rows = n;
        MH_LAUNCH("quant_x", k_quant_terms, dim3((unsigned)((thr + 255) / 256)), dim3(256), 0, s, xb, nullptr, n, H,
                  q, q + (size_t)kTerms * n * H);
        const int groups = (F / 32 + kWaves - 1) / kWaves;
        MH_LAUNCH("moe_gu_mfma", k_moe_gemm<0>, dim3((unsigned)(E * groups)), dim3(64 * kWaves), kGemmLds, s, A);
    }
    // down over the quantized h (list order)
    {
        const int64_t thr = (int64_t)N * (F / 32);
        A.bq = q;
        A.bs = q + (size_t)kTerms * N * F;
        A.b_rows = N;
        MH_LAUNCH("quant_h", k_quant_terms, dim3((unsigned)((thr + 255) / 256)), dim3(256), 0, s, hbuf, nullptr, N,
                  F, q, q + (size_t)kTerms * N * F);
        const int groups = (H / 32 + kWaves - 1) / kWaves;
        MH_LAUNCH("moe_down_mfma", k_moe_gemm<1>, dim3((unsigned)(E * groups)), dim3(64 * kWaves), kGemmLds, s, A);
    }
    return hip_check(hipGetLastError(), "prefill MFMA launches");
}

}  // namespace mh
