// mh_decode.hip — a whole MoE decode step (every layer of a stack, batch 1)
// in one cooperative launch: the MoE half of forward()'s layer loop
// (engine/midge.c:557-560) with moe() (engine/midge.c:469-549) per layer.
//
// One block per CU, 512 threads. Per layer:
//   A  router     every block reads x (the previous layer's output, as
//                 sequence-tagged words), forms xb = rmsnorm(x) * w in LDS;
//                 the router's rows are spread over the blocks and each
//                 logit is published as a tagged word.
//   route         every block gathers the tagged logits (from one of
//                 kLR copies, so that few blocks poll each line) and ranks
//                 them (stable top-k, ties to the lower index) itself: all
//                 reach the same selection and weights, with no broadcast.
//   B  gate/up    each block takes an even share of the routed experts'
//                 (gate, up) row pairs, with the bias + clamped SwiGLU
//                 epilogue -> h[k][ffn]; then a grid barrier.
//   C  down       each block owns a slice of output rows for all k experts.
//                 MXFP4 stacks: the rows are loaded during the barrier,
//                 staged in LDS and multiplied on the matrix cores (f16 MFMA
//                 over h split into two f16 terms); otherwise they are
//                 loaded into registers between the barrier's arrive and wait
//                 and multiplied on the vector ALUs. Epilogue: y = Wd h + bd,
//                 moe = sum_i w_i y_i in selection order, x += moe, written
//                 as tagged words for the next layer (plain floats after the
//                 last layer).
// Tagged words carry the producer's sequence number next to the value in one
// 64-bit store, so a consumer needs no separate barrier: it polls the words
// it needs until every tag matches. The one full barrier per layer (before
// the down phase, which needs all of h) is a gather/broadcast over per-block
// flags (measured faster than every block polling every flag). Every wait is
// bounded: one that does not complete within ~1 s raises an error flag and
// every block exits.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <vector>

#include "mh_gemv.cuh"

namespace mh {

struct StepLayer {
    const uint8_t *experts;
    const uint8_t *router_w;
    const float *router_s;   // q8r row scales (unused for an f32 router)
    const float *router_b;
    const float *norm_w;
};

struct StepArgs {
    const StepLayer *layers;
    int n_layers, H, F, E, K;
    int CH, CF;              // 16-byte chunks per expert row: H / 32, F / 32
    uint64_t stride;
    uint64_t off[9];
    float alpha, limit, eps;
    int act_plain, router_norm;
    float *x;                // [H], in place
    int32_t *sel;            // [L][K] or null
    float *w;                // [L][K] or null
    uint32_t *usage;         // [L][E] or null
    uint64_t *lw;            // [kLR][lws] tagged logits: kLR copies, lws words apart
    int lws;
    uint64_t *xw;            // [H] tagged x between layers
    float *h;                // [K][F] scratch (VALU path)
    uint16_t *h16;           // [2][K][Fpad] f16 planes of h (MFMA path)
    int Fpad;                // ffn rounded up to 128
    unsigned *flags;         // [gridDim.x] barrier flags
    unsigned *go;            // barrier release word (written by block 0)
    unsigned seq0;           // first sequence number of this launch (3 per layer)
    unsigned *err;
    unsigned long long *trace;   // [L][kStamps][gridDim.x] per-block phase timestamps, or null
    int res_floats;              // LDS floats of the reduced-rows area
    int red_floats;              // LDS floats of the partial-sum area
};

namespace {

constexpr int kThreads = 512;   // 8 waves: 2 per SIMD, up to 256 VGPRs each
constexpr int kUP = 9;          // gate/up row pairs in flight per thread
constexpr int kUC = 12;         // down rows in flight per thread
constexpr int kNX = 8;          // x elements per thread in the router phase (H <= kNX * kThreads)
constexpr unsigned kSpinLimit = 1u << 20;
constexpr int kStamps = 24;     // phase timestamps per layer and block while profiling
constexpr int kEL = 2;          // logits per lane in the routing wave (E <= 64 * kEL)
constexpr int kLR = 8;          // copies of the logits (each polled by NB / kLR blocks)
constexpr int kGoCopies = 8;    // copies of the barrier's release word
constexpr int kGoStride = 64;   // words between them (256 B)
// static LDS capacities of the one-launch step (plan creation checks a
// stack against them)
constexpr int kHMax = 3072;         // hidden size
constexpr int kResMax = 1024;       // floats of reduced rows
constexpr int kRedMax = 8192;       // floats of partial sums

// Memory access. Every load goes through a buffer resource (32-bit offsets,
// out-of-range reads return 0). Weights are streamed with the nontemporal
// hint. Data that blocks exchange inside the launch (x, logits, h) is
// written with device-scope stores and read with device-scope loads, which
// are coherent across the XCDs' L2 caches: the barriers then need no L2
// write-back or invalidate, and read-only weights stay cached.
constexpr int kNT = 2;     // cache-policy bits: nontemporal
constexpr int kDev = 16;   // cache-policy bits: device scope
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Every resource here is uniform across the block; the pointer fields read
// from the layer table are made scalar explicitly (readfirstlane), otherwise
// the compiler keeps them in vector registers and wraps every buffer access
// in a loop over the distinct values.
__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void *u = (void *)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ mh_u4 ld_w16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
}
__device__ __forceinline__ uint32_t ld_w2(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kNT);
}
__device__ __forceinline__ float ld_f(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float ld_dev(rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kDev));
}
__device__ __forceinline__ mh_u4 ld_dev16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kDev);
}
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// An opaque copy of v: values derived from it are recomputed where they are
// used instead of being hoisted out of the layer loop and held in registers
// (or spilled) across every phase.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Arrive: every wave's stores have completed (device-scope stores complete
// at the device coherence point), then thread 0 publishes `seq`.
__device__ __forceinline__ void bar_arrive(unsigned *flags, unsigned seq) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(&flags[blockIdx.x], seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gather/broadcast wait: block 0's first wave polls every block's flag (one
// load per lane per round) and then publishes `seq` in the kGoCopies copies
// of the release word; every other block polls copy b % kGoCopies (one word
// polled by every block congests its line). Returns false (in every thread) if the
// barrier timed out. Loads after the wait are issued only once it has
// returned, so device-scope loads see every store made before the arrives.
__device__ __forceinline__ bool bar_wait(const unsigned *flags, unsigned *go, unsigned seq, unsigned *err,
                                         int *s_ok) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        unsigned spins = 0;
        bool ok = true;
        if (blockIdx.x == 0) {
            const int nb = gridDim.x;
            for (;;) {
                bool done = true;
                for (int i = lane; i < nb; i += 64) {
                    unsigned f = __hip_atomic_load(&flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((int)(f - seq) < 0) done = false;
                }
                if (__all(done)) break;
                if (++spins > kSpinLimit) {
                    ok = false;
                    break;
                }
            }
            if (ok && lane < kGoCopies)
                __hip_atomic_store(go + lane * kGoStride, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (lane == 0) {
            const unsigned *g = go + (blockIdx.x % kGoCopies) * kGoStride;
            while ((int)(__hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - seq) < 0) {
                __builtin_amdgcn_s_sleep(1);
                if (++spins > kSpinLimit) {
                    ok = false;
                    break;
                }
            }
        }
        if (lane == 0) {
            *s_ok = ok ? 1 : 0;
            if (!ok) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    __syncthreads();
    return *s_ok != 0;
}

// Sum over the block (all threads get it). `part` is LDS [16].
__device__ __forceinline__ float block_sum(float v, float *part) {
    v = mh_wave_sum(v);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) s += part[i];
    __syncthreads();
    return s;
}

// Tagged words: (tag << 32) | value bits in one device-scope 64-bit store.
__device__ __forceinline__ void st_tag(uint64_t *p, unsigned tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Maximum over the wave (every lane gets it): DPP within rows of 16, then
// row broadcasts; lanes a DPP step does not write keep their value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return fmaxf(v, __int_as_float(o));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v);   // row_mirror
    v = dpp_max_step<0x142, 0xA>(v);   // row_bcast:15
    v = dpp_max_step<0x143, 0xC>(v);   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the wave with DPP (the result is valid in lane 63): within rows
// of 16, then the row broadcasts; rows a step does not write add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add_step(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add_step<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_add_step<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_add_step<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_add_step<0x140, 0xF>(v);   // row_mirror
    v = dpp_add_step<0x142, 0xA>(v);   // row_bcast:15
    v = dpp_add_step<0x143, 0xC>(v);   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Stable top-k over the wave's E <= 64 * kEL logits (lane holds element
// lane + 64 j in v[j]; absent elements are -inf): k rounds of "largest
// remaining value, lowest index among equals"; only values > -1e30
// qualify, unfilled slots get -1 (engine/midge.c:476-486). Lane i < k ends
// with slot i's expert in *sel and its logit in *val (-1e30 if unfilled).
__device__ __forceinline__ void wave_topk(float *v, int k, int *sel, float *val) {
    const int lane = threadIdx.x & 63;
    *sel = -1;
    *val = -1e30f;
    for (int i = 0; i < k; ++i) {
        float lm = -INFINITY;
#pragma unroll
        for (int j = 0; j < kEL; ++j) lm = fmaxf(lm, v[j]);
        const float m = wave_max(lm);
        int idx = -1;
        if (m > -1e30f) {
#pragma unroll
            for (int j = kEL - 1; j >= 0; --j) {
                const unsigned long long hit = __ballot(v[j] == m);
                if (hit) idx = 64 * j + (__ffsll((long long)hit) - 1);
            }
        }
        if (idx >= 0 && (idx & 63) == lane) {
#pragma unroll
            for (int j = 0; j < kEL; ++j)
                if (j == (idx >> 6)) v[j] = -INFINITY;   // taken
        }
        if (lane == i) {
            *sel = idx;
            *val = idx >= 0 ? m : -1e30f;
        }
    }
}

// Routing weight of slot `lane` (engine/midge.c:502-512), by one wave from
// wave_topk's per-lane results: softmax over the k selected logits
// (router_norm; the denominator summed in slot order) or the slot's entry of
// the softmax over all E logits (v: kEL per lane, -inf past E).
__device__ __forceinline__ float wave_weight(const float *v, int k, int router_norm, float val) {
    if (router_norm) {
        const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), 0));
        const float ex = expf(val - mx);
        float den = 0.f;
        for (int i = 0; i < k; ++i) den += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), i));
        return ex / den;
    }
    float lm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kEL; ++j) lm = fmaxf(lm, v[j]);
    const float m = wave_max(lm);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < kEL; ++j) sum += v[j] > -INFINITY ? expf(v[j] - m) : 0.f;
    return expf(val - m) / wave_sum_dpp(sum);
}

__device__ __forceinline__ float act_fn(float g, float u, float alpha, float limit, int plain) {
    if (plain) return g / (1.0f + expf(-g)) * u;
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    if (u < -limit) u = -limit;
    const float a = g / (1.0f + expf(-alpha * g));
    return a * (u + 1.0f);
}

// Phase A's inputs that do not depend on x, loaded ahead of time (for layer
// 0 at kernel start, for layer l + 1 after layer l's output): the elements
// of this block's router row that this thread's x elements meet (as raw
// bits: int8 or f32), that row's scale and bias, and the norm weights of
// this thread's x elements.
struct RouterPref {
    uint32_t rw[kNX];
    float rs, rb;
    float nw[kNX];
};

template <int RDT>
__device__ __forceinline__ RouterPref prefetch_router(const StepArgs &A, int l) {
    RouterPref p;
    const StepLayer Lp = A.layers[l];
    const int b = blockIdx.x, t = threadIdx.x, H = A.H;
    const int e = b < A.E ? b : 0;
    constexpr uint32_t wb = RDT == MH_DT_Q8R ? 1u : 4u;   // bytes per router weight
    const rsrc_t rw = make_rsrc(Lp.router_w, (uint32_t)A.E * (uint32_t)H * wb);
#pragma unroll
    for (int k = 0; k < kNX; ++k) {   // past H: the next row's weights (or 0), met by x = 0
        const uint32_t o = ((uint32_t)e * (uint32_t)H + (uint32_t)(t + k * kThreads)) * wb;
        if constexpr (RDT == MH_DT_Q8R) p.rw[k] = __builtin_amdgcn_raw_buffer_load_b8(rw, o, 0, 0);
        else p.rw[k] = __builtin_amdgcn_raw_buffer_load_b32(rw, o, 0, 0);
    }
    p.rs = 1.0f;
    if constexpr (RDT == MH_DT_Q8R) p.rs = ld_f(make_rsrc(Lp.router_s, (uint32_t)A.E * 4u), (uint32_t)e * 4u);
    p.rb = ld_f(make_rsrc(Lp.router_b, (uint32_t)A.E * 4u), (uint32_t)e * 4u);
    const rsrc_t rn = make_rsrc(Lp.norm_w, (uint32_t)H * 4u);
#pragma unroll
    for (int k = 0; k < kNX; ++k) p.nw[k] = ld_f(rn, (uint32_t)(t + k * kThreads) * 4u);   // 0 past H
    return p;
}

template <int RDT>
__device__ __forceinline__ float router_weight(uint32_t bits) {
    if constexpr (RDT == MH_DT_Q8R) return (float)(int8_t)(uint8_t)bits;
    else return __uint_as_float(bits);
}

// Two sums over the block at once (all threads get them). `part` is LDS [16].
__device__ __forceinline__ float2 block_sum2(float a, float c, float *part) {
    a = wave_sum_dpp(a);
    c = wave_sum_dpp(c);
    if ((threadIdx.x & 63) == 0) {
        part[2 * (threadIdx.x >> 6)] = a;
        part[2 * (threadIdx.x >> 6) + 1] = c;
    }
    __syncthreads();
    float sa = 0.f, sc = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) {
        sa += part[2 * i];
        sc += part[2 * i + 1];
    }
    __syncthreads();
    return make_float2(sa, sc);
}

// ---------------------------------------------------------------- MFMA
// The down projection of an MXFP4 stack runs on V_MFMA_F32_16X16X32_F16
// (measured layout on gfx950: lane l holds A row l % 16 and B column l % 16,
// 8 consecutive K values 8 (l / 16) .. +7 each; output lane l holds column
// l % 16 of rows 4 (l / 16) + i).
//   A  16 of the block's down rows (rows of different routed experts may
//      share a tile), e2m1 converted to f16 with the chunk's power-of-two
//      scale, which is exact (the plan scans every scale)
//   B  h split into two f16 terms (hi = h rounded, lo = h - hi rounded:
//      within 2^-22 |h|), written by the producing block as two planes;
//      column 2 i + term holds routed slot i's term, so a B operand is one
//      16-byte load and row rho's dot product is columns 2 i + 0, 2 i + 1 of
//      its slot i summed
// A K step of 128 = 4 lane groups x 32 takes one 16-byte MXFP4 chunk per
// lane group: lane (m, g) converts dword j of its chunk for the step's j-th
// MFMA, and B lane (n, g) supplies elements 8 j .. 8 j + 7 of the same chunk.
// The weights cannot be loaded in this lane layout directly (16 rows x 64 B
// per instruction streams from HBM ~25% slower than whole rows), so they are
// loaded as whole rows and staged through LDS.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kQ = 3;                  // 128-column K steps per wave (ffn <= 8 * kQ * 128)
constexpr int kKPad = 8 * kQ * 128;    // largest padded ffn
constexpr int kRTC = 3;                // down row tiles (k * rows per block <= 48)
constexpr int kSD = kKPad / 32 + 1;    // LDS row stride (chunks) of the staged down rows

__device__ __forceinline__ v8h fp4x8_f16(uint32_t w, float s) {
    const v2h a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0);
    const v2h b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1);
    const v2h c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2);
    const v2h d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3);
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ uint32_t dword_of(const mh_u4 &q, int j) {
    return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}
// v of lane + K within the lane's row of 16 (0 past the row's end)
template <int K>
__device__ __forceinline__ float dpp_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + K, 0xF, 0xF, false));
}
__device__ __forceinline__ void st_dev16(rsrc_t r, uint32_t off, uint16_t v) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kDev);
}

// The down rows [0, rows) of the block's slice (row rho = i * RC + j: slot i,
// row j), staged in LDS at a stride of SD chunks, times h's two f16 planes
// (hb: this lane's B operands, loaded by the caller), NT = ceil(rows / 16)
// row tiles; row rho's partial (columns 2 i, 2 i + 1 summed) goes to
// red[w * 48 + rho].
template <int NT>
__device__ __forceinline__ void dn_mfma_t(const uint8_t *sw, const uint16_t *ss, const v8h (*hb)[4], int SD, int CF,
                                          int rows, int RC, float *red) {
    const int tt = opaque(threadIdx.x);
    const int lane = tt & 63, m = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tt >> 6);
    const int NQC = (CF + 3) >> 2;
    v4f acc[NT];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) acc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kQ; ++u) {
        const int q = kQ * wv + u;
        if (q >= NQC) break;
        const int c = min(4 * q + g, CF - 1);   // past F: B is zero
        mh_u4 qa[NT];
        float sc[NT];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            const int o = min(16 * rt + m, rows - 1) * SD + c;
            qa[rt] = *(const mh_u4 *)(sw + (size_t)o * 16);
            sc[rt] = mh_f16(ss[o]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp4x8_f16(dword_of(qa[rt], j), sc[rt]), hb[u][j], acc[rt],
                                                                 0, 0, 0);
    }
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const float v = acc[rt][ii];
            const float v1 = dpp_shl<1>(v);
            const int rho = 16 * rt + 4 * g + ii;
            if (rho < rows && m == 2 * (rho / RC)) red[wv * 48 + rho] = v + v1;
        }
    }
}

template <int RDT, int XDT, bool MF>
__global__ void __launch_bounds__(kThreads) k_decode_step(StepArgs A) {
    constexpr int XE = mh_chunk<XDT>::E;   // elements per expert chunk (32)
    constexpr int RE = mh_chunk<RDT>::E;   // elements per router chunk (16 int8 / 4 f32)
    // LDS is static (capacities are checked at plan creation).
    __shared__ float s_part[16];
    __shared__ int s_sel[16];
    __shared__ float s_w[16];
    __shared__ int s_ok;
    __shared__ __attribute__((aligned(16))) float s_xs[kHMax];       // x at layer start
    // xb = rmsnorm(x) * w in 32-element groups padded to 33 floats: thread c
    // reads group c element by element, and the padding puts the 64 lanes of
    // a wave in 64 distinct LDS banks
    __shared__ __attribute__((aligned(16))) float s_xbs[kHMax / 32 * 33];
    __shared__ __attribute__((aligned(16))) float s_res[kResMax];    // reduced rows / staged logits
    __shared__ __attribute__((aligned(16))) float s_red[kRedMax];    // partial sums
    __shared__ __attribute__((aligned(16))) float s_bds[kThreads];   // [K][rows of this block's down slice]
    // MFMA path: the block's down rows ([16 kRTC rows][kSD chunks]) and scales
    __shared__ __attribute__((aligned(16))) uint8_t s_dw[MF ? 16 * kRTC * kSD * 16 : 16];
    __shared__ uint16_t s_ds[MF ? 16 * kRTC * kSD : 2];
    const int H = A.H, F = A.F, E = A.E, K = A.K;
    float *xs = s_xs, *xbs = s_xbs, *res = s_res, *red = s_red, *bds = s_bds;
    const int NB = gridDim.x, b = blockIdx.x, t = threadIdx.x;
    const int wave = t >> 6;

    // per-block phase timestamps (100 MHz), written by thread 0 while profiling
    unsigned long long *tr = (A.trace && t == 0) ? A.trace + b : nullptr;
#define MH_STAMP(ph) \
    if (tr) tr[(size_t)(l * kStamps + (ph)) * NB] = wall_clock64()

    const rsrc_t rx = make_rsrc(A.x, (uint32_t)H * 4u);
    const rsrc_t rh = make_rsrc(A.h, (uint32_t)K * (uint32_t)F * 4u);
    const uint32_t layer_bytes = (uint32_t)((uint64_t)E * A.stride - 1u) + 1u;   // < 4 GiB (plan check)
    const int CR = H / RE;   // router chunks per row
    RouterPref pf = prefetch_router<RDT>(A, 0);
    const rsrc_t rh16 = make_rsrc(A.h16, (uint32_t)(2 * K * A.Fpad) * 2u);
    for (int l = 0; l < A.n_layers; ++l) {
        const StepLayer Ly = A.layers[l];
        // sequence numbers of this layer: logits and routing record, the
        // barrier before the down phase, x for the next layer
        const unsigned tagA = A.seq0 + 3u * (unsigned)l, tagB = tagA + 1u, tagC = tagA + 2u;
        MH_STAMP(0);
        // ------------------------------------------------ A: router
        {
            float xv[kNX];
            if (l == 0) {
#pragma unroll
                for (int k = 0; k < kNX; ++k) xv[k] = ld_dev(rx, (uint32_t)(t + k * kThreads) * 4u);   // 0 past H
            } else {
                // the previous layer's x, tagged tagA - 1: load all, re-poll the late ones
                uint64_t wv[kNX];
                const unsigned want = tagA - 1u;
                const int tt = opaque(t);
#pragma unroll
                for (int k = 0; k < kNX; ++k) {
                    const int i = tt + k * kThreads;
                    wv[k] = i < H ? ld_tag(A.xw + i) : (uint64_t)want << 32;
                }
                bool late = false;
                for (unsigned spins = 0;; ++spins) {
                    bool ready = true;
#pragma unroll
                    for (int k = 0; k < kNX; ++k) ready = ready && (unsigned)(wv[k] >> 32) == want;
                    if (ready) break;
                    if (spins > kSpinLimit) {
                        late = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int k = 0; k < kNX; ++k) {
                        const int i = tt + k * kThreads;
                        if (i < H && (unsigned)(wv[k] >> 32) != want) wv[k] = ld_tag(A.xw + i);
                    }
                }
                if (__syncthreads_or(late)) {
                    if (t == 0) __hip_atomic_store(A.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    return;
                }
#pragma unroll
                for (int k = 0; k < kNX; ++k) xv[k] = __uint_as_float((uint32_t)wv[k]);
            }
            MH_STAMP(15);
            // the sum of squares and this block's logit in one pass: the
            // row's dot with xb = x * inv * w is inv * (row . (x * w))
            float ss = 0.f, dp = 0.f;
#pragma unroll
            for (int k = 0; k < kNX; ++k) {
                ss = __builtin_fmaf(xv[k], xv[k], ss);
                dp = __builtin_fmaf(router_weight<RDT>(pf.rw[k]), xv[k] * pf.nw[k], dp);
            }
            const float2 sums = block_sum2(ss, dp, s_part);
            const float inv = 1.0f / sqrtf(sums.x / (float)H + A.eps);
            if (b < E && t < kLR) {   // one copy per logit replica
                float p = sums.y * inv;
                if constexpr (RDT == MH_DT_Q8R) p *= pf.rs;
                st_tag(A.lw + (size_t)t * A.lws + b, tagA, p + pf.rb);
            }
#pragma unroll
            for (int k = 0; k < kNX; ++k) {
                const int i = t + k * kThreads;
                if (i < H) {
                    xs[i] = xv[k];
                    xbs[(i >> 5) * 33 + (i & 31)] = xv[k] * inv * pf.nw[k];
                }
            }
        }
        __syncthreads();
        // router rows beyond the grid (more experts than blocks): over xb
        for (int e = b + NB; e < E; e += NB) {
            float p = 0.f;
            const rsrc_t rw = make_rsrc(Ly.router_w, (uint32_t)E * (uint32_t)CR * 16u);
            for (int c = t; c < CR; c += kThreads) {
                const mh_u4 q = ld_w16(rw, (uint32_t)(e * CR + c) * 16u);
                const int i0 = c * RE;   // a router chunk lies inside one 32-element group
                p += mh_dot_chunk<RDT>(q, xbs + (i0 >> 5) * 33 + (i0 & 31));
            }
            p = block_sum(p, s_part);
            if (t < kLR) {
                if constexpr (RDT == MH_DT_Q8R) p *= Ly.router_s[e];
                st_tag(A.lw + (size_t)t * A.lws + e, tagA, p + Ly.router_b[e]);
            }
        }
        MH_STAMP(1);

        // ------------------------------------------------ route
        {
            // Every block routes: its first wave gathers the logits from
            // replica b % kLR (kEL per lane: element lane + 64 j) and selects
            // the stable top-k and the weights, so no routing record has to
            // be broadcast; all blocks reach the same selection from the same
            // words. (One copy polled by every block congests its lines: 32
            // pollers per copy do not.) The block's other waves wait at the
            // barrier below.
            bool late = false;
            if (wave == 0) {
                const int lane = t;
                const int tt = opaque(t);
                uint64_t *lr = A.lw + (size_t)(b % kLR) * A.lws;
                uint64_t wv[kEL];
#pragma unroll
                for (int j = 0; j < kEL; ++j) {
                    const int e = tt + 64 * j;
                    wv[j] = e < E ? ld_tag(lr + e) : (uint64_t)tagA << 32;
                }
                for (unsigned spins = 0;; ++spins) {
                    bool ready = true;
#pragma unroll
                    for (int j = 0; j < kEL; ++j) ready = ready && (unsigned)(wv[j] >> 32) == tagA;
                    if (__all(ready)) break;
                    if (spins > kSpinLimit) {
                        late = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int j = 0; j < kEL; ++j) {
                        const int e = tt + 64 * j;
                        if (e < E && (unsigned)(wv[j] >> 32) != tagA) wv[j] = ld_tag(lr + e);
                    }
                }
                MH_STAMP(16);
                float v[kEL], v0[kEL];
#pragma unroll
                for (int j = 0; j < kEL; ++j) {
                    v[j] = lane + 64 * j < E ? __uint_as_float((uint32_t)wv[j]) : -INFINITY;
                    v0[j] = v[j];
                }
                int my_sel;
                float my_val;
                wave_topk(v, K, &my_sel, &my_val);
                MH_STAMP(17);
                const float my_w = wave_weight(v0, K, A.router_norm, my_val);
                MH_STAMP(18);
                if (lane < K) {
                    // (addresses from an opaque lane: recomputed here, not
                    // hoisted out of the layer loop and spilled)
                    const int ln = opaque(lane);
                    s_sel[ln] = my_sel;
                    s_w[ln] = my_w;
                    if (b == 0) {
                        if (A.sel) A.sel[(size_t)l * K + ln] = my_sel;
                        if (A.w) A.w[(size_t)l * K + ln] = my_w;
                        if (A.usage && my_sel >= 0)
                            __hip_atomic_fetch_add(&A.usage[(size_t)l * E + my_sel], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            if (__syncthreads_or(late)) {
                if (t == 0) __hip_atomic_store(A.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                return;
            }
        }
        MH_STAMP(2);

        // ------------------------------------------------ B: gate/up
        const rsrc_t rex = make_rsrc(Ly.experts, layer_bytes);
        mh_u4 qd[kUC];       // this thread's down rows (loaded in phase B, used in phase C)
        uint32_t sd[kUC];
        float bd_pref = 0.f;
        {
            // Rows come in (gate, up) pairs: pair p of the k experts laid end
            // to end is row p % F of expert p / F. The block takes pairs
            // [p_begin, p_begin + np); they span at most two experts (np <= F,
            // plan check): expert ia from row rb, then ia + 1.
            const int C = A.CH;
            const int ns = kThreads / C;
            const int tt = opaque(t);
            const int slot = tt / C, c = tt - slot * C;
            const bool active = slot < ns;
            const int PB = (K * F + NB - 1) / NB;
            const int p_begin = b * PB;
            const int np = max(0, min(K * F, p_begin + PB) - p_begin);
            const int ia = min(p_begin / F, K - 1), rb = p_begin - ia * F;
            const int e_a = s_sel[ia], e_b = ia + 1 < K ? s_sel[ia + 1] : -1;
            const uint32_t eo_a = e_a >= 0 ? (uint32_t)e_a * (uint32_t)A.stride : 0u;
            const uint32_t eo_b = e_b >= 0 ? (uint32_t)e_b * (uint32_t)A.stride : 0u;
            const uint32_t od0 = (uint32_t)A.off[0], od1 = (uint32_t)A.off[3];
            const uint32_t os0 = (uint32_t)A.off[1], os1 = (uint32_t)A.off[4];
            float xr[XE];
#pragma unroll
            for (int j = 0; j < XE; ++j) xr[j] = active ? xbs[c * 33 + j] : 0.f;
            // One pass (plan check: np <= ns * kUP). Branch-free loads: a
            // past-the-end pair or an idle slot re-reads the block's last pair
            // and is masked out in the math; scale bits stay raw until every
            // load is in flight.
            mh_u4 qg[kUP], qu[kUP];
            uint32_t sg[kUP], su[kUP];
            const int sl = active ? slot : ns - 1;
            const int plast = max(np - 1, 0);
#pragma unroll
            for (int u = 0; u < kUP; ++u) {
                const int pr = rb + min(u * ns + sl, plast);
                const bool second = pr >= F;
                const uint32_t eo = second ? eo_b : eo_a;
                const uint32_t rc = (uint32_t)((second ? pr - F : pr) * C + c);
                qg[u] = ld_w16(rex, eo + od0 + rc * 16u);
                qu[u] = ld_w16(rex, eo + od1 + rc * 16u);
                sg[u] = ld_w2(rex, eo + os0 + rc * 2u);
                su[u] = ld_w2(rex, eo + os1 + rc * 2u);
            }
            // this thread's epilogue pair's biases, behind the weights
            float bg_pref, bu_pref;
            {
                const int pr = rb + min(t, plast);
                const bool second = pr >= F;
                const uint32_t eo = second ? eo_b : eo_a;
                const uint32_t r4 = (uint32_t)(second ? pr - F : pr) * 4u;
                bg_pref = ld_f(rex, eo + (uint32_t)A.off[2] + r4);
                bu_pref = ld_f(rex, eo + (uint32_t)A.off[5] + r4);
            }
            __builtin_amdgcn_sched_barrier(0);   // all loads issued before any math
            MH_STAMP(9);
#pragma unroll
            for (int u = 0; u < kUP; ++u) {
                const int pp = u * ns + slot;
                const bool inr = active && pp < np;
                const bool valid = inr && (rb + pp >= F ? e_b : e_a) >= 0;
                const float g = mh_dot_chunk<XDT>(qg[u], xr) * (valid ? mh_f16((uint16_t)sg[u]) : 0.f);
                const float v = mh_dot_chunk<XDT>(qu[u], xr) * (valid ? mh_f16((uint16_t)su[u]) : 0.f);
                if (inr) {
                    red[(2 * pp) * C + c] = g;
                    red[(2 * pp + 1) * C + c] = v;
                }
                __builtin_amdgcn_sched_barrier(0);   // one pair's math at a time
            }
            MH_STAMP(10);
            if constexpr (!MF) {
                // the gate/up weight registers are free: start the down slice
                // now, so it streams in during the reduction, the epilogue and
                // the barrier (branch-free: out-of-range rows re-read row 0 of
                // the slice, idle slots and unfilled routing slots the first
                // routed expert; all are masked out in the math)
                const int CD = A.CF, nsC = kThreads / CD, spe = nsC / K;
                const int td = opaque(t);
                const int dslot = td / CD, dc = td - dslot * CD;
                const int di = dslot / spe, dsub = dslot - di * spe;
                const int de = di < K ? s_sel[di] : -1;
                const int ea = de >= 0 ? de : max(s_sel[0], 0);
                const uint32_t eo = (uint32_t)ea * (uint32_t)A.stride;
                const int RC = (H + NB - 1) / NB, r_begin = b * RC;
                const int nr = max(0, min(H, r_begin + RC) - r_begin);
                const int rows_ok = nr > 0 ? nr : 1, r0 = min(r_begin, H - 1);
#pragma unroll
                for (int u = 0; u < kUC; ++u) {
                    const int j = min(dsub + spe * u, rows_ok - 1);
                    const uint32_t rc = (uint32_t)((r0 + j) * CD + dc);
                    qd[u] = ld_w16(rex, eo + (uint32_t)A.off[6] + rc * 16u);
                    sd[u] = ld_w2(rex, eo + (uint32_t)A.off[7] + rc * 2u);
                }
                if (t < K * nr) {   // the down biases: (expert ib, row jb) -> thread ib * nr + jb
                    const int ib = t / nr, jb = t - ib * nr;
                    const int eb = s_sel[ib];
                    if (eb >= 0)
                        bd_pref = ld_f(rex, (uint32_t)eb * (uint32_t)A.stride + (uint32_t)A.off[8] +
                                                (uint32_t)(r_begin + jb) * 4u);
                }
            }
            __syncthreads();
            block_reduce_rows(red, C, 2 * np, kThreads / 64, res, [](int) { return true; });
            __syncthreads();
            MH_STAMP(11);
            if constexpr (MF) {
                if (wave == 0) {
                    // epilogue (np <= 64: one pair per lane): h as two f16
                    // planes, hi = h rounded, lo = (h - hi) rounded; then
                    // arrive as soon as this wave's stores are complete
                    if (t < np) {
#pragma clang fp contract(off)
                        const int pr = rb + t;
                        const bool second = pr >= F;
                        const int e = second ? e_b : e_a;
                        float hv = 0.f;
                        if (e >= 0)
                            hv = act_fn(res[2 * t] + bg_pref, res[2 * t + 1] + bu_pref, A.alpha, A.limit, A.act_plain);
                        const _Float16 hi = (_Float16)hv;
                        const _Float16 lo = (_Float16)(hv - (float)hi);
                        const uint32_t o = (uint32_t)((second ? ia + 1 : ia) * A.Fpad + (second ? pr - F : pr));
                        st_dev16(rh16, o * 2u, __builtin_bit_cast(uint16_t, hi));
                        st_dev16(rh16, ((uint32_t)(K * A.Fpad) + o) * 2u, __builtin_bit_cast(uint16_t, lo));
                    }
                    __builtin_amdgcn_s_waitcnt(0);
                    if (t == 0)
                        __hip_atomic_store(&A.flags[b], tagB, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    // waves 1.. load the block's down rows (whole rows per
                    // instruction: thread (slot, chunk)) while the barrier
                    // completes, then stage them in LDS as row rho = i * RC + j
                    // at a stride of SD chunks (odd: the MFMA lanes' 16 rows
                    // fall in distinct banks)
                    const int CD = A.CF, SD = CD | 1, nsC = (kThreads - 64) / CD, spe = nsC / K;
                    const int RC = (H + NB - 1) / NB, r_begin = b * RC;
                    const int nr = max(0, min(H, r_begin + RC) - r_begin);
                    if (nr > 0) {
                        const int td = opaque(t) - 64;
                        const int dslot = td / CD, dc = td - dslot * CD;
                        const int di = dslot / spe, dsub = dslot - di * spe;
                        const int de = di < K ? s_sel[di] : -1;
                        const int ea = de >= 0 ? de : max(s_sel[0], 0);
                        const uint32_t eo = (uint32_t)ea * (uint32_t)A.stride;
#pragma unroll
                        for (int u = 0; u < kUC; ++u) {
                            const uint32_t rc = (uint32_t)((r_begin + min(dsub + spe * u, nr - 1)) * CD + dc);
                            qd[u] = ld_w16(rex, eo + (uint32_t)A.off[6] + rc * 16u);
                            sd[u] = ld_w2(rex, eo + (uint32_t)A.off[7] + rc * 2u);
                        }
                        // the down biases: (expert ib, row jb) -> thread 64 + ib * nr + jb
                        const int tb = min(td, K * nr - 1);
                        const int ib = tb / nr, jb = tb - ib * nr;
                        const int eb = s_sel[ib];
                        const float bdv = ld_f(rex, (uint32_t)max(eb, 0) * (uint32_t)A.stride + (uint32_t)A.off[8] +
                                                        (uint32_t)(r_begin + jb) * 4u);
                        if (di < K) {
#pragma unroll
                            for (int u = 0; u < kUC; ++u) {
                                const int j = dsub + spe * u;
                                if (j < nr) {
                                    const int o = (di * RC + j) * SD + dc;
                                    *(mh_u4 *)(s_dw + (size_t)o * 16) = qd[u];
                                    s_ds[o] = (uint16_t)sd[u];
                                }
                            }
                        }
                        if (td < K * nr) bds[td] = eb >= 0 ? bdv : 0.f;
                    }
                }
            } else {
                // epilogue: pair t -> h (np <= F <= kThreads pairs: one per thread)
                if (t < np) {
                    const int pr = rb + t;
                    const bool second = pr >= F;
                    const int e = second ? e_b : e_a;
                    float hv = 0.f;
                    if (e >= 0) hv = act_fn(res[2 * t] + bg_pref, res[2 * t + 1] + bu_pref, A.alpha, A.limit, A.act_plain);
                    st_dev(A.h + (size_t)(second ? ia + 1 : ia) * F + (second ? pr - F : pr), hv);
                }
            }
        }
        MH_STAMP(3);
        if constexpr (!MF) bar_arrive(A.flags, tagB);

        // ------------------------------------------------ C: down + combine
        if constexpr (MF) {
            const int CF = A.CF, NQC = (CF + 3) >> 2;
            const int RC = (H + NB - 1) / NB, r_begin = b * RC;
            const int nr = max(0, min(H, r_begin + RC) - r_begin);
            const int rowsC = K * RC;
            // a block without output rows reads no h (the next layer's
            // producers may overwrite it as soon as every x row is in)
            if (nr > 0 || b == 0) {
                MH_STAMP(4);
                if (!bar_wait(A.flags, A.go, tagB, A.err, &s_ok)) return;
                MH_STAMP(5);
                const int tt = opaque(t);
                const int lane = tt & 63, m = lane & 15, g = lane >> 4;
                const int wv = __builtin_amdgcn_readfirstlane(tt >> 6);
                // B: column m = 2 i + term reads 8 values of plane (m & 1),
                // slot i = m / 2
                // (lanes of unused columns and K steps past the end read
                // past the buffer, which returns zeros: no branch)
                v8h hb[kQ][4];
#pragma unroll
                for (int u = 0; u < kQ; ++u) {
                    const int q = kQ * wv + u;
                    const bool use = q < NQC && m < 2 * K;
                    const uint32_t e16 = (uint32_t)(((m & 1) * K + (m >> 1)) * A.Fpad + 128 * q + 32 * g);
                    const uint32_t o = use ? e16 * 2u : 0x80000000u;
#pragma unroll
                    for (int j = 0; j < 4; ++j) hb[u][j] = __builtin_bit_cast(v8h, ld_dev16(rh16, o + 16u * j));
                }
                MH_STAMP(12);
                switch ((rowsC + 15) >> 4) {   // block-uniform (plan check: rows <= 16 kRTC)
                case 1: dn_mfma_t<1>(s_dw, s_ds, hb, CF | 1, CF, rowsC, RC, red); break;
                case 2: dn_mfma_t<2>(s_dw, s_ds, hb, CF | 1, CF, rowsC, RC, red); break;
                case 3: dn_mfma_t<3>(s_dw, s_ds, hb, CF | 1, CF, rowsC, RC, red); break;
                default: break;
                }
                MH_STAMP(13);
                __syncthreads();
                if (t < rowsC) {
                    float sum = 0.f;
#pragma unroll
                    for (int w = 0; w < kThreads / 64; ++w) sum += red[w * 48 + t];
                    res[t] = sum;
                }
                __syncthreads();
                MH_STAMP(14);
                for (int j = t; j < nr; j += kThreads) {
#pragma clang fp contract(off)
                    const int r = r_begin + j;
                    float moe = 0.f;
                    for (int ii = 0; ii < K; ++ii) {
                        if (s_sel[ii] < 0) continue;
                        const float y = res[ii * RC + j] + bds[ii * nr + j];
                        moe = moe + s_w[ii] * y;
                    }
                    if (l + 1 < A.n_layers) st_tag(A.xw + r, tagC, xs[r] + moe);
                    else st_dev(A.x + r, xs[r] + moe);
                }
            }
        } else {
            // one pass (plan check): slot -> (expert i, row phase sub), rows
            // j = sub + spe * u of this block's slice
            const int C = A.CF;
            const int nsC = kThreads / C;
            const int tt = opaque(t);
            const int slot = tt / C, c = tt - slot * C;
            const int RC = (H + NB - 1) / NB;
            const int r_begin = b * RC;
            const int nr = max(0, min(H, r_begin + RC) - r_begin);
            const int spe = nsC / K;
            const int i = slot / spe, sub = slot - i * spe;
            const bool act = i < K;
            const int e = act ? s_sel[i] : -1;
            __builtin_amdgcn_sched_barrier(0);
            MH_STAMP(4);
            if (!bar_wait(A.flags, A.go, tagB, A.err, &s_ok)) return;
            MH_STAMP(5);
            float xr[XE];
            {
                const uint32_t hb = (uint32_t)((act ? i : 0) * F + c * XE) * 4u;
#pragma unroll
                for (int jj = 0; jj < XE / 4; ++jj) {
                    const mh_u4 v = ld_dev16(rh, hb + (uint32_t)jj * 16u);
                    xr[4 * jj + 0] = act ? __uint_as_float(v.x) : 0.f;
                    xr[4 * jj + 1] = act ? __uint_as_float(v.y) : 0.f;
                    xr[4 * jj + 2] = act ? __uint_as_float(v.z) : 0.f;
                    xr[4 * jj + 3] = act ? __uint_as_float(v.w) : 0.f;
                }
            }
            MH_STAMP(12);
#pragma unroll
            for (int u = 0; u < kUC; ++u) {
                const int j = sub + spe * u;
                const bool valid = e >= 0 && j < nr;
                const float p = mh_dot_chunk<XDT>(qd[u], xr) * (valid ? mh_f16((uint16_t)sd[u]) : 0.f);
                if (act && j < nr) red[(i * RC + j) * C + c] = p;
                __builtin_amdgcn_sched_barrier(0);
            }
            if (t < K * nr) bds[t] = bd_pref;
            MH_STAMP(13);
            __syncthreads();
            block_reduce_rows(red, C, K * RC, kThreads / 64, res, [&](int it) { return it % RC < nr; });
            __syncthreads();
            MH_STAMP(14);
            // combine in selection order: moe = sum_i w_i (dot_i + bd_i); x += moe
            for (int j = t; j < nr; j += kThreads) {
#pragma clang fp contract(off)
                const int r = r_begin + j;
                float moe = 0.f;
                for (int ii = 0; ii < K; ++ii) {
                    if (s_sel[ii] < 0) continue;
                    const float y = res[ii * RC + j] + bds[ii * nr + j];
                    moe = moe + s_w[ii] * y;
                }
                if (l + 1 < A.n_layers) st_tag(A.xw + r, tagC, xs[r] + moe);
                else st_dev(A.x + r, xs[r] + moe);
            }
        }
        MH_STAMP(6);
        if (l + 1 < A.n_layers) pf = prefetch_router<RDT>(A, l + 1);
        MH_STAMP(7);
    }
#undef MH_STAMP
}

__global__ void k_fill_u32(unsigned *p, int n, unsigned v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// Flags a down-projection MXFP4 scale that the MFMA path cannot apply
// exactly in f16: it must be zero or a power of two in [2^-23, 2^13], so that
// every e2m1 value times it is an f16.
__global__ void k_scan_scales(const uint8_t *experts, uint64_t stride, uint64_t od, int n, unsigned *bad) {
    const uint16_t *d = (const uint16_t *)(experts + (uint64_t)blockIdx.y * stride + od);
    bool ok = true;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned v = d[i], e = (v >> 10) & 31u, mn = v & 1023u;
        ok = ok && ((v & 0x7FFFu) == 0 || (e == 0 && mn >= 2 && (mn & (mn - 1)) == 0) || (e != 0 && e <= 28 && mn == 0));
    }
    if (!ok) atomicOr(bad, 1u);
}

template <int RDT, int XDT, bool MF>
int launch_t(const StepArgs &A, int nb, size_t lds, hipStream_t s) {
    auto k = k_decode_step<RDT, XDT, MF>;
    // the LDS attribute and the occupancy query once per device and
    // instantiation (both cost host time comparable to a small step)
    static int ready_dev = -1, per_cu = 0;
    static size_t ready_lds = 0;
    int dev = 0;
    MH_HIP(hipGetDevice(&dev));
    if (dev != ready_dev || lds != ready_lds) {
        MH_HIP(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        MH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, lds));
        ready_dev = dev;
        ready_lds = lds;
    }
    if (per_cu < 1) return fail(MH_E_UNSUPPORTED, "decode step: a %d-thread block with %zu B LDS does not fit a CU", kThreads, lds);
    StepArgs a = A;
    void *args[] = {&a};
    const bool prof = profiling();
    if (prof) prof_begin("decode_step", s);
    // One block per CU with the occupancy checked above: every block is
    // resident at once. The cooperative launch makes the runtime verify that
    // too; MIDGE_HIP_COOP=0 selects a plain launch of the same grid (for
    // tools that do not handle cooperative dispatches). A block that were
    // not resident would make the grid's bounded waits time out and report
    // an error through mh_sync, never hang.
    const char *coop = getenv("MIDGE_HIP_COOP");
    hipError_t e;
    if (coop && coop[0] == '0')
        e = hipLaunchKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s);
    else
        e = hipLaunchCooperativeKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s);
    if (prof) prof_end(s);
    return hip_check(e, "decode step cooperative launch");
}

}  // namespace

// Barrier words: nb flags, then (from a 128-byte line) kGoCopies release
// words kGoStride apart.
static int go_offset(int nb) { return (nb + 63) / 32 * 32; }
static int flag_words(int nb) { return go_offset(nb) + kGoCopies * kGoStride; }

// Scratch and tables a stack keeps for the one-launch path.
struct StepPlan {
    StepLayer *layers = nullptr;   // device [L]
    unsigned *flags = nullptr;     // device [flag_words(nb)]: flags, then the release word's copies
    uint64_t *tagged = nullptr;    // device: logit copies [kLR][lws] | x [H], tagged words
    size_t tagged_words = 0;
    unsigned long long *trace = nullptr;   // device [L][16][nb] (filled while profiling)
    int n_layers = 0;
    unsigned *err = nullptr;       // host-mapped pinned [1]: set by a timed-out barrier
    unsigned *err_dev = nullptr;   // its device address
    float *h = nullptr;            // device [K][F]
    uint16_t *h16 = nullptr;       // device [2][K][Fpad]
    int Fpad = 0;
    int mf = 0;                    // 1 = the MFMA path may run the expert GEMVs
    unsigned seq = 0;              // next barrier sequence number
    int nb = 0;
    int ok = 0;                    // 1 = eligible, 0 = not (reason recorded)
    char why[160] = {0};
};

int step_plan_create(const DevLayer *layers, int n_layers, StepPlan **out) {
    StepPlan *p = new StepPlan();
    *out = p;
    const DevLayer &L0 = layers[0];
    auto reject = [&](const char *why) {
        snprintf(p->why, sizeof(p->why), "%s", why);
        p->ok = 0;
        return MH_OK;
    };
    if (L0.expert_dt != MH_DT_MXFP4 && L0.expert_dt != MH_DT_Q4G32) return reject("experts are not 4-bit g32");
    if (L0.hidden % 32 || L0.ffn % 32 || L0.hidden / 32 > kThreads || L0.ffn / 32 > kThreads)
        return reject("hidden/ffn not multiples of 32 or too wide");
    if (L0.n_experts > 64 * kEL || L0.top_k > 16) return reject("too many experts");
    if (L0.expert_stride * (uint64_t)L0.n_experts >= (1ull << 32)) return reject("a layer's experts exceed 4 GiB");
    for (int l = 0; l < n_layers; l++) {
        const DevLayer &L = layers[l];
        if (L.router.dt != L0.router.dt || L.expert_dt != L0.expert_dt || L.act_plain != L0.act_plain ||
            L.router_norm != L0.router_norm || L.alpha != L0.alpha || L.limit != L0.limit ||
            L.norm_eps != L0.norm_eps)
            return reject("layers differ in dtype or activation parameters");
        if ((uintptr_t)L.router.data % 16 || (uintptr_t)L.experts % 16) return reject("unaligned weights");
    }
    if (L0.router.dt != MH_DT_Q8R && L0.router.dt != MH_DT_F32) return reject("router is not q8r or f32");
    const int re = L0.router.dt == MH_DT_Q8R ? 16 : 4;
    if (L0.hidden % re) return reject("router width not a chunk multiple");
    const int nb = device_cus();
    {
        const int H = (int)L0.hidden, F = (int)L0.ffn, K = L0.top_k;
        if (H > kNX * kThreads) return reject("hidden exceeds the router phase's per-thread share");
        // gate/up: a block's pairs span at most two experts and the epilogue
        // has one pair per thread
        const int PB = (K * F + nb - 1) / nb;
        if (PB > F || PB > kThreads) return reject("a block's gate/up pairs span more than two experts");
        if (PB > (kThreads / (H / 32)) * kUP) return reject("gate/up does not fit one pass");
        // down: one pass, every routed expert gets slots, each slot's rows of
        // the block's slice fit kUC iterations, one bias per thread
        const int nsC = kThreads / (F / 32);
        const int spe = K > 0 ? nsC / K : 0;
        const int RC = (H + nb - 1) / nb;
        if (spe < 1 || RC > spe * kUC || K * RC > kThreads) return reject("down phase does not fit one pass");
    }
    // MFMA down path: MXFP4 experts, the clamped SwiGLU (|h| <= limit (limit +
    // 1) fits f16), shapes within the tiles, exact f16 scales (scanned below)
    {
        const int H = (int)L0.hidden, F = (int)L0.ffn, K = L0.top_k;
        const int RC = (H + nb - 1) / nb, PB = (K * F + nb - 1) / nb;
        const int spe = K > 0 ? (kThreads - 64) / (F / 32) / K : 0;   // down rows in flight: waves 1..
        const float lim = L0.limit;
        p->mf = L0.expert_dt == MH_DT_MXFP4 && !L0.act_plain && lim >= 0.f && lim * (lim + 1.f) < 60000.f &&
                F <= kKPad && K * RC <= 16 * kRTC && 2 * K <= 16 && PB <= 64 && spe >= 1 && RC <= spe * kUC &&
                K * RC <= kThreads - 64;
    }
    std::vector<StepLayer> host((size_t)n_layers);
    for (int l = 0; l < n_layers; l++) {
        const DevLayer &L = layers[l];
        host[(size_t)l] = StepLayer{L.experts, L.router.data, (const float *)L.router.scales, L.router_b, L.mlp_norm};
    }
    MH_HIP(hipMalloc(&p->layers, sizeof(StepLayer) * (size_t)n_layers));
    MH_HIP(hipMemcpy(p->layers, host.data(), sizeof(StepLayer) * (size_t)n_layers, hipMemcpyHostToDevice));
    MH_HIP(hipMalloc(&p->flags, sizeof(unsigned) * (size_t)flag_words(nb)));
    MH_HIP(hipMalloc(&p->trace, sizeof(unsigned long long) * kStamps * (size_t)n_layers * (size_t)nb));
    p->n_layers = n_layers;
    MH_HIP(hipHostMalloc((void **)&p->err, sizeof(unsigned), hipHostMallocMapped));
    *p->err = 0;
    MH_HIP(hipHostGetDevicePointer((void **)&p->err_dev, p->err, 0));
    watch_async_error(p->err, "decode step: a grid barrier timed out (blocks not co-resident)");
    p->tagged_words = (size_t)kLR * ((L0.n_experts + 15) / 16 * 16 + 32) + (size_t)L0.hidden;
    MH_HIP(hipMalloc(&p->tagged, sizeof(uint64_t) * p->tagged_words));
    MH_HIP(hipMemset(p->tagged, 0, sizeof(uint64_t) * p->tagged_words));
    MH_HIP(hipMalloc(&p->h, sizeof(float) * (size_t)L0.top_k * (size_t)L0.ffn));
    p->Fpad = (int)((L0.ffn + 127) / 128 * 128);
    MH_HIP(hipMalloc(&p->h16, sizeof(uint16_t) * 2 * (size_t)L0.top_k * (size_t)p->Fpad));
    MH_HIP(hipMemset(p->h16, 0, sizeof(uint16_t) * 2 * (size_t)L0.top_k * (size_t)p->Fpad));   // the padding stays 0
    if (p->mf) {
        unsigned *bad = nullptr;
        MH_HIP(hipMalloc(&bad, sizeof(unsigned)));
        MH_HIP(hipMemset(bad, 0, sizeof(unsigned)));
        const int n_dn = (int)(L0.hidden * (L0.ffn / 32));
        for (int l = 0; l < n_layers; l++) {
            const DevLayer &L = layers[l];
            hipLaunchKernelGGL(k_scan_scales, dim3(16, (unsigned)L.n_experts), dim3(256), 0, 0, L.experts,
                               L.expert_stride, L.off[7], n_dn, bad);
        }
        unsigned hb = 0;
        MH_HIP(hipGetLastError());
        MH_HIP(hipMemcpy(&hb, bad, sizeof(unsigned), hipMemcpyDeviceToHost));
        (void)hipFree(bad);
        if (hb) p->mf = 0;   // the VALU path handles any f16 scale
    }
    MH_HIP(hipMemset(p->flags, 0, sizeof(unsigned) * (size_t)flag_words(nb)));
    MH_HIP(hipDeviceSynchronize());
    p->seq = 1;
    p->nb = nb;
    p->ok = 1;
    return MH_OK;
}

void step_plan_destroy(StepPlan *p) {
    if (!p) return;
    (void)hipFree(p->layers);
    (void)hipFree(p->flags);
    (void)hipFree(p->trace);
    unwatch_async_error(p->err);
    (void)hipHostFree(p->err);
    (void)hipFree(p->tagged);
    (void)hipFree(p->h);
    (void)hipFree(p->h16);
    delete p;
}

bool step_plan_ok(const StepPlan *p) { return p && p->ok; }

int step_run(StepPlan *p, const DevLayer *layers, int n_layers, float *x, int32_t *sel, float *w,
             uint32_t *usage, hipStream_t s) {
    const DevLayer &L0 = layers[0];
    StepArgs A;
    A.layers = p->layers;
    A.n_layers = n_layers;
    A.H = (int)L0.hidden;
    A.F = (int)L0.ffn;
    A.E = L0.n_experts;
    A.K = L0.top_k;
    A.CH = A.H / 32;
    A.CF = A.F / 32;
    A.stride = L0.expert_stride;
    for (int i = 0; i < 9; i++) A.off[i] = L0.off[i];
    A.alpha = L0.alpha;
    A.limit = L0.limit;
    A.eps = L0.norm_eps;
    A.act_plain = L0.act_plain;
    A.router_norm = L0.router_norm;
    A.x = x;
    A.sel = sel;
    A.w = w;
    A.usage = usage;
    A.lws = (A.E + 15) / 16 * 16 + 32;   // copies 256 B past a line boundary apart
    A.lw = p->tagged;
    A.xw = p->tagged + (size_t)kLR * A.lws;
    A.go = p->flags + go_offset(p->nb);
    A.h = p->h;
    A.h16 = p->h16;
    A.Fpad = p->Fpad;
    A.flags = p->flags;
    A.trace = profiling() ? p->trace : nullptr;
    A.err = p->err_dev;
    const unsigned nbar = 3u * (unsigned)n_layers;
    if (p->seq > 0xF0000000u) {   // wrap: restart the sequence from a clean slate
        MH_LAUNCH("fill", k_fill_u32, dim3(1), dim3(256), 0, s, p->flags, flag_words(p->nb), 0u);
        MH_LAUNCH("fill", k_fill_u32, dim3(8), dim3(256), 0, s, (unsigned *)p->tagged, (int)(2 * p->tagged_words), 0u);
        p->seq = 1;
    }
    A.seq0 = p->seq;
    p->seq += nbar;
    const int nb = p->nb;
    const int PB = (A.K * A.F + nb - 1) / nb, RC = (A.H + nb - 1) / nb;
    A.res_floats = std::max(64 * kEL, std::max(2 * PB, A.K * RC)) + 64;
    const int nsB = kThreads / A.CH;
    A.red_floats = std::max(2 * nsB * kUP * A.CH, A.K * RC * A.CF);
    const char *nm = getenv("MIDGE_HIP_NO_MFMA");   // per call, so callers can A/B the two paths
    const bool mf = p->mf && !(nm && nm[0] && nm[0] != '0');
    if (A.H > kHMax || A.res_floats > kResMax || A.red_floats > kRedMax)
        return fail(MH_E_UNSUPPORTED, "decode step: shape exceeds the kernel's LDS capacities");
    const size_t lds = 0;
    if (A.trace)   // stamps a block does not reach (a skipped phase) stay 0
        MH_LAUNCH("fill", k_fill_u32, dim3(64), dim3(256), 0, s, (unsigned *)p->trace,
                  (int)(2 * (size_t)kStamps * n_layers * p->nb), 0u);
    int rc;
    if (L0.router.dt == MH_DT_Q8R) {
        if (L0.expert_dt == MH_DT_MXFP4)
            rc = mf ? launch_t<MH_DT_Q8R, MH_DT_MXFP4, true>(A, nb, lds, s)
                    : launch_t<MH_DT_Q8R, MH_DT_MXFP4, false>(A, nb, lds, s);
        else
            rc = launch_t<MH_DT_Q8R, MH_DT_Q4G32, false>(A, nb, lds, s);
    } else {
        if (L0.expert_dt == MH_DT_MXFP4)
            rc = mf ? launch_t<MH_DT_F32, MH_DT_MXFP4, true>(A, nb, lds, s)
                    : launch_t<MH_DT_F32, MH_DT_MXFP4, false>(A, nb, lds, s);
        else
            rc = launch_t<MH_DT_F32, MH_DT_Q4G32, false>(A, nb, lds, s);
    }
    if (rc || !A.trace) return rc;
    // profiling: fold the per-block phase timestamps (100 MHz clock) into
    // the profile: the mean over blocks and the slowest block of each span
    std::vector<unsigned long long> tr((size_t)kStamps * n_layers * nb);
    MH_HIP(hipMemcpyAsync(tr.data(), p->trace, tr.size() * 8, hipMemcpyDeviceToHost, s));
    MH_HIP(hipStreamSynchronize(s));
    // (name, from, to, only block 0)
    static const struct { const char *name; int a, b; bool b0; } spans[] = {
        {"x_wait", 0, 15, false},   {"router", 15, 1, false},     {"route", 1, 2, false},
        {"route0_gather", 1, 16, true}, {"route0_rank", 16, 17, true}, {"route0_weights", 17, 18, true},
        {"route0_publish", 18, 2, true}, {"gate_up", 2, 3, false}, {"gu_issue", 2, 9, false},
        {"gu_math", 9, 10, false},  {"gu_reduce", 10, 11, false}, {"gu_epilogue", 11, 3, false},
        {"barrier_arrive_prefetch", 3, 4, false}, {"barrier_wait", 4, 5, false}, {"down_combine", 5, 6, false},
        {"dn_hload", 5, 12, false}, {"dn_math", 12, 13, false},  {"dn_reduce", 13, 14, false},
        {"dn_combine", 14, 6, false}, {"tail", 6, 7, false},     {"layer", 0, 7, false}};
    char name[96];
    auto at = [&](int l, int st, int b) { return (double)tr[((size_t)l * kStamps + st) * nb + b]; };
    for (int l = 0; l < n_layers; l++) {
        for (const auto &sp : spans) {
            const int nbk = sp.b0 ? 1 : nb;
            double sum = 0, mx = 0;
            int cnt = 0;
            for (int b = 0; b < nbk; b++) {
                if (at(l, sp.b, b) == 0 || at(l, sp.a, b) == 0) continue;
                const double d = at(l, sp.b, b) - at(l, sp.a, b);
                sum += d;
                mx = std::max(mx, d);
                ++cnt;
            }
            snprintf(name, sizeof(name), "decode_step/%s", sp.name);
            prof_add(name, cnt ? sum / cnt * 1e-5 : 0.0);
            snprintf(name, sizeof(name), "decode_step/%s.max", sp.name);
            prof_add(name, mx * 1e-5);
        }
        // the critical path: from the first block's layer start to the last
        // block's logit, the last block's routing record and the last arrival
        double t0 = 1e300, lastA = 0, lastR = 0, lastB = 0, lastC = 0;
        for (int b = 0; b < nb; b++) {
            t0 = std::min(t0, at(l, 0, b));
            lastA = std::max(lastA, at(l, 1, b));
            lastR = std::max(lastR, at(l, 2, b));
            lastB = std::max(lastB, at(l, 3, b));
            lastC = std::max(lastC, at(l, 6, b));
        }
        // every stamp's earliest and latest block, from the layer's first start
        static const int order[] = {0, 15, 1, 16, 17, 18, 2, 9, 10, 11, 3, 4, 5, 12, 13, 14, 6, 7};
        for (int st : order) {
            double lo = 1e300, hi = 0;
            for (int b = 0; b < nb; b++) {
                if (st >= 16 && b > 0) break;   // block 0 only
                if (at(l, st, b) == 0) continue;
                const double v = at(l, st, b) - t0;
                lo = std::min(lo, v);
                hi = std::max(hi, v);
            }
            snprintf(name, sizeof(name), "decode_step/t%02d.first", st);
            prof_add(name, lo * 1e-5);
            snprintf(name, sizeof(name), "decode_step/t%02d.last", st);
            prof_add(name, hi * 1e-5);
        }
        prof_add("decode_step/crit_logits", (lastA - t0) * 1e-5);
        prof_add("decode_step/crit_routed", (lastR - t0) * 1e-5);
        prof_add("decode_step/crit_h", (lastB - t0) * 1e-5);
        prof_add("decode_step/crit_x", (lastC - t0) * 1e-5);
    }
    return MH_OK;
}

}  // namespace mh
