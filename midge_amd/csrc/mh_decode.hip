// mh_decode.hip — a whole MoE decode step (every layer of a stack, batch 1)
// in one launch: the MoE half of forward()'s layer loop (engine/midge.c:
// 557-560) with moe() (engine/midge.c:469-549) per layer.
//
// Two kernels share the routing phase (route_layer):
//
// k_decode_grp — MXFP4 experts with the clamped SwiGLU (gpt-oss), the
//   default. The grid is G blocks per routed slot (G * K blocks, at most one
//   per CU). Block (slot i, index gi) owns gate/up pairs [PB gi, +PB) and
//   down rows [RB gi, +RB) of slot i's expert, so a block's work touches one
//   expert and its h comes from its own group of G blocks. Per layer:
//     A  every block forms x itself: R.x at layer 0, else the previous
//        layer's x plus moe = sum_i w_i y_i (engine/midge.c:544-548) from the
//        y words every block published (one of kYR copies); then xb =
//        rmsnorm(x) * w in LDS; blocks b < E compute router logit b and
//        publish it in kLR copies;
//     R  every block's first wave gathers the logits and ranks them itself
//        (stable top-k, ties to the lower index) up to its own slot: all
//        blocks reach the same selection and nothing is broadcast;
//     B  the block issues its weight loads, the gate/up pairs first and the
//        down rows behind them, so the layer's weights stream as one
//        transfer; the first wave then ranks the remaining slots and forms
//        the weights while the loads fly; the gate/up math runs as the data
//        arrives; bias + clamped SwiGLU give h, published as tagged words
//        (h as two f16 terms) to the slot's group;
//     C  the down rows are staged in LDS; each wave polls only the part of
//        h that its matrix-core K steps read and multiplies (f16 MFMA); the
//        down bias completes y_i for the block's rows;
//     D  every block publishes its rows of y_i in kYR copies (32-bit words
//        with a 4-bit tag, double-buffered by layer parity); after the last
//        layer the slot-0 block of each row slice forms x += moe for its
//        rows into R.x.
//   There is no grid-wide barrier: every exchange is a tagged word the
//   consumer polls, and every block gathers every block's y once per layer,
//   which also orders the reuse of the exchange buffers from layer to layer.
//
// k_decode_step — the vector-ALU path (q4g32 experts, plain SiLU, down
//   scales the f16 path cannot hold exactly). One block per CU; a block
//   takes an even share of all routed (gate, up) pairs and, after one grid
//   barrier, a slice of output rows for every routed expert.
//
// Tagged words carry the producer's sequence number next to the value in one
// 64-bit store, so a consumer polls the data itself. Every wait is bounded:
// one that does not complete within ~1 s raises an error flag and every
// block exits.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <utility>
#include <vector>

#include "mh_gemv.cuh"
#include "mh_mfma16.cuh"
#include "mh_xchg.cuh"

namespace mh {

struct StepLayer {
    const uint8_t *experts;
    const uint8_t *router_w;
    const float *router_s;   // q8r row scales (unused for an f32 router)
    const float *router_b;
    const float *norm_w;
};

// What the routing phase reads and writes, common to both kernels.
struct RouteArgs {
    const StepLayer *layers;
    int n_layers, H, E, K;
    float eps;
    int router_norm;
    float *x;                // [H] input at layer 0 (and the last layer's output)
    int32_t *sel;            // [L][K] or null
    float *w;                // [L][K] or null
    uint32_t *usage;         // [L][E] or null
    uint64_t *lw;            // [kLR][lws] tagged logits: kLR copies, lws words apart
    int lws;
    unsigned *err;
    unsigned long long *trace;   // [L][kStamps][gridDim.x] per-block phase timestamps, or null
};

struct StepArgs {            // k_decode_step
    RouteArgs R;
    int F;
    int CH, CF;              // 16-byte chunks per expert row: H / 32, F / 32
    uint64_t stride;
    uint64_t off[9];
    float alpha, limit;
    int act_plain;
    uint64_t *xw;            // [H] tagged x between layers
    float *h;                // [K][F] scratch
    unsigned *flags;         // [gridDim.x] barrier flags
    unsigned *go;            // barrier release word (written by block 0)
    unsigned seq0;           // first sequence number of this launch (3 per layer)
};

struct GrpArgs {             // k_decode_grp
    RouteArgs R;
    int F;
    int CH, CF;              // 16-byte chunks per row: H / 32 (gate/up), F / 32 (down)
    int G, PB, RB;           // blocks per slot; gate/up pairs and down rows per block
    uint64_t stride;
    uint64_t off[9];
    float alpha, limit;
    uint64_t *hw;            // [kHR][K][hws] tagged h (payload: hi f16 | lo f16 << 16)
    int hws;
    uint32_t *yw;            // [2][kYR][K][yws] y words (layer parity, copy, slot): f32 with a 4-bit tag
    int yws;
    uint64_t *y1;            // [K][yws] tagged y of slots 1.. (one-layer launches)
    unsigned *flags;         // [gridDim.x] per-block flags: x of layer 0 read (one-layer launches)
    unsigned seq0;           // first sequence number of this launch (4 per layer)
    unsigned bank;           // the y tags' bank: the plan's count of launches of several layers, mod 2
    // routing given (one layer, one token; null otherwise): x += w_i
    // expert_{sel_i}(xb) over the K slots in ascending expert order
    const float *gxb;        // [H] the normed input
    const int32_t *gsel;     // [K]
    const float *gw;         // [K]
};

namespace {

constexpr int kThreads = 512;   // 8 waves: 2 per SIMD, up to 256 VGPRs each
constexpr int kUP = 9;          // gate/up row pairs in flight per thread
constexpr int kUC = 12;         // down rows in flight per thread (k_decode_step)
constexpr int kUD = 9;          // down rows in flight per thread (k_decode_grp)
constexpr int kPD = 4;          // gate/up pairs in flight per thread (k_decode_grp)
static_assert(kPD <= kUP, "k_decode_grp's gate/up pipeline depth");
constexpr int kNX = 8;          // x elements per thread in the router phase (H <= kNX * kThreads)
constexpr int kStamps = 24;     // phase timestamps per layer and block while profiling
constexpr int kEL = 2;          // logits per lane in the routing wave (E <= 64 * kEL)
constexpr int kLR = 8;          // copies of the logits (each polled by NB / kLR blocks)
constexpr int kYR = 8;          // copies of y (k_decode_grp: each polled by NB / kYR blocks)
constexpr int kHR = 2;          // copies of h (k_decode_grp: each polled by G / kHR blocks)
constexpr int kGoCopies = 8;    // copies of the barrier's release word
constexpr int kGoStride = 64;   // words between them (256 B)
constexpr int kMaxK = 16;       // engine/midge.c:44 MAX_TOPK
constexpr int kMaxGrpK = 4;     // top-k of k_decode_grp (every block gathers k x H words of y per layer)
// static LDS capacities (plan creation checks a stack against them)
constexpr int kHMax = 3072;         // hidden size
constexpr int kNG = (kHMax + kThreads - 1) / kThreads;   // x elements per thread in k_decode_grp's y gather
constexpr int kResMax = 1024;       // floats of reduced rows
constexpr int kRedMax = 8192;       // floats of partial sums
constexpr int kQ = 3;               // 128-column K steps per wave (ffn <= 8 * kQ * 128)
constexpr int kKPad = 8 * kQ * 128; // largest ffn of k_decode_grp
constexpr int kRBMax = 48;          // down rows per block of k_decode_grp (3 matrix-core row tiles)
constexpr int kSDMax = kKPad / 32 + 1;   // LDS row stride (chunks) of the staged down rows
constexpr int kGrpBig = kRBMax * kSDMax * 16 > kRedMax * 4 ? kRBMax * kSDMax * 16 : kRedMax * 4;
constexpr int kScW = 8192;          // bytes per staged scale window of k_decode_grp (gate, up, down)
constexpr int kScLoads = 3;         // 16-byte scale loads per thread (3 windows <= kScLoads * 512 chunks)

// Memory access. Every load goes through a buffer resource (32-bit offsets,
// out-of-range reads return 0). Weights are streamed with the nontemporal
// hint. Data that blocks exchange inside the launch (x, logits, h, y) is
// written with device-scope stores and read with device-scope loads, which
// are coherent across the XCDs' L2 caches: the exchanges then need no L2
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

// Per-block phase timestamps (100 MHz wall clock), written by thread 0 of
// each block while profiling: trace[(layer * kStamps + id) * blocks + block].
struct Stamper {
    unsigned long long *tr;
    int nb;
    __device__ __forceinline__ void operator()(int l, int id) const {
        if (tr) tr[(size_t)(l * kStamps + id) * nb] = wall_clock64();
    }
};

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
            if (!ok) raise_err(err);
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


// y words (k_decode_grp): one 32-bit word per value, an f32 rounded to a
// multiple of 16 units in the last place (within 2^-20 relative; inf and nan
// keep their class) whose low 4 bits carry a tag, never 0 (zeroed memory
// never reads as ready). Launches alternate between two banks of tags (1..7
// and 8..14); within a launch the tag of layer l is its bank's (l / 2) mod 7.
// Every launch of several layers writes every y location at least once (a
// one-layer launch uses its own tagged words instead), and kernel boundaries
// order one launch's stores before the next launch's loads, so a location
// holds this launch's words or the previous launch's (the other bank); within
// a launch a location is written once per two layers and every reader has
// read its previous value before it is written again.
__device__ __forceinline__ uint32_t ynib(unsigned bank, int l) { return 1u + 7u * bank + (unsigned)(l >> 1) % 7u; }
__device__ __forceinline__ uint32_t y_word(float v, uint32_t nib) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t r = (u & 0x7F800000u) == 0x7F800000u ? u : u + 8u;   // a carry rounds up into the exponent
    return (r & ~15u) | nib;
}
__device__ __forceinline__ float y_val(uint32_t w) { return __uint_as_float(w & ~15u); }
__device__ __forceinline__ uint32_t ld_u32_dev(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u32_dev(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stable top-k over the wave's E <= 64 * kEL logits (lane holds element
// lane + 64 j in v[j]; absent elements are -inf): k rounds of "largest
// remaining value, lowest index among equals"; only values > -1e30
// qualify, unfilled slots get -1 (engine/midge.c:476-486). Lane i < k ends
// with slot i's expert in *sel and its logit in *val (-1e30 if unfilled).
__device__ __forceinline__ void wave_topk(float *v, int k, int *sel, float *val, int i0 = 0) {
    const int lane = threadIdx.x & 63;
    if (i0 == 0) {
        *sel = -1;
        *val = -1e30f;
    }
    for (int i = i0; i < k; ++i) {
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
__device__ __forceinline__ RouterPref prefetch_router(const RouteArgs &R, int l) {
    RouterPref p;
    const StepLayer Lp = R.layers[l];
    const int b = blockIdx.x, t = threadIdx.x, H = R.H;
    const int e = b < R.E ? b : 0;
    constexpr uint32_t wb = RDT == MH_DT_Q8R ? 1u : 4u;   // bytes per router weight
    const rsrc_t rw = make_rsrc(Lp.router_w, (uint32_t)R.E * (uint32_t)H * wb);
#pragma unroll
    for (int k = 0; k < kNX; ++k) {   // past H: the next row's weights (or 0), met by x = 0
        const uint32_t o = ((uint32_t)e * (uint32_t)H + (uint32_t)(t + k * kThreads)) * wb;
        if constexpr (RDT == MH_DT_Q8R) p.rw[k] = __builtin_amdgcn_raw_buffer_load_b8(rw, o, 0, 0);
        else p.rw[k] = __builtin_amdgcn_raw_buffer_load_b32(rw, o, 0, 0);
    }
    p.rs = 1.0f;
    if constexpr (RDT == MH_DT_Q8R) p.rs = ld_f(make_rsrc(Lp.router_s, (uint32_t)R.E * 4u), (uint32_t)e * 4u);
    p.rb = ld_f(make_rsrc(Lp.router_b, (uint32_t)R.E * 4u), (uint32_t)e * 4u);
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

// LDS of the routing phase.
struct RouteLds {
    float *part;     // [16]
    int *sel;        // [kMaxK]
    float *w;        // [kMaxK]
    float *xs;       // [H] x at layer start
    float *xbs;      // xb = rmsnorm(x) * w in 32-element groups padded to 33 floats
};

// x of layer l from R.x (layer 0) or as tagged words from xsrc (tag xtag, the
// previous layer's output that k_decode_step publishes): thread t gets
// elements t + k kThreads (0 past H); each thread loads its <= kNX words and
// re-polls only the late ones. Returns false (in every thread) if a wait
// timed out.
__device__ __forceinline__ bool gather_x_tagged(const RouteArgs &R, int l, uint64_t *xsrc, unsigned xtag,
                                                float (&xv)[kNX]) {
    const int H = R.H, t = threadIdx.x;
    if (l == 0) {
        const rsrc_t rx = make_rsrc(R.x, (uint32_t)H * 4u);
#pragma unroll
        for (int k = 0; k < kNX; ++k) xv[k] = ld_dev(rx, (uint32_t)(t + k * kThreads) * 4u);   // 0 past H
        return true;
    }
    uint64_t wv[kNX];
    const int tt = opaque(t);
#pragma unroll
    for (int k = 0; k < kNX; ++k) {
        const int i = tt + k * kThreads;
        wv[k] = i < H ? ld_tag(xsrc + i) : (uint64_t)xtag << 32;
    }
    bool late = false;
    for (unsigned spins = 0;; ++spins) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < kNX; ++k) ready = ready && tag_is(wv[k], xtag);
        if (ready) break;
        if (spins > kSpinLimit) {
            late = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < kNX; ++k) {
            const int i = tt + k * kThreads;
            if (i < H && !tag_is(wv[k], xtag)) wv[k] = ld_tag(xsrc + i);
        }
    }
    if (__syncthreads_or(late)) {
        if (t == 0) raise_err(R.err);
        return false;
    }
#pragma unroll
    for (int k = 0; k < kNX; ++k) xv[k] = __uint_as_float((uint32_t)wv[k]);
    return true;
}

// The ranking wave's state between route_layer (ranked up to a given slot)
// and route_finish (the remaining slots, the weights and the records).
struct RankState {
    float v[kEL], v0[kEL];
    int sel;
    float val;
};

// The rest of layer l's routing after a route_layer that ranked slots
// [0, from] (wave 0): slots from + 1 .. K - 1, the weights into S.sel / S.w,
// block 0's records. The caller's next block barrier publishes them.
__device__ __forceinline__ void route_finish(const RouteArgs &R, int l, const RouteLds &S, RankState &rs, int from) {
    const int E = R.E, K = R.K, t = threadIdx.x;
    if (t >= 64) return;
    const int lane = t;
    wave_topk(rs.v, K, &rs.sel, &rs.val, from + 1);
    const float my_w = wave_weight(rs.v0, K, R.router_norm, rs.val);
    if (lane < K) {
        const int ln = opaque(lane);
        S.sel[ln] = rs.sel;
        S.w[ln] = my_w;
        if (blockIdx.x == 0) {
            if (R.sel) R.sel[(size_t)l * K + ln] = rs.sel;
            if (R.w) R.w[(size_t)l * K + ln] = my_w;
            if (R.usage && rs.sel >= 0)
                __hip_atomic_fetch_add(&R.usage[(size_t)l * E + rs.sel], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Phase A and the routing of layer l, common to both kernels.
//  - x: getx(xv) fills this thread's elements t + k kThreads of x (0 past H)
//    and returns false if a wait timed out (gather_x_tagged, or k_decode_grp's
//    combine of the previous layer's y).
//  - One DPP-reduced block sum gives both sum(x^2) and this block's router
//    dot with x * w (the norm weights): logit b = inv * dot * scale + bias,
//    with inv = 1 / sqrt(mean(x^2) + eps) factored out of the row's dot
//    (engine/mkern.h:238-243, then the router matvec). Blocks b < E publish
//    it in kLR copies; rows beyond the grid are looped over.
//  - xb = x * inv * w goes to LDS in 32-element groups padded to 33 floats:
//    a thread reading group c element by element and its wave's 64 lanes
//    then hit 64 distinct banks.
//  - Every block's first wave gathers the E logits from copy b % kLR and
//    ranks them (wave_topk: the reference's insertion order, ties to the
//    lower index) and computes the weights; block 0 records sel, w and the
//    usage counts. The block's other waves wait at the closing barrier.
//    With `split` (k_decode_grp) the wave ranks slots 0 .. upto only, the
//    block's own expert, and leaves the rest to route_finish: a block needs
//    only its slot's expert to issue its weight loads.
// Returns false, with the error flag raised, if a wait timed out (every
// thread of the block returns the same value).
template <int RDT, class GetX>
__device__ __forceinline__ bool route_layer(const RouteArgs &R, const RouterPref &pf, int l, GetX getx,
                                            unsigned ltag, const RouteLds &S, const Stamper &stamp,
                                            RankState *split = nullptr, int upto = 0) {
    const int H = R.H, E = R.E, K = R.K;
    const int NB = gridDim.x, b = blockIdx.x, t = threadIdx.x;
    const StepLayer Ly = R.layers[l];
    {
        float xv[kNX];
        if (!getx(xv)) return false;
        stamp(l, 15);
        float ss = 0.f, dp = 0.f;
#pragma unroll
        for (int k = 0; k < kNX; ++k) {
            ss = __builtin_fmaf(xv[k], xv[k], ss);
            dp = __builtin_fmaf(router_weight<RDT>(pf.rw[k]), xv[k] * pf.nw[k], dp);
        }
        const float2 sums = block_sum2(ss, dp, S.part);
        const float inv = 1.0f / sqrtf(sums.x / (float)H + R.eps);
        if (b < E && t < kLR) {   // one copy per logit replica
            float p = sums.y * inv;
            if constexpr (RDT == MH_DT_Q8R) p *= pf.rs;
            st_tag(R.lw + (size_t)t * R.lws + b, ltag, p + pf.rb);
        }
#pragma unroll
        for (int k = 0; k < kNX; ++k) {
            const int i = t + k * kThreads;
            if (i < H) {
                S.xs[i] = xv[k];
                S.xbs[(i >> 5) * 33 + (i & 31)] = xv[k] * inv * pf.nw[k];
            }
        }
    }
    __syncthreads();
    // router rows beyond the grid (more experts than blocks): over xb
    constexpr int RE = mh_chunk<RDT>::E;   // elements per router chunk (16 int8 / 4 f32)
    const int CR = H / RE;
    for (int e = b + NB; e < E; e += NB) {
        float p = 0.f;
        const rsrc_t rw = make_rsrc(Ly.router_w, (uint32_t)E * (uint32_t)CR * 16u);
        for (int c = t; c < CR; c += kThreads) {
            const mh_u4 q = ld_w16(rw, (uint32_t)(e * CR + c) * 16u);
            const int i0 = c * RE;   // a router chunk lies inside one 32-element group
            p += mh_dot_chunk<RDT>(q, S.xbs + (i0 >> 5) * 33 + (i0 & 31));
        }
        p = block_sum(p, S.part);
        if (t < kLR) {
            if constexpr (RDT == MH_DT_Q8R) p *= Ly.router_s[e];
            st_tag(R.lw + (size_t)t * R.lws + e, ltag, p + Ly.router_b[e]);
        }
    }
    stamp(l, 1);
    bool late = false;
    if (t < 64) {
        const int lane = t;
        const int tt = opaque(t);
        uint64_t *lr = R.lw + (size_t)(b % kLR) * R.lws;
        uint64_t wv[kEL];
#pragma unroll
        for (int j = 0; j < kEL; ++j) {
            const int e = tt + 64 * j;
            wv[j] = e < E ? ld_tag(lr + e) : (uint64_t)ltag << 32;
        }
        for (unsigned spins = 0;; ++spins) {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < kEL; ++j) ready = ready && tag_is(wv[j], ltag);
            if (__all(ready)) break;
            if (spins > kSpinLimit) {
                late = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < kEL; ++j) {
                const int e = tt + 64 * j;
                if (e < E && !tag_is(wv[j], ltag)) wv[j] = ld_tag(lr + e);
            }
        }
        if (b == 0) stamp(l, 16);
        float v[kEL], v0[kEL];
#pragma unroll
        for (int j = 0; j < kEL; ++j) {
            v[j] = lane + 64 * j < E ? __uint_as_float((uint32_t)wv[j]) : -INFINITY;
            v0[j] = v[j];
        }
        int my_sel;
        float my_val;
        if (split) {
            // slots 0 .. upto only: the block's own expert (S.sel[upto]); the
            // rest after the caller has issued its weight loads
            wave_topk(v, upto + 1, &my_sel, &my_val);
            if (lane == upto) S.sel[opaque(lane)] = my_sel;
#pragma unroll
            for (int j = 0; j < kEL; ++j) {
                split->v[j] = v[j];
                split->v0[j] = v0[j];
            }
            split->sel = my_sel;
            split->val = my_val;
        }
        if (!split) wave_topk(v, K, &my_sel, &my_val);
        if (b == 0) stamp(l, 17);
        const float my_w = split ? 0.f : wave_weight(v0, K, R.router_norm, my_val);
        if (b == 0) stamp(l, 18);
        if (lane < K && !split) {
            // (addresses from an opaque lane: recomputed here, not hoisted
            // out of the layer loop and spilled)
            const int ln = opaque(lane);
            S.sel[ln] = my_sel;
            S.w[ln] = my_w;
            if (b == 0) {
                if (R.sel) R.sel[(size_t)l * K + ln] = my_sel;
                if (R.w) R.w[(size_t)l * K + ln] = my_w;
                if (R.usage && my_sel >= 0)
                    __hip_atomic_fetch_add(&R.usage[(size_t)l * E + my_sel], 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (__syncthreads_or(late)) {
        if (t == 0) raise_err(R.err);
        return false;
    }
    return true;
}

// ---------------------------------------------------------------- MFMA
// The down projection of k_decode_grp runs on V_MFMA_F32_16X16X32_F16
// (measured layout on gfx950: lane l holds A row l % 16 and B column l % 16,
// 8 consecutive K values 8 (l / 16) .. +7 each; output lane l holds column
// l % 16 of rows 4 (l / 16) + i).
//   A  16 of the block's down rows, e2m1 converted to f16 with the chunk's
//      power-of-two scale, which is exact (the plan scans every scale)
//   B  h as two f16 terms (hi = h rounded, lo = h - hi rounded: within
//      2^-22 |h|) in columns 0 and 1; the other columns are zero
// A K step of 128 = 4 lane groups x 32 takes one 16-byte MXFP4 chunk per
// lane group: lane (m, g) converts dword j of its chunk for the step's j-th
// MFMA, and B lane (n, g) supplies elements 8 j .. 8 j + 7 of the same chunk.
// The weights cannot be loaded in this lane layout directly (16 rows x 64 B
// per instruction streams from HBM ~25% slower than whole rows), so they are
// loaded as whole rows and staged through LDS.
// One wave's share of the down projection: the K steps q = kQ wave .. +kQ
// (128 columns each) of the block's down rows [0, rows), staged in LDS at a
// stride of SD chunks (sw; their f16 scales ss at a stride of CF), times the
// wave's h terms hp
// ([2][kQ * 128] f16: hi, lo of columns 128 kQ wave + ...), NT = ceil(rows /
// 16) row tiles. Row rho's partial (the hi and lo columns summed) goes to
// out[rho].
template <int NT>
__device__ __forceinline__ void dn_mfma_grp(const uint8_t *sw, const uint16_t *ss, const _Float16 *hp, int SD, int CF,
                                            int rows, float *out) {
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
        v8h hb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hb[j] = m < 2 ? *(const v8h *)(hp + m * (kQ * 128) + 128 * u + 32 * g + 8 * j) : v8h{};
        mh_u4 qa[NT];
        float sc[NT];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            const int row = min(16 * rt + m, rows - 1);
            qa[rt] = *(const mh_u4 *)(sw + (size_t)(row * SD + c) * 16);
            sc[rt] = mh_f16(ss[row * CF + c]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp4x8_f16(dword_of(qa[rt], j), sc[rt]), hb[j], acc[rt],
                                                                 0, 0, 0);
    }
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const float v = acc[rt][ii];
            const float v1 = dpp_shl<1>(v);
            const int rho = 16 * rt + 4 * g + ii;
            if (rho < rows && m == 0) out[rho] = v + v1;
        }
    }
}

// ------------------------------------------------------- k_decode_grp

// GV: the routing is given (A.gxb, A.gsel, A.gw; one layer), a separate
// instantiation so that the routed kernel's registers are unaffected.
template <int RDT, bool GV>
__global__ void __launch_bounds__(kThreads) k_decode_grp(GrpArgs A) {
    // LDS is static (capacities are checked at plan creation).
    __shared__ float s_part[16];
    __shared__ int s_sel[kMaxK];
    __shared__ float s_w[kMaxK];
    __shared__ __attribute__((aligned(16))) float s_xs[kHMax];
    __shared__ __attribute__((aligned(16))) float s_xbs[kHMax / 32 * 33];
    __shared__ __attribute__((aligned(16))) float s_res[kResMax];
    // the gate/up partial sums, then (once they are reduced) the down rows
    __shared__ __attribute__((aligned(16))) uint8_t s_big[kGrpBig];
    // the block's f16 scales: gate rows, up rows, down rows (3 windows)
    __shared__ __attribute__((aligned(16))) uint8_t s_sc[3 * kScW];
    __shared__ __attribute__((aligned(16))) _Float16 s_hp[kThreads / 64][2 * kQ * 128];
    __shared__ float s_dred[kThreads / 64 * kRBMax];
    __shared__ float s_bd[kRBMax];
    __shared__ float s_y[kMaxGrpK * kRBMax];   // the last layer's combine: y_i of the block's rows
    const RouteArgs &R = A.R;
    const int H = R.H, F = A.F, K = R.K;
    const int b = blockIdx.x, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    // (Numbering the blocks so that each XCD runs a contiguous range of
    // slots and rows was measured 2-3% slower than this plain order.)
    const int NB = (int)gridDim.x, n = b;
    const int slot = n / A.G, gi = n - slot * A.G;
    const int p0 = A.PB * gi, np = max(0, min(F - p0, A.PB));
    const int r0 = A.RB * gi, nr = max(0, min(H - r0, A.RB));   // >= 1 (plan check)
    const Stamper stamp{(R.trace && t == 0) ? R.trace + b : nullptr, (int)gridDim.x};
    const RouteLds S{s_part, s_sel, s_w, s_xs, s_xbs};
    const uint32_t layer_bytes = (uint32_t)((uint64_t)R.E * A.stride - 1u) + 1u;   // < 4 GiB (plan check)
    uint64_t *hsrc = A.hw + (size_t)((gi % kHR) * K + slot) * A.hws;
    const size_t ycopy = (size_t)K * A.yws;   // words between copies of y
    for (int l = 0; l < R.n_layers; ++l) {
        const StepLayer Ly = R.layers[l];
        // sequence numbers of this layer: logits, h, y (the fourth is unused)
        const unsigned tagL = A.seq0 + 4u * (unsigned)l, tagH = tagL + 1u, tagY = tagL + 2u;
        stamp(l, 0);
        RankState rks;   // the ranking wave's state (routed launches)
        // routing given: this thread's xb elements t + k kThreads (stored to
        // LDS once the weight loads are issued) and, in a slot-0 block, x of
        // its row for the combine
        float gxv[GV ? kNG : 1];
        float gx0 = 0.f;
        if constexpr (GV) {
            // expert_apply with the routing given (no norm, no router); a slot
            // whose expert is out of range is unfilled. x is read and written
            // only by the combine, each element by one block, so no block
            // waits for another's reads. The selection is loaded first: the
            // barrier then waits for it alone, and xb and x arrive while the
            // weight loads are issued.
            const int tk = min(t, K - 1);
            const int ge = A.gsel[tk];
            const float gwv = A.gw[tk];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < kNG; ++k) gxv[k] = A.gxb[min(t + k * kThreads, H - 1)];
            if (slot == 0) gx0 = R.x[r0 + min(t, nr - 1)];
            __builtin_amdgcn_sched_barrier(0);
            if (t < K) {
                s_sel[t] = ge >= 0 && ge < R.E ? ge : -1;
                s_w[t] = gwv;
            }
            __syncthreads();
        } else {
            // x (l): R.x at layer 0, else x (l - 1) + moe (l - 1) with moe =
            // sum_i w_i y_i in selection order, each product and sum rounded
            // on its own (engine/midge.c:544-548), from the y words every
            // block published (layer l - 1's parity, copy n % kYR). Every
            // block forms the same x from the same words with the previous
            // layer's selection and weights (still in LDS).
            auto getx = [&](float (&xv)[kNX]) __attribute__((always_inline)) {
                if (l == 0) return gather_x_tagged(R, 0, nullptr, 0u, xv);
                const uint32_t nib = ynib(A.bank, l - 1);
                const uint32_t *ys = A.yw + (size_t)(((l - 1) & 1) * kYR + n % kYR) * ycopy;
                // (branch-free: slots past K and elements past H re-read the
                // last slot's last element, a word of this layer)
                const int tt = opaque(t);
                auto yaddr = [&](int s, int k) __attribute__((always_inline)) {
                    return ys + (size_t)min(s, K - 1) * A.yws + min(tt + k * kThreads, H - 1);
                };
                uint32_t yv[kMaxGrpK][kNG];
#pragma unroll
                for (int s = 0; s < kMaxGrpK; ++s)
#pragma unroll
                    for (int k = 0; k < kNG; ++k) yv[s][k] = ld_u32_dev(yaddr(s, k));
                bool late = false;
                for (unsigned spins = 0;; ++spins) {
                    bool ready = true;
#pragma unroll
                    for (int s = 0; s < kMaxGrpK; ++s)
#pragma unroll
                        for (int k = 0; k < kNG; ++k) ready = ready && (yv[s][k] & 15u) == nib;
                    if (ready) break;
                    if (spins > kSpinLimit) {
                        late = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int k = 0; k < kNG; ++k) {   // an element's K words are re-read together
                        bool rd = true;
#pragma unroll
                        for (int s = 0; s < kMaxGrpK; ++s) rd = rd && (yv[s][k] & 15u) == nib;
                        if (!rd) {
#pragma unroll
                            for (int s = 0; s < kMaxGrpK; ++s) yv[s][k] = ld_u32_dev(yaddr(s, k));
                        }
                    }
                }
                if (__syncthreads_or(late)) {
                    if (t == 0) raise_err(R.err);
                    return false;
                }
#pragma unroll
                for (int k = 0; k < kNX; ++k) {
#pragma clang fp contract(off)
                    const int i = t + k * kThreads;
                    float moe = 0.f;
                    if (k < kNG) {
#pragma unroll
                        for (int s = 0; s < kMaxGrpK; ++s)
                            if (s < K && s_sel[s] >= 0) moe = moe + s_w[s] * y_val(yv[s][min(k, kNG - 1)]);
                    }
                    xv[k] = i < H ? s_xs[min(i, H - 1)] + moe : 0.f;
                }
                return true;
            };
            // the router row's loads are issued here and land while x is on
            // its way (held across the layer they would cost 18 registers)
            const RouterPref pf = prefetch_router<RDT>(R, l);
            if (!route_layer<RDT>(R, pf, l, getx, tagL, S, stamp, &rks, slot)) return;
        }
        // x (0) read: the last layer's combine overwrites R.x only once every
        // block has raised this flag
        if (l == 0 && R.n_layers == 1 && t == 0 && !GV)
            __hip_atomic_store(&A.flags[b], A.seq0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        stamp(l, 2);
        const int e = s_sel[slot];   // block-uniform
        // A slot with nothing routed (fewer than k logits above -1e30) skips
        // the h exchange and publishes y = 0. Every block gathers every
        // block's y at the next layer's start, which orders the reuse of the
        // exchange buffers (the logits, h, and y of the same parity) from
        // layer to layer.
        float y = 0.f;               // row t of this slot's y (t < nr)
        if (e >= 0) {
            const rsrc_t rex = make_rsrc(Ly.experts, layer_bytes);
            const uint32_t eo = (uint32_t)e * (uint32_t)A.stride;
            const int tt = opaque(t);
            // -------------------------------------- B: every load at once
            // gate/up: thread (slot gs, chunk c) takes pairs pp = u ns + gs
            // (whole rows per instruction: a wave reads 1 KB of contiguous
            // row); past-the-end pairs and idle slots re-read the last pair
            // and are masked out in the math
            const int C = A.CH, ns = kThreads / C;
            const int gs = tt / C, c = tt - gs * C;
            const bool gact = gs < ns;
            const int gsl = gact ? gs : ns - 1;
            const int plast = max(np - 1, 0);
            float xr[32];   // this thread's chunk of xb (read from LDS once the loads are issued)
            // the scales first: the block's gate, up and down scale rows are
            // three contiguous ranges, loaded as 16-byte chunks of their
            // aligned windows (mis: the range's offset in its window)
            const int CD = A.CF;
            const uint32_t sa0 = eo + (uint32_t)A.off[1] + (uint32_t)(p0 * C) * 2u;
            const uint32_t sa1 = eo + (uint32_t)A.off[4] + (uint32_t)(p0 * C) * 2u;
            const uint32_t sa2 = eo + (uint32_t)A.off[7] + (uint32_t)(r0 * CD) * 2u;
            const int mis0 = (int)(sa0 & 15u), mis1 = (int)(sa1 & 15u), mis2 = (int)(sa2 & 15u);
            const int n0 = (mis0 + np * C * 2 + 15) >> 4, n1 = (mis1 + np * C * 2 + 15) >> 4;
            const int n2 = (mis2 + nr * CD * 2 + 15) >> 4;
            mh_u4 qs[kScLoads];
#pragma unroll
            for (int k = 0; k < kScLoads; ++k) {
                const int q = tt + kThreads * k;
                const uint32_t a = q < n0 ? (sa0 & ~15u) + (uint32_t)q * 16u
                                 : q < n0 + n1 ? (sa1 & ~15u) + (uint32_t)(q - n0) * 16u
                                               : (sa2 & ~15u) + (uint32_t)min(q - n0 - n1, n2 - 1) * 16u;
                qs[k] = ld_w16(rex, a);
            }
            // gate/up pairs in flight: kPD per thread, pair u + kPD issued
            // after pair u's math (loads complete in issue order, and a
            // wave's first loads complete only when its last do if all of
            // the layer's loads are in flight at once: the depth lets the
            // math run as the stream arrives)
            mh_u4 qg[kUP], qu[kUP];
            const uint32_t og = eo + (uint32_t)A.off[0], ou = eo + (uint32_t)A.off[3];
            auto issue_gu = [&](int u) __attribute__((always_inline)) {
                const uint32_t rc = (uint32_t)((p0 + min(u * ns + gsl, plast)) * C + c);
                qg[u] = ld_w16(rex, og + rc * 16u);
                qu[u] = ld_w16(rex, ou + rc * 16u);
            };
#pragma unroll
            for (int u = 0; u < kPD; ++u) issue_gu(u);
            const uint32_t pb4 = (uint32_t)(p0 + min(t, plast)) * 4u;
            const float bg = ld_f(rex, eo + (uint32_t)A.off[2] + pb4);
            const float bu = ld_f(rex, eo + (uint32_t)A.off[5] + pb4);
            __builtin_amdgcn_sched_barrier(0);
            stamp(l, 9);
            // the other slots' experts and the weights, while the loads fly
            if constexpr (!GV) route_finish(R, l, S, rks, slot);
            // the scale windows into LDS (their loads were issued first, so
            // they complete first)
#pragma unroll
            for (int k = 0; k < kScLoads; ++k) {
                const int q = tt + kThreads * k;
                const int o = q < n0 ? q * 16 : q < n0 + n1 ? kScW + (q - n0) * 16 : 2 * kScW + (q - n0 - n1) * 16;
                if (q < n0 + n1 + n2) *(mh_u4 *)(s_sc + o) = qs[k];
            }
            if constexpr (GV) {
#pragma unroll
                for (int k = 0; k < kNG; ++k) {
                    const int i = t + k * kThreads;
                    if (i < H) s_xbs[(i >> 5) * 33 + (i & 31)] = gxv[k];
                }
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < 32; ++j) xr[j] = gact ? s_xbs[c * 33 + j] : 0.f;
            const uint16_t *scg = (const uint16_t *)(s_sc + mis0), *scu = (const uint16_t *)(s_sc + kScW + mis1);
            // gate/up math as the data arrives, each pair's math followed by
            // the next pair's loads and, once those are all issued, by the
            // down rows (needed only after the h exchange), so that a load
            // whose issue waits for room in the memory pipeline holds up no
            // math whose data is in. Down row j = u nsd + ds is thread (slot
            // ds, chunk dc)'s (whole rows per instruction).
            const int nsd = kThreads / CD;
            const int ds = tt / CD, dc = tt - ds * CD;
            const bool dact = ds < nsd;
            const int dsl = dact ? ds : nsd - 1;
            const uint32_t od = eo + (uint32_t)A.off[6];
            mh_u4 qd[kUD];
            float *red = (float *)s_big;
#pragma unroll
            for (int u = 0; u < kUP; ++u) {
                const int pp = u * ns + gs;
                const bool inr = gact && pp < np;
                const int so = min(pp, plast) * C + c;
                const float gv = mh_dot_mxfp4(qg[u], xr) * (inr ? mh_f16(scg[so]) : 0.f);
                const float uv = mh_dot_mxfp4(qu[u], xr) * (inr ? mh_f16(scu[so]) : 0.f);
                if (inr) {
                    red[(2 * pp) * C + c] = gv;
                    red[(2 * pp + 1) * C + c] = uv;
                }
                if (u + kPD < kUP) issue_gu(u + kPD);
                if (u >= kUP - kPD) {
                    const int i = u - (kUP - kPD);
#pragma unroll
                    for (int d = i * kUD / kPD; d < (i + 1) * kUD / kPD; ++d) {
                        const uint32_t rc = (uint32_t)((r0 + min(d * nsd + dsl, nr - 1)) * CD + dc);
                        qd[d] = ld_w16(rex, od + rc * 16u);
                    }
                }
                if (u == 0) stamp(l, 19);
                if (u == kUP / 2) stamp(l, 20);
                __builtin_amdgcn_sched_barrier(0);   // one pair's math at a time
            }
            const float bdv = ld_f(rex, eo + (uint32_t)A.off[8] + (uint32_t)(r0 + min(t, nr - 1)) * 4u);
            stamp(l, 10);
            if (R.trace && t == kThreads - 64) R.trace[(size_t)(l * kStamps + 21) * gridDim.x + b] = wall_clock64();
            __syncthreads();
            stamp(l, 22);
            block_reduce_rows(red, C, 2 * np, kThreads / 64, s_res, [](int) { return true; });
            __syncthreads();
            stamp(l, 11);
            // epilogue (np <= 64: one pair per lane of wave 0): bias, clamped
            // SwiGLU (engine/midge.c:531-538), h as two f16 terms, published
            // in kHR copies for the slot's group
            if (t < np) {
                const float hv = act_fn(s_res[2 * t] + bg, s_res[2 * t + 1] + bu, A.alpha, A.limit, 0);
                const _Float16 hi = (_Float16)hv;
                const _Float16 lo = (_Float16)(hv - (float)hi);
                const uint32_t pay = (uint32_t)__builtin_bit_cast(uint16_t, hi) |
                                     ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
#pragma unroll
                for (int cp = 0; cp < kHR; ++cp)
                    st_tag_u(A.hw + (size_t)(cp * K + slot) * A.hws + p0 + t, tagH, pay);
            }
            stamp(l, 3);
            // -------------------------------------- C: down
            // this wave's part of h: its K steps read columns [kb, kb + 128 kQ)
            const int kb = kQ * 128 * wave;
            uint64_t hv[2 * kQ];
#pragma unroll
            for (int m2 = 0; m2 < 2 * kQ; ++m2) {
                const int k = kb + lane + 64 * m2;
                hv[m2] = k < F ? ld_tag(hsrc + k) : (uint64_t)tagH << 32;
            }
            // stage the down rows while h is on its way: row j of the slice at
            // a stride of SD chunks (odd: the matrix-core lanes' 16 rows fall
            // in distinct banks); s_big's partial sums are reduced already
            const int SD = CD | 1;
            if (dact) {
#pragma unroll
                for (int u = 0; u < kUD; ++u) {
                    const int j = u * nsd + ds;
                    if (j < nr) *(mh_u4 *)(s_big + (size_t)(j * SD + dc) * 16) = qd[u];
                }
            }
            if (t < nr) s_bd[t] = bdv;
            stamp(l, 4);
            __syncthreads();   // the staged rows are visible to every wave
            bool late = false;
            for (unsigned spins = 0;; ++spins) {
                bool ready = true;
#pragma unroll
                for (int m2 = 0; m2 < 2 * kQ; ++m2) ready = ready && tag_is(hv[m2], tagH);
                if (ready) break;
                if (spins > kSpinLimit) {
                    late = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int m2 = 0; m2 < 2 * kQ; ++m2) {
                    const int k = kb + lane + 64 * m2;
                    if (k < F && !tag_is(hv[m2], tagH)) hv[m2] = ld_tag(hsrc + k);
                }
            }
            // the wave's h terms into its LDS planes (zeros past F); a wave's
            // LDS accesses are performed in order, so its lanes read these
            // after the writes without a block barrier
            _Float16 *hp = s_hp[wave];
#pragma unroll
            for (int m2 = 0; m2 < 2 * kQ; ++m2) {
                const uint32_t pv = (uint32_t)hv[m2];
                hp[lane + 64 * m2] = __builtin_bit_cast(_Float16, (uint16_t)(pv & 0xFFFFu));
                hp[kQ * 128 + lane + 64 * m2] = __builtin_bit_cast(_Float16, (uint16_t)(pv >> 16));
            }
            __builtin_amdgcn_wave_barrier();
            if (wave == 0) stamp(l, 5);
            if (!late) {
                const uint16_t *scd = (const uint16_t *)(s_sc + 2 * kScW + mis2);
                switch ((nr + 15) >> 4) {   // block-uniform (plan check: nr <= 16 * 3)
                case 1: dn_mfma_grp<1>(s_big, scd, hp, SD, CD, nr, s_dred + wave * kRBMax); break;
                case 2: dn_mfma_grp<2>(s_big, scd, hp, SD, CD, nr, s_dred + wave * kRBMax); break;
                case 3: dn_mfma_grp<3>(s_big, scd, hp, SD, CD, nr, s_dred + wave * kRBMax); break;
                default: break;
                }
            }
            if (wave == 0) stamp(l, 13);
            if (__syncthreads_or(late)) {
                if (t == 0) raise_err(R.err);
                return;
            }
            if (t < nr) {
                float sum = 0.f;
#pragma unroll
                for (int w = 0; w < kThreads / 64; ++w) sum += s_dred[w * kRBMax + t];
                y = sum + s_bd[t];   // the matvec, then wk_addbias (engine/midge.c:539-541)
            }
        } else if constexpr (!GV) {
            route_finish(R, l, S, rks, slot);
            __syncthreads();   // the selection and weights before any later read
        }
        // -------------------------------------- D: y
        // every block publishes its rows of its slot's y (0 for a slot with
        // nothing routed): in kYR copies of the layer's parity, or, in a
        // one-layer launch, as tagged words read only by the slot-0 block of
        // the same rows
        const uint32_t nibY = ynib(A.bank, l);
        const bool one = R.n_layers == 1;
        const uint32_t ymine = y_word(y, nibY);
        if (t < nr) {
            if (!one) {
                uint32_t *yd = A.yw + (size_t)((l & 1) * kYR) * ycopy + (size_t)slot * A.yws + r0;
#pragma unroll
                for (int cp = 0; cp < kYR; ++cp) st_u32_dev(yd + (size_t)cp * ycopy + t, ymine);
            } else if (slot > 0) {
                st_tag(A.y1 + (size_t)slot * A.yws + r0 + t, tagY, y);
            }
        }
        stamp(l, 14);
        // the last layer's combine (slot 0 of each row slice): x (L) = x (L - 1)
        // + moe (its own slot's y from registers), written to R.x once every
        // block has read x (0) from there: in a launch of several layers every
        // block's y of the layer before shows it; in a one-layer launch the
        // flags every block raised after reading x (0). The y words of a
        // launch of several layers are rounded as its gathers see them.
        if (l + 1 == R.n_layers && slot == 0) {
            bool late = false;
            const int tq = opaque(t);
            const int iq = tq / kRBMax, jq = tq - iq * kRBMax;
            const bool hasy = iq >= 1 && iq < K && jq < nr;
            const uint32_t *yp = A.yw + (size_t)((l & 1) * kYR) * ycopy + (size_t)iq * A.yws + r0 + jq;
            uint64_t *yq = A.y1 + (size_t)iq * A.yws + r0 + jq;
            auto ready = [&](uint64_t w) { return one ? tag_is(w, tagY) : ((uint32_t)w & 15u) == nibY; };
            auto load = [&]() { return one ? ld_tag(yq) : (uint64_t)ld_u32_dev(yp); };
            uint64_t yw = hasy ? load() : (one ? (uint64_t)tagY << 32 : (uint64_t)nibY);
            const bool wflags = one && !GV;   // x (0) read by every block (routed one-layer launches)
            bool up = true;
            if (wflags)
                for (int i = tq; i < NB; i += kThreads)
                    up = up && __hip_atomic_load(&A.flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == A.seq0;
            for (unsigned spins = 0; !ready(yw) || !up; ++spins) {
                if (spins > kSpinLimit) {
                    late = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (!ready(yw)) yw = load();
                up = true;
                if (wflags)
                    for (int i = tq; i < NB; i += kThreads)
                        up = up && __hip_atomic_load(&A.flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == A.seq0;
            }
            if (hasy) s_y[iq * kRBMax + jq] = one ? __uint_as_float((uint32_t)yw) : y_val((uint32_t)yw);
            if (t < nr) s_y[t] = one ? y : y_val(ymine);
            if (__syncthreads_or(late)) {
                if (t == 0) raise_err(R.err);
                return;
            }
            if (t < nr && GV) {
#pragma clang fp contract(off)
                // routing given: each slot's w_i y_i added into x in ascending
                // expert order, slot order among equal ids (the expert-major
                // loop, engine/midge.c:595-611, with expert_apply's
                // x_out += weight * moe, midge.c:465-466)
                float acc = gx0;
                int prev = -1;
                for (int n2 = 0; n2 < K; ++n2) {
                    int best = 0x7fffffff;
                    for (int i = 0; i < K; ++i) {
                        const int key = s_sel[i] * kMaxGrpK + i;
                        if (s_sel[i] >= 0 && key > prev && key < best) best = key;
                    }
                    if (best == 0x7fffffff) break;
                    prev = best;
                    const int i = best % kMaxGrpK;
                    acc = acc + s_w[i] * s_y[i * kRBMax + t];
                }
                st_dev(R.x + r0 + t, acc);
            } else if (t < nr) {
#pragma clang fp contract(off)
                float moe = 0.f;
                for (int i = 0; i < K; ++i) {
                    if (s_sel[i] < 0) continue;
                    moe = moe + s_w[i] * s_y[i * kRBMax + t];
                }
                st_dev(R.x + r0 + t, s_xs[r0 + t] + moe);
            }
        }
        stamp(l, 6);
        stamp(l, 7);
    }
}

// ------------------------------------------------------ k_decode_step

template <int RDT, int XDT>
__global__ void __launch_bounds__(kThreads) k_decode_step(StepArgs A) {
    constexpr int XE = mh_chunk<XDT>::E;   // elements per expert chunk (32)
    // LDS is static (capacities are checked at plan creation).
    __shared__ float s_part[16];
    __shared__ int s_sel[kMaxK];
    __shared__ float s_w[kMaxK];
    __shared__ int s_ok;
    __shared__ __attribute__((aligned(16))) float s_xs[kHMax];
    __shared__ __attribute__((aligned(16))) float s_xbs[kHMax / 32 * 33];
    __shared__ __attribute__((aligned(16))) float s_res[kResMax];    // reduced rows
    __shared__ __attribute__((aligned(16))) float s_red[kRedMax];    // partial sums
    __shared__ __attribute__((aligned(16))) float s_bds[kThreads];   // [K][rows of this block's down slice]
    const RouteArgs &R = A.R;
    const int H = R.H, F = A.F, K = R.K;
    float *res = s_res, *red = s_red, *bds = s_bds;
    const int NB = gridDim.x, b = blockIdx.x, t = threadIdx.x;
    const Stamper stamp{(R.trace && t == 0) ? R.trace + b : nullptr, NB};
    const RouteLds S{s_part, s_sel, s_w, s_xs, s_xbs};
    const rsrc_t rh = make_rsrc(A.h, (uint32_t)K * (uint32_t)F * 4u);
    const uint32_t layer_bytes = (uint32_t)((uint64_t)R.E * A.stride - 1u) + 1u;   // < 4 GiB (plan check)
    RouterPref pf = prefetch_router<RDT>(R, 0);
    for (int l = 0; l < R.n_layers; ++l) {
        const StepLayer Ly = R.layers[l];
        // sequence numbers of this layer: logits, the barrier before the down
        // phase, x for the next layer
        const unsigned tagA = A.seq0 + 3u * (unsigned)l, tagB = tagA + 1u, tagC = tagA + 2u;
        stamp(l, 0);
        auto getx = [&](float (&xv)[kNX]) __attribute__((always_inline)) {
            return gather_x_tagged(R, l, A.xw, tagA - 1u, xv);
        };
        if (!route_layer<RDT>(R, pf, l, getx, tagA, S, stamp)) return;
        stamp(l, 2);

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
            for (int j = 0; j < XE; ++j) xr[j] = active ? s_xbs[c * 33 + j] : 0.f;
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
            stamp(l, 9);
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
            stamp(l, 10);
            {
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
            stamp(l, 11);
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
        stamp(l, 3);
        bar_arrive(A.flags, tagB);

        // ------------------------------------------------ C: down + combine
        {
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
            stamp(l, 4);
            if (!bar_wait(A.flags, A.go, tagB, R.err, &s_ok)) return;
            stamp(l, 5);
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
            stamp(l, 12);
#pragma unroll
            for (int u = 0; u < kUC; ++u) {
                const int j = sub + spe * u;
                const bool valid = e >= 0 && j < nr;
                const float p = mh_dot_chunk<XDT>(qd[u], xr) * (valid ? mh_f16((uint16_t)sd[u]) : 0.f);
                if (act && j < nr) red[(i * RC + j) * C + c] = p;
                __builtin_amdgcn_sched_barrier(0);
            }
            if (t < K * nr) bds[t] = bd_pref;
            stamp(l, 13);
            __syncthreads();
            block_reduce_rows(red, C, K * RC, kThreads / 64, res, [&](int it) { return it % RC < nr; });
            __syncthreads();
            stamp(l, 14);
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
                if (l + 1 < R.n_layers) st_tag(A.xw + r, tagC, s_xs[r] + moe);
                else st_dev(R.x + r, s_xs[r] + moe);
            }
        }
        stamp(l, 6);
        if (l + 1 < R.n_layers) pf = prefetch_router<RDT>(R, l + 1);
        stamp(l, 7);
    }
}

__global__ void k_fill_u32(unsigned *p, int n, unsigned v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// Flags (bit) an MXFP4 scale that the f16 matrix-core paths cannot apply
// exactly: it must be zero or a power of two in [2^-23, 2^13], so that every
// e2m1 value times it is an f16.
__global__ void k_scan_scales(const uint8_t *experts, uint64_t stride, uint64_t od, int n, unsigned *bad,
                              unsigned bit) {
    const uint16_t *d = (const uint16_t *)(experts + (uint64_t)blockIdx.y * stride + od);
    bool ok = true;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned v = d[i], e = (v >> 10) & 31u, mn = v & 1023u;
        ok = ok && ((v & 0x7FFFu) == 0 || (e == 0 && mn >= 2 && (mn & (mn - 1)) == 0) || (e != 0 && e <= 28 && mn == 0));
    }
    if (!ok) atomicOr(bad, bit);
}

// Launch of a one-launch step: nb blocks of kThreads. Every block must be
// resident at once (the blocks wait on each other): the plan sizes the grid
// to at most one block per CU, and the occupancy is checked here (the query
// once per device and kernel: it costs host time comparable to a small
// step). A plain launch is the default; the COOP switch makes it a
// cooperative launch, whose runtime check of co-residency costs ~18 us of
// device time per call. A block that were not resident would make the grid's
// bounded waits time out and report an error through mh_sync, never hang.
template <class Args>
int launch_step(const void *k, const Args &A, int nb, hipStream_t s, int *ready_dev, int *per_cu) {
    int dev = 0;
    MH_HIP(hipGetDevice(&dev));
    if (dev != *ready_dev) {
        MH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k, kThreads, 0));
        *ready_dev = dev;
    }
    if (*per_cu < 1) return fail(MH_E_UNSUPPORTED, "decode step: a %d-thread block does not fit a CU", kThreads);
    Args a = A;
    void *args[] = {&a};
    const bool prof = profiling();
    if (prof) prof_begin("decode_step", s);
    hipError_t e;
    if (sw(SW_COOP))
        e = hipLaunchCooperativeKernel(k, dim3(nb), dim3(kThreads), args, 0u, s);
    else
        e = hipLaunchKernel(k, dim3(nb), dim3(kThreads), args, 0u, s);
    if (prof) prof_end(s);
    return hip_check(e, "decode step launch");
}

template <int RDT, bool GV>
int launch_grp(const GrpArgs &A, int nb, hipStream_t s) {
    static int ready_dev = -1, per_cu = 0;
    return launch_step((const void *)k_decode_grp<RDT, GV>, A, nb, s, &ready_dev, &per_cu);
}

template <int RDT, int XDT>
int launch_flat(const StepArgs &A, int nb, hipStream_t s) {
    static int ready_dev = -1, per_cu = 0;
    return launch_step((const void *)k_decode_step<RDT, XDT>, A, nb, s, &ready_dev, &per_cu);
}

}  // namespace

// Barrier words: nb flags, then (from a 128-byte line) kGoCopies release
// words kGoStride apart.
static int go_offset(int nb) { return (nb + 63) / 32 * 32; }
static int flag_words(int nb) { return go_offset(nb) + kGoCopies * kGoStride; }
// Words between copies of an exchanged vector of n words: rounded up to 16
// words, plus 32 (copies start 256 B past a line boundary apart).
static int copy_stride(int n) { return (n + 15) / 16 * 16 + 32; }

// Scratch and tables a stack keeps for the one-launch paths.
struct StepPlan {
    StepLayer *layers = nullptr;   // device [L]
    unsigned *flags = nullptr;     // device [flag_words(nb)]: flags, then the release word's copies
    uint64_t *tagged = nullptr;    // device: exchanged words (tag_layout)
    size_t tagged_words = 0;
    unsigned long long *trace = nullptr;   // device [L][kStamps][nb] (filled while profiling)
    int n_layers = 0;
    unsigned *err = nullptr;       // host-mapped pinned [1]: set by a timed-out wait
    unsigned *err_dev = nullptr;   // its device address
    float *h = nullptr;            // device [K][F] (k_decode_step)
    unsigned seq = 0;              // next sequence number
    unsigned launches = 0;         // k_decode_grp launches of several layers so far (the y tags' bank)
    int nb = 0;                    // CUs: k_decode_step's grid
    int flat = 0;                  // 1 = k_decode_step can run the stack
    int grp = 0;                   // 1 = k_decode_grp can run the stack
    int G = 0, PB = 0, RB = 0;     // k_decode_grp's shape (grid G * K)
    int ok = 0;                    // 1 = one of the kernels is eligible
    int few = 0;                   // 1 = every MXFP4 scale is f16-exact (the expert-grouped kernels)
    char why[160] = {0};
    std::vector<std::pair<void *, uint64_t>> mem;   // device allocations (counted)
};

template <class T>
static int plan_alloc(StepPlan *p, T **out, uint64_t bytes, const char *what) {
    void *v = nullptr;
    MH_TRY(dev_alloc(&v, bytes, what));
    p->mem.push_back({v, bytes});
    *out = (T *)v;
    return MH_OK;
}

// Frees a plan's device and pinned memory; the plan stays ineligible. Called
// by step_plan_destroy, and by mh_shutdown for plans still alive.
static void plan_release(void *key) {
    StepPlan *p = (StepPlan *)key;
    for (auto &m : p->mem) dev_release(m.first, m.second);
    p->mem.clear();
    p->layers = nullptr;
    p->flags = nullptr;
    p->trace = nullptr;
    p->tagged = nullptr;
    p->h = nullptr;
    if (p->err) {
        unwatch_async_error(p->err);
        (void)hipHostFree(p->err);
    }
    p->err = p->err_dev = nullptr;
    p->flat = p->grp = p->ok = 0;
}

// Exchange-word layout in StepPlan::tagged (offsets in 64-bit words): the
// logits' kLR copies; x (k_decode_step); h's kHR x K planes (k_decode_grp);
// y's 2 parities x kYR copies x K rows of 32-bit words (k_decode_grp; yws
// in 32-bit words); y's K rows of tagged words for one-layer launches of
// k_decode_grp.
struct TagLayout {
    int lws, xws, hws, yws;
    size_t lw, xw, hw, yw, y1, total;
};
static TagLayout tag_layout(const DevLayer &L0) {
    TagLayout t;
    t.lws = copy_stride(L0.n_experts);
    t.xws = copy_stride((int)L0.hidden);
    t.hws = copy_stride((int)L0.ffn);
    t.yws = copy_stride((int)L0.hidden);
    t.lw = 0;
    t.xw = t.lw + (size_t)kLR * t.lws;
    t.hw = t.xw + (size_t)t.xws;
    t.yw = t.hw + (size_t)kHR * L0.top_k * t.hws;
    t.y1 = t.yw + ((size_t)2 * kYR * L0.top_k * t.yws + 1) / 2;
    t.total = t.y1 + (size_t)L0.top_k * t.yws;
    return t;
}

// k_decode_grp's grid for a shape: the largest G <= cus / K for which every
// block of a group owns at least one gate/up pair and one down row.
static bool grp_shape(int cus, int H, int F, int K, int *G, int *PB, int *RB) {
    for (int g = cus / K; g >= 1; --g) {
        const int pb = (F + g - 1) / g, rb = (H + g - 1) / g;
        if ((g - 1) * pb < F && (g - 1) * rb < H) {
            *G = g;
            *PB = pb;
            *RB = rb;
            return true;
        }
    }
    return false;
}

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
    if (L0.n_experts > 64 * kEL || L0.top_k > kMaxK) return reject("too many experts");
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
    const int H = (int)L0.hidden, F = (int)L0.ffn, K = L0.top_k;
    if (H > kNX * kThreads || H > kHMax) return reject("hidden exceeds the router phase's per-thread share");
    {
        // k_decode_step: a block's gate/up pairs span at most two experts and
        // the epilogue has one pair per thread; the down phase is one pass in
        // which every routed expert gets slots, each slot's rows of the
        // block's slice fit kUC iterations, one bias per thread
        const int PB = (K * F + nb - 1) / nb;
        const int nsC = kThreads / (F / 32);
        const int spe = K > 0 ? nsC / K : 0;
        const int RC = (H + nb - 1) / nb;
        const int res = std::max(64 * kEL, std::max(2 * PB, K * RC)) + 64;
        const int red = std::max(2 * (kThreads / (H / 32)) * kUP * (H / 32), K * RC * (F / 32));
        p->flat = PB <= F && PB <= kThreads && PB <= (kThreads / (H / 32)) * kUP && spe >= 1 && RC <= spe * kUC &&
                  K * RC <= kThreads && res <= kResMax && red <= kRedMax;
    }
    {
        // k_decode_grp: MXFP4 experts, the clamped SwiGLU (|h| <= limit (limit
        // + 1) fits f16), every block's pairs in one pass and its rows in the
        // matrix-core tiles, exact f16 down scales (scanned below)
        const float lim = L0.limit;
        int G = 0, PB = 0, RB = 0;
        bool ok = L0.expert_dt == MH_DT_MXFP4 && !L0.act_plain && lim >= 0.f && lim * (lim + 1.f) < 60000.f &&
                  F <= kKPad && K <= kMaxGrpK && grp_shape(nb, H, F, K, &G, &PB, &RB);
        if (ok) {
            const int CH = H / 32, CF = F / 32;
            ok = PB <= (kThreads / CH) * kUP && PB <= 64 && 2 * PB <= kResMax - 64 && 2 * PB * CH <= kRedMax &&
                 RB <= (kThreads / CF) * kUD && RB <= kRBMax && RB * (CF | 1) <= kRBMax * kSDMax &&
                 PB * CH * 2 + 16 <= kScW && RB * CF * 2 + 16 <= kScW &&
                 2 * ((PB * CH * 2 + 30) / 16) + (RB * CF * 2 + 30) / 16 <= kScLoads * kThreads;
        }
        p->grp = ok ? 1 : 0;
        p->G = G;
        p->PB = PB;
        p->RB = RB;
    }
    if (!p->flat && !p->grp) return reject("no one-launch kernel fits the shape");
    std::vector<StepLayer> host((size_t)n_layers);
    for (int l = 0; l < n_layers; l++) {
        const DevLayer &L = layers[l];
        host[(size_t)l] = StepLayer{L.experts, L.router.data, (const float *)L.router.scales, L.router_b, L.mlp_norm};
    }
    register_owner(p, plan_release);
    MH_TRY(plan_alloc(p, &p->layers, sizeof(StepLayer) * (size_t)n_layers, "decode plan layers"));
    MH_HIP(hipMemcpy(p->layers, host.data(), sizeof(StepLayer) * (size_t)n_layers, hipMemcpyHostToDevice));
    MH_TRY(plan_alloc(p, &p->flags, sizeof(unsigned) * (size_t)flag_words(nb), "decode plan flags"));
    MH_TRY(plan_alloc(p, &p->trace, sizeof(unsigned long long) * kStamps * (size_t)n_layers * (size_t)nb,
                      "decode plan stamps"));
    p->n_layers = n_layers;
    MH_HIP(hipHostMalloc((void **)&p->err, sizeof(unsigned), hipHostMallocMapped));
    *p->err = 0;
    MH_HIP(hipHostGetDevicePointer((void **)&p->err_dev, p->err, 0));
    watch_async_error(p->err, "decode step: an exchange timed out (blocks not co-resident)");
    p->tagged_words = tag_layout(L0).total;
    MH_TRY(plan_alloc(p, &p->tagged, sizeof(uint64_t) * p->tagged_words, "decode plan exchange words"));
    MH_HIP(hipMemset(p->tagged, 0, sizeof(uint64_t) * p->tagged_words));
    MH_TRY(plan_alloc(p, &p->h, sizeof(float) * (size_t)L0.top_k * (size_t)L0.ffn, "decode plan h"));
    if (L0.expert_dt == MH_DT_MXFP4) {
        // down scales (bit 1: the expert-group kernel), gate and up scales
        // (bit 2: with bit 1, the expert-grouped kernels of batches 2-16)
        unsigned *bad = nullptr;
        MH_TRY(dev_alloc((void **)&bad, sizeof(unsigned), "decode plan scale scan"));
        MH_HIP(hipMemset(bad, 0, sizeof(unsigned)));
        const int n_dn = (int)(L0.hidden * (L0.ffn / 32)), n_gu = (int)(L0.ffn * (L0.hidden / 32));
        for (int l = 0; l < n_layers; l++) {
            const DevLayer &L = layers[l];
            hipLaunchKernelGGL(k_scan_scales, dim3(16, (unsigned)L.n_experts), dim3(256), 0, 0, L.experts,
                               L.expert_stride, L.off[7], n_dn, bad, 1u);
            hipLaunchKernelGGL(k_scan_scales, dim3(16, (unsigned)L.n_experts), dim3(256), 0, 0, L.experts,
                               L.expert_stride, L.off[1], n_gu, bad, 2u);
            hipLaunchKernelGGL(k_scan_scales, dim3(16, (unsigned)L.n_experts), dim3(256), 0, 0, L.experts,
                               L.expert_stride, L.off[4], n_gu, bad, 2u);
        }
        unsigned hb = 0;
        const hipError_t le = hipGetLastError();
        const hipError_t ce = le != hipSuccess ? le : hipMemcpy(&hb, bad, sizeof(unsigned), hipMemcpyDeviceToHost);
        dev_release(bad, sizeof(unsigned));
        MH_HIP(ce);
        if (hb & 1u) p->grp = 0;   // the vector-ALU kernel handles any f16 scale
        p->few = hb == 0u;
    }
    MH_HIP(hipMemset(p->flags, 0, sizeof(unsigned) * (size_t)flag_words(nb)));
    MH_HIP(hipDeviceSynchronize());
    p->seq = 1;
    p->nb = nb;
    p->ok = p->flat || p->grp;
    if (!p->ok) snprintf(p->why, sizeof(p->why), "down scales not exact in f16 and the vector-ALU kernel does not fit");
    return MH_OK;
}

void step_plan_destroy(StepPlan *p) {
    if (!p) return;
    unregister_owner(p);
    plan_release(p);
    delete p;
}

bool step_plan_ok(const StepPlan *p) { return p && p->ok; }
bool step_plan_few(const StepPlan *p) { return p && p->few; }

namespace {

// A span between two phase stamps: mean over blocks (or block 0 only).
struct Span {
    const char *name;
    int a, b;
    bool b0;
};
const Span kGrpSpans[] = {
    {"x_wait", 0, 15, false},        {"router", 15, 1, false},       {"route", 1, 2, false},
    {"route0_gather", 1, 16, true},  {"route0_rank", 16, 17, true},  {"route0_weights", 17, 18, true},
    {"route0_publish", 18, 2, true}, {"gu_issue", 2, 9, false},      {"gu_math", 9, 10, false},
    {"gu_reduce", 10, 11, false},    {"h_publish", 11, 3, false},    {"dn_stage", 3, 4, false},
    {"h_wait", 4, 5, false},         {"dn_math", 5, 13, false},      {"y_publish", 13, 14, false},
    {"combine", 14, 6, false},       {"tail", 6, 7, false},          {"layer", 0, 7, false},
    {"gu_first_pair", 9, 19, false}, {"gu_mid_pair", 19, 20, false}, {"gu_last_pair", 20, 10, false},
    {"gu_wave7_lag", 10, 21, false}, {"gu_barrier", 10, 22, false}};
const int kGrpOrder[] = {0, 15, 1, 16, 17, 18, 2, 9, 19, 20, 10, 21, 22, 11, 3, 4, 5, 13, 14, 6, 7};
const Span kFlatSpans[] = {
    {"x_wait", 0, 15, false},        {"router", 15, 1, false},       {"route", 1, 2, false},
    {"route0_gather", 1, 16, true},  {"route0_rank", 16, 17, true},  {"route0_weights", 17, 18, true},
    {"route0_publish", 18, 2, true}, {"gate_up", 2, 3, false},       {"gu_issue", 2, 9, false},
    {"gu_math", 9, 10, false},       {"gu_reduce", 10, 11, false},   {"gu_epilogue", 11, 3, false},
    {"barrier_arrive_prefetch", 3, 4, false}, {"barrier_wait", 4, 5, false}, {"down_combine", 5, 6, false},
    {"dn_hload", 5, 12, false},      {"dn_math", 12, 13, false},     {"dn_reduce", 13, 14, false},
    {"dn_combine", 14, 6, false},    {"tail", 6, 7, false},          {"layer", 0, 7, false}};
const int kFlatOrder[] = {0, 15, 1, 16, 17, 18, 2, 9, 10, 11, 3, 4, 5, 12, 13, 14, 6, 7};

// Folds the per-block phase stamps (100 MHz clock) of a profiled launch into
// the profile: per span the mean over blocks and the slowest block; per
// stamp the earliest and latest block from the layer's first start; the
// critical path to the last logit, routing, h and x.
template <size_t NS, size_t NO>
int fold_stamps(const StepPlan *p, int n_layers, int nb, const Span (&spans)[NS], const int (&order)[NO],
                hipStream_t s) {
    std::vector<unsigned long long> tr((size_t)kStamps * n_layers * nb);
    MH_HIP(hipMemcpyAsync(tr.data(), p->trace, tr.size() * 8, hipMemcpyDeviceToHost, s));
    MH_HIP(hipStreamSynchronize(s));
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
        double t0 = 1e300, lastA = 0, lastR = 0, lastB = 0, lastC = 0;
        for (int b = 0; b < nb; b++) {
            t0 = std::min(t0, at(l, 0, b));
            lastA = std::max(lastA, at(l, 1, b));
            lastR = std::max(lastR, at(l, 2, b));
            lastB = std::max(lastB, at(l, 3, b));
            lastC = std::max(lastC, at(l, 6, b));
        }
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
            prof_add(name, lo < 1e299 ? lo * 1e-5 : 0.0);
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

}  // namespace

int step_run(StepPlan *p, const DevLayer *layers, int first, int n_layers, float *x, int32_t *sel, float *w,
             uint32_t *usage, hipStream_t s, const float *gxb, const int32_t *gsel, const float *gw) {
    if (!p || !p->ok) return fail(MH_E_UNSUPPORTED, "decode step: no one-launch kernel for this stack");
    if (first < 0 || n_layers < 1 || first + n_layers > p->n_layers)
        return fail(MH_E_ARG, "decode step: layers [%d, %d) outside the plan's %d", first, first + n_layers, p->n_layers);
    const DevLayer &L0 = layers[first];
    const bool grp = p->grp && !sw(SW_NO_MFMA);
    if (gxb) {
        // routing given: k_decode_grp only, one layer; xb must not overlap x
        // (the combine writes x while other blocks may still read xb)
        if (!grp) return fail(MH_E_UNSUPPORTED, "expert apply: the expert-group kernel does not fit this stack");
        if (n_layers != 1 || !gsel || !gw) return fail(MH_E_ARG, "expert apply: one layer with sel and w");
        const uintptr_t xa = (uintptr_t)x, ba = (uintptr_t)gxb, nbyt = (uintptr_t)L0.hidden * 4u;
        if (xa < ba + nbyt && ba < xa + nbyt) return fail(MH_E_UNSUPPORTED, "expert apply: xb overlaps x");
    }
    if (!grp && !p->flat) return fail(MH_E_UNSUPPORTED, "decode step: the vector-ALU kernel does not fit this stack");
    const TagLayout tl = tag_layout(L0);
    RouteArgs R;
    R.layers = p->layers + first;
    R.n_layers = n_layers;
    R.H = (int)L0.hidden;
    R.E = L0.n_experts;
    R.K = L0.top_k;
    R.eps = L0.norm_eps;
    R.router_norm = L0.router_norm;
    R.x = x;
    R.sel = sel;
    R.w = w;
    R.usage = usage;
    R.lw = p->tagged + tl.lw;
    R.lws = tl.lws;
    R.err = p->err_dev;
    R.trace = profiling() ? p->trace : nullptr;
    const unsigned per_layer = grp ? 4u : 3u;
    if (p->seq > 0xF0000000u) {   // wrap: restart the sequence from a clean slate
        MH_LAUNCH("fill", k_fill_u32, dim3(1), dim3(256), 0, s, p->flags, flag_words(p->nb), 0u);
        MH_LAUNCH("fill", k_fill_u32, dim3(64), dim3(256), 0, s, (unsigned *)p->tagged, (int)(2 * p->tagged_words), 0u);
        p->seq = 1;
    }
    const unsigned seq0 = p->seq;
    p->seq += per_layer * (unsigned)n_layers;
    const int nb = grp ? p->G * R.K : p->nb;
    if (R.trace)   // stamps a block does not reach (a skipped phase) stay 0
        MH_LAUNCH("fill", k_fill_u32, dim3(64), dim3(256), 0, s, (unsigned *)p->trace,
                  (int)(2 * (size_t)kStamps * n_layers * nb), 0u);
    const bool q8 = L0.router.dt == MH_DT_Q8R;
    int rc;
    if (grp) {
        GrpArgs A;
        A.R = R;
        A.F = (int)L0.ffn;
        A.CH = R.H / 32;
        A.CF = A.F / 32;
        A.G = p->G;
        A.PB = p->PB;
        A.RB = p->RB;
        A.stride = L0.expert_stride;
        for (int i = 0; i < 9; i++) A.off[i] = L0.off[i];
        A.alpha = L0.alpha;
        A.limit = L0.limit;
        A.hw = p->tagged + tl.hw;
        A.hws = tl.hws;
        A.yw = (uint32_t *)(p->tagged + tl.yw);
        A.yws = tl.yws;
        A.flags = p->flags;
        A.seq0 = seq0;
        A.y1 = p->tagged + tl.y1;
        A.bank = p->launches & 1u;
        if (n_layers > 1) ++p->launches;
        A.gxb = gxb;
        A.gsel = gsel;
        A.gw = gw;
        if (gxb)
            rc = q8 ? launch_grp<MH_DT_Q8R, true>(A, nb, s) : launch_grp<MH_DT_F32, true>(A, nb, s);
        else
            rc = q8 ? launch_grp<MH_DT_Q8R, false>(A, nb, s) : launch_grp<MH_DT_F32, false>(A, nb, s);
    } else {
        StepArgs A;
        A.R = R;
        A.F = (int)L0.ffn;
        A.CH = R.H / 32;
        A.CF = A.F / 32;
        A.stride = L0.expert_stride;
        for (int i = 0; i < 9; i++) A.off[i] = L0.off[i];
        A.alpha = L0.alpha;
        A.limit = L0.limit;
        A.act_plain = L0.act_plain;
        A.xw = p->tagged + tl.xw;
        A.h = p->h;
        A.flags = p->flags;
        A.go = p->flags + go_offset(p->nb);
        A.seq0 = seq0;
        if (L0.expert_dt == MH_DT_MXFP4)
            rc = q8 ? launch_flat<MH_DT_Q8R, MH_DT_MXFP4>(A, nb, s) : launch_flat<MH_DT_F32, MH_DT_MXFP4>(A, nb, s);
        else
            rc = q8 ? launch_flat<MH_DT_Q8R, MH_DT_Q4G32>(A, nb, s) : launch_flat<MH_DT_F32, MH_DT_Q4G32>(A, nb, s);
    }
    if (rc || !R.trace) return rc;
    return grp ? fold_stamps(p, n_layers, nb, kGrpSpans, kGrpOrder, s)
               : fold_stamps(p, n_layers, nb, kFlatSpans, kFlatOrder, s);
}

}  // namespace mh
