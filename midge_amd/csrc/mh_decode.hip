// mh_decode.hip — a whole MoE decode step (every layer of a stack, batch 1)
// in one cooperative launch: the MoE half of forward()'s layer loop
// (engine/midge.c:557-560) with moe() (engine/midge.c:469-549) per layer.
//
// One block per CU, 512 threads. Per layer, three phases separated by
// grid barriers:
//   A  router     every block loads x, forms xb = rmsnorm(x) in LDS; the
//                 router's rows are spread over the blocks -> logits.
//   B  gate/up    every block runs the same stable top-k on the logits, then
//                 its share of the routed experts' gate/up rows (the pairs of
//                 all k experts laid end to end and cut evenly), with the
//                 bias + clamped SwiGLU epilogue -> h[k][ffn].
//   C  down       each block owns a slice of output rows for all k experts;
//                 their weights are loaded into registers between the
//                 barrier's arrive and wait, so the load overlaps the wait.
//                 Epilogue: y = Wd h + bd, moe = sum_i w_i y_i in selection
//                 order, x += moe.
// Barriers are contention-free: each block publishes a monotonically
// increasing sequence number in its own flag; one wave per block polls all
// flags with a single vector load per lane. Waits are bounded: a barrier that
// does not complete within ~1 s raises an error flag and every block exits.
#include <stdio.h>

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
    float *logits;           // [E] scratch
    float *h;                // [K][F] scratch
    unsigned *flags;         // [gridDim.x] barrier flags
    unsigned *go;            // barrier release word (written by block 0)
    unsigned seq0;           // sequence number of this launch's first barrier
    unsigned *err;
    unsigned long long *trace;   // [L][16] phase timestamps of block 0, or null
    int red_floats;              // LDS floats of the partial-sum area
};

namespace {

constexpr int kThreads = 512;   // 8 waves: 2 per SIMD, up to 256 VGPRs each
constexpr int kUB = 12;         // gate/up row iterations in flight per thread
constexpr int kUC = 12;         // down row iterations in flight per thread
constexpr unsigned kSpinLimit = 1u << 20;

__device__ __forceinline__ void bar_arrive(unsigned *flags, unsigned seq) {
    __builtin_amdgcn_s_waitcnt(0);   // this wave's stores have landed
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_store(&flags[blockIdx.x], seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Gather/broadcast wait: block 0's first wave polls every block's flag (one
// vector load per lane per round) and then publishes `seq` in *go; every
// other block polls that single word. A few hundred loads per round in
// total, instead of every block sweeping every flag. Returns false (in every
// thread) if the barrier timed out.
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
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "agent");
            if (ok && lane == 0) __hip_atomic_store(go, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (lane == 0) {
            while ((int)(__hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - seq) < 0) {
                __builtin_amdgcn_s_sleep(1);
                if (++spins > kSpinLimit) {
                    ok = false;
                    break;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
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
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += part[i];
    __syncthreads();
    return s;
}

// Stable top-k by one wave over LDS logits v[E] (ties to the lower index;
// only values > -1e30 qualify; unfilled slots get -1, engine/midge.c:476-486)
// and the routing weights (engine/midge.c:502-512). Results in LDS.
__device__ void wave_topk(const float *v, int E, int k, int router_norm, int *s_sel, float *s_val, float *s_w) {
    const int lane = threadIdx.x & 63;
    unsigned long long taken = 0;   // bit j: element lane + 64 j is taken
    for (int i = 0; i < k; ++i) {
        float bv = -1e30f;
        int bi = INT32_MAX;
        for (int j = 0; lane + 64 * j < E; ++j) {
            const int e = lane + 64 * j;
            if (!((taken >> j) & 1ull) && v[e] > bv) {
                bv = v[e];
                bi = e;
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (bi != INT32_MAX && (bi & 63) == lane) taken |= 1ull << (bi >> 6);
        if (lane == 0) {
            s_sel[i] = bi == INT32_MAX ? -1 : bi;
            s_val[i] = bi == INT32_MAX ? -1e30f : bv;
        }
    }
    float fmx = 0.f, fden = 0.f;
    if (!router_norm) {
        float m = -INFINITY;
        for (int e = lane; e < E; e += 64) m = fmaxf(m, v[e]);
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float s = 0.f;
        for (int e = lane; e < E; e += 64) s += expf(v[e] - m);
        fden = mh_wave_sum(s);
        fmx = m;
    }
    if (lane == 0) {
        if (router_norm) {
            const float mx = s_val[0];
            float den = 0.f;
            for (int i = 0; i < k; ++i) {
                s_w[i] = expf(s_val[i] - mx);
                den += s_w[i];
            }
            for (int i = 0; i < k; ++i) s_w[i] /= den;
        } else {
            for (int i = 0; i < k; ++i) s_w[i] = expf(s_val[i] - fmx) / fden;
        }
    }
}

__device__ __forceinline__ float act_fn(float g, float u, float alpha, float limit, int plain) {
    if (plain) return g / (1.0f + expf(-g)) * u;
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    if (u < -limit) u = -limit;
    const float a = g / (1.0f + expf(-alpha * g));
    return a * (u + 1.0f);
}

// Phase A's inputs that do not depend on x, loaded ahead of time: this
// block's first router-row chunk and the first kNW norm weights per thread
// (for layer 0 at kernel start, for layer l + 1 before layer l's last wait).
constexpr int kNW = 4;
struct RouterPref {
    mh_u4 rq;
    float nw[kNW];
};

__device__ __forceinline__ RouterPref prefetch_router(const StepArgs &A, int l, int CR) {
    RouterPref p;
    const StepLayer Lp = A.layers[l];
    const int b = blockIdx.x, t = threadIdx.x;
    p.rq = mh_u4{0u, 0u, 0u, 0u};
    if (b < A.E && t < CR) p.rq = mh_load16(mh_global(Lp.router_w + (size_t)b * CR * 16 + (size_t)t * 16));
#pragma unroll
    for (int k = 0; k < kNW; ++k) {
        const int i = t + k * (int)blockDim.x;
        p.nw[k] = i < A.H ? *(const float __attribute__((address_space(1))) *)mh_global(Lp.norm_w + i) : 0.f;
    }
    return p;
}

template <int RDT, int XDT>
__global__ void __launch_bounds__(kThreads) k_decode_step(StepArgs A) {
    constexpr int XE = mh_chunk<XDT>::E;   // elements per expert chunk (32)
    constexpr int RE = mh_chunk<RDT>::E;   // elements per router chunk (16 int8 / 4 f32)
    extern __shared__ float lds[];
    __shared__ float s_part[16];
    __shared__ int s_sel[16];
    __shared__ float s_w[16];
    __shared__ float s_val[16];
    __shared__ int s_ok;
    const int H = A.H, F = A.F, E = A.E, K = A.K;
    float *xs = lds;             // x at layer start
    float *xbs = xs + H;         // rmsnorm(x) * w
    float *res = xbs + H;        // reduced rows / staged logits
    const int res_floats = max(max(E, 2 * K * F / (int)gridDim.x + 2), K * ((H + gridDim.x - 1) / gridDim.x)) + 64;
    float *red = res + res_floats;
    float *bds = red + A.red_floats;   // [K][rows of this block's down slice]
    const int NB = gridDim.x, b = blockIdx.x, t = threadIdx.x;
    const int nw = blockDim.x >> 6, wave = t >> 6, lane = t & 63;
    unsigned seq = A.seq0;

    unsigned long long *tr = (A.trace && b == 0 && t == 0) ? A.trace : nullptr;
    // Phase A's inputs that do not depend on x are loaded ahead: this
    // block's first router row chunk and the first kNW norm weights of each
    // thread, for layer 0 here and for layer l + 1 before layer l's last
    // barrier wait.
    const int CR = H / RE;                 // router chunks per row
    RouterPref pf = prefetch_router(A, 0, CR);
    for (int l = 0; l < A.n_layers; ++l) {
        const StepLayer Ly = A.layers[l];
        if (tr) tr[l * 16 + 0] = wall_clock64();
        // ------------------------------------------------ A: router
        float ss = 0.f;
        for (int i = t; i < H; i += blockDim.x) {
            const float v = A.x[i];
            xs[i] = v;
            ss = __builtin_fmaf(v, v, ss);
        }
        ss = block_sum(ss, s_part);
        const float inv = 1.0f / sqrtf(ss / (float)H + A.eps);
#pragma unroll
        for (int k = 0; k < kNW; ++k) {
            const int i = t + k * (int)blockDim.x;
            if (i < H) xbs[i] = xs[i] * inv * pf.nw[k];
        }
        for (int i = t + kNW * (int)blockDim.x; i < H; i += blockDim.x) xbs[i] = xs[i] * inv * Ly.norm_w[i];
        __syncthreads();
        for (int e = b; e < E; e += NB) {
            float p = 0.f;
            for (int c = t; c < CR; c += blockDim.x) {
                const mh_u4 q = (e == (int)blockIdx.x && c == t) ? pf.rq
                                                   : mh_load16(mh_global(Ly.router_w + (size_t)e * CR * 16 + (size_t)c * 16));
                p += mh_dot_chunk<RDT>(q, xbs + (size_t)c * RE);
            }
            p = block_sum(p, s_part);
            if (t == 0) {
                if constexpr (RDT == MH_DT_Q8R) p *= Ly.router_s[e];
                A.logits[e] = p + Ly.router_b[e];
            }
        }
        if (tr) tr[l * 16 + 1] = wall_clock64();
        bar_arrive(A.flags, seq);
        if (!bar_wait(A.flags, A.go, seq, A.err, &s_ok)) return;
        ++seq;
        if (tr) tr[l * 16 + 2] = wall_clock64();

        // ------------------------------------------------ B: gate/up
        for (int e = t; e < E; e += blockDim.x) res[e] = A.logits[e];
        __syncthreads();
        if (wave == 0) wave_topk(res, E, K, A.router_norm, s_sel, s_val, s_w);
        __syncthreads();
        if (tr) tr[l * 16 + 8] = wall_clock64();
        if (b == 0 && t < K) {
            if (A.sel) A.sel[(size_t)l * K + t] = s_sel[t];
            if (A.w) A.w[(size_t)l * K + t] = s_w[t];
            if (A.usage && s_sel[t] >= 0) A.usage[(size_t)l * E + s_sel[t]] += 1u;
        }
        {
            const int C = A.CH;
            const int ns = blockDim.x / C;
            const int slot = t / C, c = t - slot * C;
            const bool active = slot < ns;
            const int TB = 2 * K * F;
            int RB = (TB + NB - 1) / NB;
            RB += RB & 1;
            const int f_begin = b * RB;
            const int nf = max(0, min(TB, f_begin + RB) - f_begin);
            float xr[XE];
#pragma unroll
            for (int j = 0; j < XE; ++j) xr[j] = active ? xbs[c * XE + j] : 0.f;
            // The block's pairs [pb, pb + nf/2) span at most two experts
            // (nf/2 <= F, checked at plan creation): expert ia from row rb,
            // then ia + 1.
            const int pb = f_begin >> 1;
            const int ia = min(pb / F, K - 1), rb = pb - ia * F;
            const int e_a = s_sel[ia], e_b = ia + 1 < K ? s_sel[ia + 1] : -1;
            const uint32_t eo_a = e_a >= 0 ? (uint32_t)e_a * (uint32_t)A.stride : 0u;
            const uint32_t eo_b = e_b >= 0 ? (uint32_t)e_b * (uint32_t)A.stride : 0u;
            const uint32_t od0 = (uint32_t)A.off[0], od1 = (uint32_t)A.off[3];
            const uint32_t os0 = (uint32_t)A.off[1], os1 = (uint32_t)A.off[4];
            float bg_pref = 0.f, bu_pref = 0.f;
            for (int f0 = 0; f0 < nf; f0 += ns * kUB) {
                // Branch-free loads (see block_gemv): a past-the-end row, an
                // idle slot or an unfilled routing slot re-reads the block's
                // last row and is masked out in the math; scale bits stay raw
                // until every load is in flight.
                mh_u4 q[kUB];
                uint32_t sb[kUB];
                const int sl = active ? slot : ns - 1;
                const mh_gbytes ex = mh_global(Ly.experts);
                if (f0 == 0) {   // this thread's epilogue pair's biases, loaded with the weights
                    const int pp = min(t, max(nf / 2 - 1, 0));
                    const int pr = rb + pp;
                    const bool second = pr >= F;
                    const uint32_t eo = second ? eo_b : eo_a;
                    const uint32_t r4 = (uint32_t)(second ? pr - F : pr) * 4u;
                    bg_pref = *(const float __attribute__((address_space(1))) *)(ex + (eo + (uint32_t)A.off[2] + r4));
                    bu_pref = *(const float __attribute__((address_space(1))) *)(ex + (eo + (uint32_t)A.off[5] + r4));
                }
#pragma unroll
                for (int u = 0; u < kUB; ++u) {
                    const int f = min(f0 + u * ns + sl, nf - 1);
                    const int m = f & 1, pr = rb + (f >> 1);
                    const bool second = pr >= F;
                    const int r = second ? pr - F : pr;
                    const uint32_t eo = second ? eo_b : eo_a;   // offsets fit 32 bits (plan check)
                    const uint32_t rc = (uint32_t)(r * C + c);
                    q[u] = mh_load16(ex + (eo + (m ? od1 : od0) + rc * 16u));
                    sb[u] = mh_load_u16(ex + (eo + (m ? os1 : os0) + rc * 2u));
                }
                __builtin_amdgcn_sched_barrier(0);   // all loads issued before any math
                if (tr && f0 == 0) tr[l * 16 + 9] = wall_clock64();
#pragma unroll
                for (int u = 0; u < kUB; ++u) {
                    const int f = f0 + u * ns + slot;
                    const bool valid = active && f < nf && (rb + (f >> 1) >= F ? e_b : e_a) >= 0;
                    const float p = mh_dot_chunk<XDT>(q[u], xr) * (valid ? mh_f16((uint16_t)sb[u]) : 0.f);
                    if (active && f < nf) red[(u * ns + slot) * C + c] = p;
                    __builtin_amdgcn_sched_barrier(0);   // one chunk's math at a time
                }
                if (tr && f0 == 0) tr[l * 16 + 10] = wall_clock64();
                __syncthreads();
                const int items = min(ns * kUB, nf - f0);
                block_reduce_rows(red, C, items, res + f0, [](int) { return true; });
                __syncthreads();
                if (tr && f0 == 0) tr[l * 16 + 11] = wall_clock64();
            }
            // epilogue: pairs (gate, up) -> h (nf / 2 <= F < blockDim.x pairs: one per thread)
            if (t < nf / 2) {
                const int pp = t;
                const int pr = rb + pp;
                const bool second = pr >= F;
                const int r = second ? pr - F : pr;
                const int i = second ? ia + 1 : ia;
                const int e = second ? e_b : e_a;
                float hv = 0.f;
                if (e >= 0) hv = act_fn(res[2 * pp] + bg_pref, res[2 * pp + 1] + bu_pref, A.alpha, A.limit, A.act_plain);
                A.h[(size_t)i * F + r] = hv;
            }
        }
        if (tr) tr[l * 16 + 3] = wall_clock64();
        bar_arrive(A.flags, seq);

        // ------------------------------------------------ C: down + combine
        {
            // one pass (checked at plan creation): slot -> (expert i, row
            // phase sub), rows j = sub + spe * u of this block's slice
            const int C = A.CF;
            const int nsC = blockDim.x / C;
            const int slot = t / C, c = t - slot * C;
            const int RC = (H + NB - 1) / NB;
            const int r_begin = b * RC;
            const int nr = max(0, min(H, r_begin + RC) - r_begin);
            const int spe = nsC / K;
            const int i = slot / spe, sub = slot - i * spe;
            const bool act = i < K;
            const int e = act ? s_sel[i] : -1;
            // idle slots and unfilled routing slots read the first routed
            // expert's rows (cache hits) and are masked out
            const int ea = e >= 0 ? e : max(s_sel[0], 0);
            const uint32_t eo = (uint32_t)ea * (uint32_t)A.stride;
            // branch-free prefetch (see phase B): out-of-range rows re-read
            // the slice's first row of expert 0's slot and are masked out
            mh_u4 q[kUC];
            uint32_t sb[kUC];
            const mh_gbytes ex = mh_global(Ly.experts);
            const uint32_t rows_ok = nr > 0 ? (uint32_t)nr : 1u;
#pragma unroll
            for (int u = 0; u < kUC; ++u) {
                const int j = min(sub + spe * u, (int)rows_ok - 1);
                const uint32_t rc = (uint32_t)((min(r_begin, H - 1) + j) * C + c);
                q[u] = mh_load16(ex + (eo + (uint32_t)A.off[6] + rc * 16u));
                sb[u] = mh_load_u16(ex + (eo + (uint32_t)A.off[7] + rc * 2u));
            }
            // the down biases of this block's rows, (expert i, row j) -> thread i * nr + j
            float bd_pref = 0.f;
            if (t < K * nr) {
                const int ib = t / nr, jb = t - ib * nr;
                const int eb = s_sel[ib];
                if (eb >= 0)
                    bd_pref = *(const float __attribute__((address_space(1))) *)(
                        ex + ((uint32_t)eb * (uint32_t)A.stride + (uint32_t)A.off[8] + (uint32_t)(r_begin + jb) * 4u));
            }
            __builtin_amdgcn_sched_barrier(0);
            if (tr) tr[l * 16 + 4] = wall_clock64();
            if (!bar_wait(A.flags, A.go, seq, A.err, &s_ok)) return;
            ++seq;
            if (tr) tr[l * 16 + 5] = wall_clock64();
            float xr[XE];
#pragma unroll
            for (int jj = 0; jj < XE; ++jj) xr[jj] = act ? A.h[(size_t)i * F + c * XE + jj] : 0.f;
            if (tr) tr[l * 16 + 12] = wall_clock64();
#pragma unroll
            for (int u = 0; u < kUC; ++u) {
                const int j = sub + spe * u;
                const bool valid = e >= 0 && j < nr;
                const float p = mh_dot_chunk<XDT>(q[u], xr) * (valid ? mh_f16((uint16_t)sb[u]) : 0.f);
                if (act && j < nr) red[(i * RC + j) * C + c] = p;
                __builtin_amdgcn_sched_barrier(0);
            }
            if (t < K * nr) bds[t] = bd_pref;
            if (tr) tr[l * 16 + 13] = wall_clock64();
            __syncthreads();
            block_reduce_rows(red, C, K * RC, res, [&](int it) { return it % RC < nr; });
            __syncthreads();
            if (tr) tr[l * 16 + 14] = wall_clock64();
            // combine in selection order: moe = sum_i w_i (dot_i + bd_i); x += moe
            for (int j = t; j < nr; j += blockDim.x) {
#pragma clang fp contract(off)
                const int r = r_begin + j;
                float moe = 0.f;
                for (int ii = 0; ii < K; ++ii) {
                    if (s_sel[ii] < 0) continue;
                    const float y = res[ii * RC + j] + bds[ii * nr + j];
                    moe = moe + s_w[ii] * y;
                }
                A.x[r] = xs[r] + moe;
            }
        }
        if (tr) tr[l * 16 + 6] = wall_clock64();
        bar_arrive(A.flags, seq);
        if (l + 1 < A.n_layers) pf = prefetch_router(A, l + 1, CR);
        if (!bar_wait(A.flags, A.go, seq, A.err, &s_ok)) return;
        ++seq;
        if (tr) tr[l * 16 + 7] = wall_clock64();
    }
}

__global__ void k_fill_u32(unsigned *p, int n, unsigned v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

template <int RDT, int XDT>
int launch_t(const StepArgs &A, int nb, size_t lds, hipStream_t s) {
    auto k = k_decode_step<RDT, XDT>;
    MH_HIP(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int per_cu = 0;
    MH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, lds));
    if (per_cu < 1) return fail(MH_E_UNSUPPORTED, "decode step: a 1024-thread block with %zu B LDS does not fit a CU", lds);
    StepArgs a = A;
    void *args[] = {&a};
    const bool prof = profiling();
    if (prof) prof_begin("decode_step", s);
    hipError_t e = hipLaunchCooperativeKernel((const void *)k, dim3(nb), dim3(kThreads), args, (unsigned)lds, s);
    if (prof) prof_end(s);
    return hip_check(e, "decode step cooperative launch");
}

}  // namespace

// Scratch and tables a stack keeps for the one-launch path.
struct StepPlan {
    StepLayer *layers = nullptr;   // device [L]
    unsigned *flags = nullptr;     // device [nb + 64]: flags, then the go word on its own line
    unsigned long long *trace = nullptr;   // device [L][8] (filled while profiling)
    int n_layers = 0;
    unsigned *err = nullptr;       // host-mapped pinned [1]: set by a timed-out barrier
    unsigned *err_dev = nullptr;   // its device address
    float *logits = nullptr;       // device [E]
    float *h = nullptr;            // device [K][F]
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
    if (L0.n_experts > 1024 || L0.top_k > 16) return reject("too many experts");
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
    int nb = device_cus();
    {   // the down phase runs in one pass: every routed expert gets slots,
        // and each slot's rows of the block's slice fit kUC iterations
        const int nsC = kThreads / (int)(L0.ffn / 32);
        const int spe = L0.top_k > 0 ? nsC / L0.top_k : 0;
        const int RC = (int)((L0.hidden + nb - 1) / nb);
        if (spe < 1 || RC > spe * kUC) return reject("down phase does not fit one pass");
        int RB = (int)((2 * L0.top_k * L0.ffn + nb - 1) / nb);
        RB += RB & 1;
        if (RB / 2 > L0.ffn) return reject("a block's gate/up range would span more than two experts");
        if ((int)(L0.hidden / 32) > kThreads || (int)(L0.hidden / 16) > kThreads) return reject("hidden too wide");
    }
    std::vector<StepLayer> host((size_t)n_layers);
    for (int l = 0; l < n_layers; l++) {
        const DevLayer &L = layers[l];
        host[(size_t)l] = StepLayer{L.experts, L.router.data, (const float *)L.router.scales, L.router_b, L.mlp_norm};
    }
    MH_HIP(hipMalloc(&p->layers, sizeof(StepLayer) * (size_t)n_layers));
    MH_HIP(hipMemcpy(p->layers, host.data(), sizeof(StepLayer) * (size_t)n_layers, hipMemcpyHostToDevice));
    MH_HIP(hipMalloc(&p->flags, sizeof(unsigned) * (size_t)(nb + 64)));
    MH_HIP(hipMalloc(&p->trace, sizeof(unsigned long long) * 16 * (size_t)n_layers));
    p->n_layers = n_layers;
    MH_HIP(hipHostMalloc((void **)&p->err, sizeof(unsigned), hipHostMallocMapped));
    *p->err = 0;
    MH_HIP(hipHostGetDevicePointer((void **)&p->err_dev, p->err, 0));
    watch_async_error(p->err, "decode step: a grid barrier timed out (blocks not co-resident)");
    MH_HIP(hipMalloc(&p->logits, sizeof(float) * (size_t)L0.n_experts));
    MH_HIP(hipMalloc(&p->h, sizeof(float) * (size_t)L0.top_k * (size_t)L0.ffn));
    MH_HIP(hipMemset(p->flags, 0, sizeof(unsigned) * (size_t)(nb + 64)));
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
    (void)hipFree(p->logits);
    (void)hipFree(p->h);
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
    A.logits = p->logits;
    A.h = p->h;
    A.flags = p->flags;
    A.go = p->flags + ((p->nb + 63) / 32) * 32;   // a separate 128-byte line
    A.trace = profiling() ? p->trace : nullptr;
    A.err = p->err_dev;
    const unsigned nbar = 3u * (unsigned)n_layers;
    if (p->seq > 0xF0000000u) {   // wrap: restart the sequence from a clean slate
        MH_LAUNCH("fill", k_fill_u32, dim3(1), dim3(256), 0, s, p->flags, p->nb + 64, 0u);
        p->seq = 1;
    }
    A.seq0 = p->seq;
    p->seq += nbar;
    const int nb = p->nb;
    const int res_floats = std::max(std::max(A.E, 2 * A.K * A.F / nb + 2), A.K * ((A.H + nb - 1) / nb)) + 64;
    const int nsB = kThreads / A.CH, nsC = kThreads / A.CF;
    const size_t red_floats = std::max((size_t)nsB * kUB * A.CH,
                                       (size_t)std::min(A.K, nsC) * (size_t)((A.H + nb - 1) / nb) * A.CF);
    A.red_floats = (int)red_floats;
    const size_t lds = ((size_t)2 * A.H + res_floats + red_floats + (size_t)A.K * ((A.H + nb - 1) / nb)) *
                       sizeof(float);
    if (lds > 160 * 1024) return fail(MH_E_UNSUPPORTED, "decode step needs %zu B of LDS", lds);
    int rc;
    if (L0.router.dt == MH_DT_Q8R)
        rc = L0.expert_dt == MH_DT_MXFP4 ? launch_t<MH_DT_Q8R, MH_DT_MXFP4>(A, nb, lds, s)
                                         : launch_t<MH_DT_Q8R, MH_DT_Q4G32>(A, nb, lds, s);
    else
        rc = L0.expert_dt == MH_DT_MXFP4 ? launch_t<MH_DT_F32, MH_DT_MXFP4>(A, nb, lds, s)
                                         : launch_t<MH_DT_F32, MH_DT_Q4G32>(A, nb, lds, s);
    if (rc || !A.trace) return rc;
    // profiling: fold block 0's phase timestamps (100 MHz clock) into the profile
    std::vector<unsigned long long> tr((size_t)16 * n_layers);
    MH_HIP(hipMemcpyAsync(tr.data(), p->trace, tr.size() * 8, hipMemcpyDeviceToHost, s));
    MH_HIP(hipStreamSynchronize(s));
    // (name, from, to) over block 0's timestamps
    static const struct { const char *name; int a, b; } spans[] = {
        {"decode_step/router", 0, 1}, {"decode_step/barrier1", 1, 2}, {"decode_step/gate_up", 2, 3},
        {"decode_step/gu_topk", 2, 8}, {"decode_step/gu_issue", 8, 9}, {"decode_step/gu_math", 9, 10},
        {"decode_step/gu_reduce", 10, 11}, {"decode_step/gu_epilogue", 11, 3},
        {"decode_step/barrier2_arrive_prefetch", 3, 4}, {"decode_step/barrier2_wait", 4, 5},
        {"decode_step/down_combine", 5, 6}, {"decode_step/dn_hload", 5, 12}, {"decode_step/dn_math", 12, 13},
        {"decode_step/dn_reduce", 13, 14}, {"decode_step/dn_combine", 14, 6}, {"decode_step/barrier3", 6, 7}};
    for (int l = 0; l < n_layers; l++)
        for (const auto &sp : spans)
            prof_add(sp.name, (double)(tr[(size_t)l * 16 + sp.b] - tr[(size_t)l * 16 + sp.a]) * 1e-5);
    return MH_OK;
}

}  // namespace mh
