// mh_moe.hip — the MoE layer on the GPU: router top-k and weights, the
// routed experts' fused gate/up + clamped SwiGLU, the down projection, the
// deterministic weighted combine, and the layer / stack entry points.
//   mh_moe, mh_moe_dev          moe(), engine/midge.c:469-549
//   mh_moe_prefill(_dev)        forward_batch() MoE half, engine/midge.c:591-611
//   mh_topk_dev                 route_topk() selection, engine/midge.c:410-433
//   mh_expert_major_dev         expert-major loop + expert_apply, midge.c:595-611, 437-467
//   mh_stack_*                  forward()'s layer loop, MoE half, midge.c:557-560
#include <vector>

#include "mh_gemv.cuh"

namespace mh {
namespace {

constexpr int kMaxTopK = 16;       // engine/midge.c:44 MAX_TOPK
constexpr int kMaxExperts = 1024;  // one wave holds 16 logits per lane

// ------------------------------------------------------------- top-k

// One wave per token: v = logits + bias; the k largest values > -1e30 in
// descending order, ties to the lower expert index (the insertion lists of
// engine/midge.c:476-486 and 410-422 produce exactly this). Unfilled slots
// get sel = `unfilled` (-1 for moe(), 0 for route_topk()) and value -1e30.
// Weights as engine/midge.c:502-512. usage (may be NULL) += 1 per filled slot.
// The top-k of one token's logits rl[E] by one whole wave (every lane calls
// it); lane 0 writes sel[k], w[k] and the usage counts. PER logits per lane
// (E <= 64 PER).
template <int PER>
__device__ __forceinline__ void wave_topk_token(const float *rl, const float *__restrict__ bias, int E, int k,
                                                int router_norm, int unfilled, int32_t *__restrict__ sel,
                                                float *__restrict__ w, uint32_t *__restrict__ usage) {
    const int lane = threadIdx.x & 63;
    float v[PER];
    bool taken[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        int e = lane + 64 * j;
        v[j] = -INFINITY;
        taken[j] = true;
        if (e < E) {
            v[j] = bias ? rl[e] + bias[e] : rl[e];
            taken[j] = false;
        }
    }
    float val[kMaxTopK];
    int idx[kMaxTopK];
    for (int i = 0; i < k; ++i) {
        // lane-local best eligible (value > -1e30, strict), lowest index on ties
        float bv = -1e30f;
        int bi = INT32_MAX;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if (!taken[j] && v[j] > bv) {   // strict: NaN and <= -1e30 never win
                bv = v[j];
                bi = lane + 64 * j;
            }
        }
        // wave argmax: the largest value, then the lowest index among the
        // lanes holding it, then that lane's own value (DPP steps, no LDS)
        const float wm = wave_max(bv);
        bi = wave_min(bv == wm ? bi : INT32_MAX);
        bv = bi == INT32_MAX ? -1e30f : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), bi & 63));
        if (bi == INT32_MAX) {
            val[i] = -1e30f;
            idx[i] = unfilled;
        } else {
            val[i] = bv;
            idx[i] = bi;
            if ((bi & 63) == lane) {
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    if (lane + 64 * j == bi) taken[j] = true;
            }
        }
    }
    float fmx = 0.f, fden = 0.f;
    if (!router_norm) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (lane + 64 * j < E) m = fmaxf(m, v[j]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (lane + 64 * j < E) s += expf(v[j] - m);
        fden = mh_wave_sum(s);
        fmx = m;
    }
    if (lane == 0) {
        float wt[kMaxTopK];
        if (router_norm) {
            const float mx = val[0];
            float den = 0.f;
            for (int i = 0; i < k; ++i) {
                wt[i] = expf(val[i] - mx);
                den += wt[i];
            }
            for (int i = 0; i < k; ++i) wt[i] /= den;
        } else {
            for (int i = 0; i < k; ++i) wt[i] = expf(val[i] - fmx) / fden;
        }
        for (int i = 0; i < k; ++i) {
            sel[i] = idx[i];
            w[i] = wt[i];
            if (usage && idx[i] >= 0 && idx[i] < E && val[i] > -1e30f) atomicAdd(&usage[idx[i]], 1u);
        }
    }
}

// Assignments a block can sort (16 tokens of up to kMaxTopK slots).
constexpr int kMaxOrder = 16 * kMaxTopK;

// Rank of key ki among the N distinct keys in sk (LDS): the keys are read in
// batches of 16 issued together (a read-compare loop waits for each read).
__device__ __forceinline__ int key_rank(const int *sk, int N, int ki) {
    int r = 0;
    for (int j0 = 0; j0 < N; j0 += 16) {
        int kv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) kv[j] = j0 + j < N ? sk[j0 + j] : INT32_MAX;
#pragma unroll
        for (int j = 0; j < 16; ++j) r += kv[j] < ki;
    }
    return r;
}

// moe = sum_i w[i] y_i[r] over a token's k slots in slot order, each product
// and sum rounded separately (engine/midge.c:514, 544). The slots' y values
// are read in batches of 4 issued together, then added in slot order.
__device__ __forceinline__ float slot_sum(const float *__restrict__ w, const float *__restrict__ ye, int64_t H,
                                          int k, int64_t r) {
#pragma clang fp contract(off)
    float moe = 0.f;
    for (int i0 = 0; i0 < k; i0 += 4) {
        float yv[4], wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            yv[i] = i0 + i < k ? ye[(size_t)(i0 + i) * H + r] : 0.f;
            wv[i] = i0 + i < k ? w[i0 + i] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i0 + i < k) moe = moe + wv[i] * yv[i];
    }
    return moe;
}

// One wave per token. With `order` (one block holding all n tokens, n k <=
// kMaxOrder), the block then sorts the assignments by expert id, stably,
// unroutable slots last: order[r] = assignment a, order[n k + r] = sel[a].
// The expert kernels walk assignments in that order, so the assignments of
// one expert run side by side and share its weight lines in the caches.
template <int PER>
__global__ void __launch_bounds__(1024)
k_topk(const float *__restrict__ rl, const float *__restrict__ bias, int n, int E, int k, int router_norm,
       int unfilled, int32_t *__restrict__ sel, float *__restrict__ w, uint32_t *__restrict__ usage,
       int32_t *__restrict__ order) {
    const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (t < n)   // wave-uniform
        wave_topk_token<PER>(rl + (size_t)t * E, bias, E, k, router_norm, unfilled, sel + (size_t)t * k,
                             w + (size_t)t * k, usage);
    if (order == nullptr) return;   // grid-uniform
    __shared__ int skey[kMaxOrder];
    const int N = n * k;
    __syncthreads();   // every wave's sel stores are visible to the block
    for (int i = threadIdx.x; i < N; i += blockDim.x) {
        const int e = sel[i];
        skey[i] = (e >= 0 && e < E ? e : E) * N + i;   // distinct keys
    }
    __syncthreads();
    for (int i = threadIdx.x; i < N; i += blockDim.x) {
        const int ki = skey[i];
        const int r = key_rank(skey, N, ki);
        order[r] = i;
        order[N + r] = ki / N < E ? ki / N : -1;
    }
}

// ------------------------------------------------------- expert FFN

struct ExpertArgs {
    const uint8_t *experts;     // layer base
    uint64_t stride;
    uint64_t off[9];
    int E, k;
    int64_t hidden, ffn;
    float alpha, limit;
    int act_plain;
};

__device__ __forceinline__ float act_fn(float g, float u, float alpha, float limit, int plain) {
    if (plain) return g / (1.0f + expf(-g)) * u;
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    if (u < -limit) u = -limit;
    const float a = g / (1.0f + expf(-alpha * g));
    return a * (u + 1.0f);
}

// The assignment of grid row y and its expert: y itself, or the y-th of the
// expert-sorted order (order[y], order[A + y] for A assignments).
struct Assignment {
    int a, e;
};
__device__ __forceinline__ Assignment assignment_of(const int32_t *__restrict__ sel,
                                                    const int32_t *__restrict__ order) {
    const int y = blockIdx.y;
    if (order) return {order[y], order[gridDim.y + y]};
    return {y, sel[y]};
}

// Gate and up rows of the expert routed for assignment a (token a / k),
// rows [blockIdx.x * rpb, +rpb): h[a][r] = act(g + bg, u + bu). Flat row f
// interleaves the two matrices: f = 2i (gate row i), 2i+1 (up row i).
template <int DT>
__global__ void __launch_bounds__(kGemvThreads)
k_expert_gu(ExpertArgs A, const int32_t *__restrict__ sel, const int32_t *__restrict__ order,
            const float *__restrict__ xb, float *__restrict__ h, int ns, int rpb) {
    constexpr int CE = gemv_chunk<DT>::E;
    extern __shared__ float lds[];
    const Assignment as = assignment_of(sel, order);
    const int a = as.a, e = as.e;
    const int r0 = blockIdx.x * rpb;
    const int nr = (int)min((int64_t)rpb, A.ffn - r0);
    float *hout = h + (size_t)a * A.ffn;
    if (e < 0 || e >= A.E) {   // unroutable slot contributes nothing
        for (int i = threadIdx.x; i < nr; i += blockDim.x) hout[r0 + i] = 0.f;
        return;
    }
    const int C = (int)(A.hidden / CE);
    float *res = lds;              // [2 * rpb]
    float *red = lds + 2 * rpb;    // [U][ns][C]
    const uint8_t *base = A.experts + (uint64_t)e * A.stride;
    const uint32_t rowbytes = (uint32_t)C * 16u * gemv_chunk<DT>::W;
    const uint32_t srow = (DT == MH_DT_Q8R) ? 0u : 2u * (uint32_t)C;   // f16 scale bytes per row (4-bit)
    float xr[CE];
    load_x<DT>(xb + (size_t)(a / A.k) * A.hidden, C, ns, xr);
    const mh_rsrc rx = gemv_rsrc(base, (uint32_t)A.stride);   // stride < 4 GiB: checked at launch
    const uint32_t od0 = (uint32_t)A.off[0], od1 = (uint32_t)A.off[3], os0 = (uint32_t)A.off[1],
                   os1 = (uint32_t)A.off[4];
    block_gemv<DT>(
        rx, rx,
        [&](int f) {
            const int m = f & 1;
            const uint32_t r = (uint32_t)(r0 + (f >> 1));
            return RowOff{(m ? od1 : od0) + mul24(r, rowbytes), (m ? os1 : os0) + mul24(r, srow)};
        },
        2 * nr, C, ns, xr, red, res);
    const float *bg = (const float *)(base + A.off[2]);
    const float *bu = (const float *)(base + A.off[5]);
    const float *rsg = (const float *)(base + A.off[1]);
    const float *rsu = (const float *)(base + A.off[4]);
    for (int i = threadIdx.x; i < nr; i += blockDim.x) {
        float g = res[2 * i], u = res[2 * i + 1];
        if constexpr (DT == MH_DT_Q8R) {
            g *= rsg[r0 + i];
            u *= rsu[r0 + i];
        }
        g += bg[r0 + i];
        u += bu[r0 + i];
        hout[r0 + i] = act_fn(g, u, A.alpha, A.limit, A.act_plain);
    }
}

// Down rows of the expert for assignment a: ye[a][r] = Wd[r] . h[a] + bd[r].
template <int DT>
__global__ void __launch_bounds__(kGemvThreads)
k_expert_down(ExpertArgs A, const int32_t *__restrict__ sel, const int32_t *__restrict__ order,
              const float *__restrict__ h, float *__restrict__ ye, int ns, int rpb) {
    constexpr int CE = gemv_chunk<DT>::E;
    extern __shared__ float lds[];
    const Assignment as = assignment_of(sel, order);
    const int a = as.a, e = as.e;
    const int r0 = blockIdx.x * rpb;
    const int nr = (int)min((int64_t)rpb, A.hidden - r0);
    float *yout = ye + (size_t)a * A.hidden;
    if (e < 0 || e >= A.E) {
        for (int i = threadIdx.x; i < nr; i += blockDim.x) yout[r0 + i] = 0.f;
        return;
    }
    const int C = (int)(A.ffn / CE);
    float *res = lds;
    float *red = lds + rpb;
    const uint8_t *base = A.experts + (uint64_t)e * A.stride;
    const uint32_t rowbytes = (uint32_t)C * 16u * gemv_chunk<DT>::W;
    const uint32_t srow = (DT == MH_DT_Q8R) ? 0u : 2u * (uint32_t)C;
    float xr[CE];
    load_x<DT>(h + (size_t)a * A.ffn, C, ns, xr);
    const mh_rsrc rx = gemv_rsrc(base, (uint32_t)A.stride);
    const uint32_t od = (uint32_t)A.off[6], os = (uint32_t)A.off[7];
    block_gemv<DT>(
        rx, rx,
        [&](int f) {
            const uint32_t r = (uint32_t)(r0 + f);
            return RowOff{od + mul24(r, rowbytes), os + mul24(r, srow)};
        },
        nr, C, ns, xr, red, res);
    const float *bd = (const float *)(base + A.off[8]);
    const float *rsd = (const float *)(base + A.off[7]);
    for (int i = threadIdx.x; i < nr; i += blockDim.x) {
        float v = res[i];
        if constexpr (DT == MH_DT_Q8R) v *= rsd[r0 + i];
        yout[r0 + i] = v + bd[r0 + i];
    }
}

// Decode combine (engine/midge.c:514, 544, 548): moe = sum_i w_i y_i in
// selection order, then x += moe; mul and add rounded separately (no FMA).
__global__ void __launch_bounds__(256)
k_combine_decode(float *__restrict__ x, const float *__restrict__ ye, const float *__restrict__ w, int64_t H,
                 int k) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= H) return;
    const float moe = slot_sum(w + (size_t)t * k, ye + (size_t)t * k * H, H, k, r);
    x[(size_t)t * H + r] = x[(size_t)t * H + r] + moe;
}

// The decode combine of one layer and the next layer's RMSNorm in one
// launch (one block of 1024 threads per token): x += moe exactly as
// k_combine_decode, then xb = x * inv * w exactly as k_rmsnorm (the same
// per-thread order of the squares and the same reductions), so the fused
// pair is bit-identical to the two launches.
__global__ void __launch_bounds__(1024)
k_combine_norm(float *__restrict__ x, const float *__restrict__ ye, const float *__restrict__ w, int64_t H, int k,
               const float *__restrict__ nw, float eps, float *__restrict__ xb) {
#pragma clang fp contract(off)
    __shared__ float part[16];
    const int t = blockIdx.x;
    float *xt = x + (size_t)t * H;
    float s = 0.f;
    for (int64_t r = threadIdx.x; r < H; r += blockDim.x) {
        const float moe = slot_sum(w + (size_t)t * k, ye + (size_t)t * k * H, H, k, r);
        const float v = xt[r] + moe;
        xt[r] = v;
        s = __builtin_fmaf(v, v, s);
    }
    s = mh_wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float ss = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) ss += part[i];
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int64_t r = threadIdx.x; r < H; r += blockDim.x) xb[(size_t)t * H + r] = xt[r] * inv * nw[r];
}

// The boundary between two layers of a decode of 2-16 tokens, in one launch:
// the previous layer's combine x += sum_i w_i y_i (as k_combine_norm; none
// before the first layer), this layer's RMSNorm (xb, as k_rmsnorm), its
// router logits, and per token the top-k and weights (wave_topk_token, as
// k_topk); the launch's last token sorts the assignments by expert.
//   Block (t, g) forms token t's x and xb itself (the same arithmetic in
//   every block of the token, bit-identical to the separate kernels) and
//   computes router rows [kCRRows g, +kCRRows), one per wave, the row's loads
//   issued first. The token's last block to arrive ranks the token and
//   writes its x back (every block of the token has read it by then); the
//   launch's last ranked token writes the order. Counters are left at zero.
constexpr int kCRRows = 16;       // router rows per block (one per wave)
constexpr int kCRMaxH = 3072;     // hidden (3 elements per thread)
// 16-byte chunks of a router row per lane: a row of kCRMaxH elements (int8:
// 3, f32: 12; loads past the row would re-read its last chunk)
template <int DT>
constexpr int cr_chunks() {
    return (kCRMaxH / mh_chunk<DT>::E + 63) / 64;
}

struct CombineRouteArgs {
    float *x;              // [n][H] residual (combined in place)
    const float *ye;       // [n k][H] the previous layer's expert outputs, or null
    const float *wprev;    // [n k] their weights
    int64_t H;
    int k;
    const float *nw;       // this layer's norm weights
    float eps;
    float *xb;             // [n][H] out
    const uint8_t *rw;     // router rows [E][H] (int8 or f32)
    const float *rs;       // int8 row scales [E]
    const float *rb;       // router bias [E] or null
    int E, router_norm, unfilled, n;
    float *rl;             // [n][E] logits (scratch)
    int32_t *sel;          // [n][k] out
    float *w;              // [n][k] out
    uint32_t *usage;       // [E] or null
    int32_t *order;        // [2 n k] out
    unsigned *cnt;         // [n + 1] arrival counters
};

template <int DT, int PER>
__global__ void __launch_bounds__(1024) k_combine_route(CombineRouteArgs A) {
#pragma clang fp contract(off)
    __shared__ float part[16];
    __shared__ __attribute__((aligned(16))) float s_xb[kCRMaxH];
    __shared__ int s_last;
    __shared__ int skey[kMaxOrder];
    constexpr int CE = mh_chunk<DT>::E;
    constexpr int kV = kCRMaxH / 1024;
    const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t H = A.H;
    const int C = (int)(H / CE), E = A.E, k = A.k;
    // this wave's router row: its loads first (they wait for nothing)
    const int e = g * kCRRows + wave;
    const bool has_row = e < E;   // wave-uniform
    const mh_rsrc rr = gemv_rsrc(A.rw, (uint32_t)E * (uint32_t)C * 16u);
    const int er = min(e, E - 1);
    constexpr int kCRChunks = cr_chunks<DT>();
    mh_u4 q[kCRChunks];
#pragma unroll
    for (int j = 0; j < kCRChunks; ++j) {
        const int c = min(lane + 64 * j, C - 1);   // past the row: the last chunk again, not used
        q[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(er * C + c) * 16u, 0, 0);
    }
    // x (combined) and the sum of its squares, as k_combine_norm / k_rmsnorm
    float *xt = A.x + (size_t)t * H;
    float v[kV];
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < kV; ++u) {
        const int64_t r = tid + 1024 * u;
        v[u] = 0.f;
        if (r < H) {
            if (A.ye) {
                v[u] = xt[r] + slot_sum(A.wprev + (size_t)t * k, A.ye + (size_t)t * k * H, H, k, r);
            } else {
                v[u] = xt[r];
            }
            s = __builtin_fmaf(v[u], v[u], s);
        }
    }
    s = mh_wave_sum(s);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    float ss = 0.f;
    for (int i = 0; i < 16; ++i) ss += part[i];
    const float inv = 1.0f / sqrtf(ss / (float)H + A.eps);
#pragma unroll
    for (int u = 0; u < kV; ++u) {
        const int64_t r = tid + 1024 * u;
        if (r < H) {
            const float xbv = v[u] * inv * A.nw[r];
            s_xb[r] = xbv;
            if (g == 0) A.xb[(size_t)t * H + r] = xbv;
        }
    }
    __syncthreads();
    // router row e of token t
    if (has_row) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < kCRChunks; ++j) {
            const int c = lane + 64 * j;
            if (c < C) acc += mh_dot_chunk<DT>(q[j], s_xb + c * CE);
        }
        acc = mh_wave_sum(acc);
        if (lane == 0) {
            float p = acc;
            if constexpr (DT == MH_DT_Q8R) p *= A.rs[e];
            __hip_atomic_store(&A.rl[(size_t)t * E + e], p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // the token's blocks count themselves in; the last ranks the token (one
    // thread's acquire serves the block: its invalidation covers the CU's
    // cache and the L2 that every wave reads through)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last = __hip_atomic_fetch_add(&A.cnt[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          gridDim.y - 1;
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(&A.cnt[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    if (A.ye) {
#pragma unroll
        for (int u = 0; u < kV; ++u) {
            const int64_t r = tid + 1024 * u;
            if (r < H) xt[r] = v[u];
        }
    }
    if (wave == 0)
        wave_topk_token<PER>(A.rl + (size_t)t * E, A.rb, E, k, A.router_norm, A.unfilled, A.sel + (size_t)t * k,
                             A.w + (size_t)t * k, A.usage);
    // the launch's last ranked token sorts the assignments (as k_topk)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last =
            __hip_atomic_fetch_add(&A.cnt[A.n], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)A.n - 1u;
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(&A.cnt[A.n], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    const int N = A.n * k;
    for (int i = tid; i < N; i += 1024) {
        const int se = A.sel[i];
        skey[i] = (se >= 0 && se < E ? se : E) * N + i;   // distinct keys
    }
    __syncthreads();
    for (int i = tid; i < N; i += 1024) {
        const int ki = skey[i];
        const int r = key_rank(skey, N, ki);
        A.order[r] = i;
        A.order[N + r] = ki / N < E ? ki / N : -1;
    }
}

// zeroes n words (a fill kernel: no memset node in a caller's graph)
__global__ void k_zero_u32(uint32_t *p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Prefill combine (engine/midge.c:595-611, 465-466): each token's
// contributions are added straight into its residual in ascending expert
// order (slot order among equal ids, as the reference's loops give).
__global__ void __launch_bounds__(256)
k_combine_prefill(float *__restrict__ x, const float *__restrict__ ye, const int32_t *__restrict__ sel,
                  const float *__restrict__ w, int64_t H, int k, int E) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= H) return;
    int order[kMaxTopK];
    for (int i = 0; i < k; ++i) order[i] = i;
    for (int i = 1; i < k; ++i) {   // insertion sort by expert id, stable
        int j = i, oi = order[i];
        while (j > 0 && sel[(size_t)t * k + order[j - 1]] > sel[(size_t)t * k + oi]) {
            order[j] = order[j - 1];
            --j;
        }
        order[j] = oi;
    }
    float acc = x[(size_t)t * H + r];
    for (int j = 0; j < k; ++j) {
        const int i = order[j];
        const int e = sel[(size_t)t * k + i];
        if (e < 0 || e >= E) continue;   // an unroutable slot adds nothing (its ye row is not written)
        acc = acc + w[(size_t)t * k + i] * ye[((size_t)t * k + i) * H + r];
    }
    x[(size_t)t * H + r] = acc;
}

// k_combine_prefill on 4 consecutive elements per thread (16-byte loads and
// stores; H % 4 == 0 and 16-byte aligned rows): each element gets the same
// adds in the same order.
__global__ void __launch_bounds__(256)
k_combine_prefill4(float *__restrict__ x, const float *__restrict__ ye, const int32_t *__restrict__ sel,
                   const float *__restrict__ w, int64_t H, int k, int E) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int64_t r = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (r >= H) return;
    int order[kMaxTopK];
    for (int i = 0; i < k; ++i) order[i] = i;
    for (int i = 1; i < k; ++i) {   // insertion sort by expert id, stable
        int j = i, oi = order[i];
        while (j > 0 && sel[(size_t)t * k + order[j - 1]] > sel[(size_t)t * k + oi]) {
            order[j] = order[j - 1];
            --j;
        }
        order[j] = oi;
    }
    float4 acc = *(const float4 *)(x + (size_t)t * H + r);
    for (int j = 0; j < k; ++j) {
        const int i = order[j];
        const int e = sel[(size_t)t * k + i];
        if (e < 0 || e >= E) continue;   // an unroutable slot adds nothing (its ye row is not written)
        const float wi = w[(size_t)t * k + i];
        const float4 v = *(const float4 *)(ye + ((size_t)t * k + i) * H + r);
        acc.x = acc.x + wi * v.x;
        acc.y = acc.y + wi * v.y;
        acc.z = acc.z + wi * v.z;
        acc.w = acc.w + wi * v.w;
    }
    *(float4 *)(x + (size_t)t * H + r) = acc;
}

template <int DT>
int launch_experts_t(const DevLayer &L, int A, const int32_t *sel, const int32_t *order, const float *xb, float *h,
                     float *ye, hipStream_t s) {
    constexpr int CE = gemv_chunk<DT>::E;
    ExpertArgs ea;
    ea.experts = L.experts;
    ea.stride = L.expert_stride;
    for (int i = 0; i < 9; i++) ea.off[i] = L.off[i];
    ea.E = L.n_experts;
    ea.k = L.top_k;
    ea.hidden = L.hidden;
    ea.ffn = L.ffn;
    ea.alpha = L.alpha;
    ea.limit = L.limit;
    ea.act_plain = L.act_plain;
    const int64_t target = (int64_t)device_cus() * 2;
    {   // gate/up: 2 * ffn flat rows per assignment
        const int C = (int)(L.hidden / CE);
        int ns, nt;
        gemv_shape(C, &ns, &nt);
        int64_t per = (L.ffn * A + target - 1) / target;   // rows per block
        int64_t step = (ns + 1) / 2;
        int64_t rpb = ((per + step - 1) / step) * step;
        if (rpb < step) rpb = step;
        if (rpb > 2048) rpb = 2048;
        const int64_t nblk = (L.ffn + rpb - 1) / rpb;
        const size_t lds = ((size_t)2 * rpb + gemv_lds_floats(ns, C)) * sizeof(float);
        MH_LAUNCH("expert_gu", k_expert_gu<DT>, dim3((unsigned)nblk, (unsigned)A), dim3(nt), lds, s, ea, sel, order, xb,
                           h, ns, (int)rpb);
        MH_TRY(hip_check(hipGetLastError(), "expert gate/up launch"));
    }
    {   // down: hidden rows per assignment
        const int C = (int)(L.ffn / CE);
        int ns, nt;
        gemv_shape(C, &ns, &nt);
        int64_t per = (L.hidden * A + target - 1) / target;
        int64_t rpb = ((per + ns - 1) / ns) * ns;
        if (rpb < ns) rpb = ns;
        if (rpb > 4096) rpb = 4096;
        const int64_t nblk = (L.hidden + rpb - 1) / rpb;
        const size_t lds = ((size_t)rpb + gemv_lds_floats(ns, C)) * sizeof(float);
        MH_LAUNCH("expert_down", k_expert_down<DT>, dim3((unsigned)nblk, (unsigned)A), dim3(nt), lds, s, ea, sel, order, h,
                           ye, ns, (int)rpb);
        MH_TRY(hip_check(hipGetLastError(), "expert down launch"));
    }
    return MH_OK;
}

// order: null (grid row y = assignment y) or the expert-sorted order of k_topk.
int launch_experts(const DevLayer &L, int A, const int32_t *sel, const int32_t *order, const float *xb, float *h,
                   float *ye, hipStream_t s) {
    switch (L.expert_dt) {
    case MH_DT_F32: return launch_experts_t<MH_DT_F32>(L, A, sel, order, xb, h, ye, s);
    case MH_DT_Q8R: return launch_experts_t<MH_DT_Q8R>(L, A, sel, order, xb, h, ye, s);
    case MH_DT_Q4G32: return launch_experts_t<MH_DT_Q4G32>(L, A, sel, order, xb, h, ye, s);
    case MH_DT_MXFP4: return launch_experts_t<MH_DT_MXFP4>(L, A, sel, order, xb, h, ye, s);
    }
    return fail(MH_E_DTYPE, "unknown expert dtype %d", L.expert_dt);
}

// order: null, or [2 n k] for the expert-sorted assignment order (n <= 16).
int launch_topk(const float *rl, const float *bias, int n, int E, int k, int router_norm, int unfilled,
                int32_t *sel, float *w, uint32_t *usage, int32_t *order, hipStream_t s) {
    if (order && (n > 16 || n * k > kMaxOrder)) return fail(MH_E_ARG, "topk: %d x %d assignments to order", n, k);
    const int per_block = order ? n : 4;
    const dim3 grid((unsigned)((n + per_block - 1) / per_block)), block(64 * per_block);
    // logits per lane: the smallest instantiation that holds E (E <= kMaxExperts)
    if (E <= 128)
        MH_LAUNCH("topk", k_topk<2>, grid, block, 0, s, rl, bias, n, E, k, router_norm, unfilled, sel, w, usage,
                  order);
    else if (E <= 256)
        MH_LAUNCH("topk", k_topk<4>, grid, block, 0, s, rl, bias, n, E, k, router_norm, unfilled, sel, w, usage,
                  order);
    else
        MH_LAUNCH("topk", k_topk<kMaxExperts / 64>, grid, block, 0, s, rl, bias, n, E, k, router_norm, unfilled, sel,
                  w, usage, order);
    return hip_check(hipGetLastError(), "topk launch");
}

// The layer boundary of a decode of 2-16 tokens in one launch
// (k_combine_route): MH_E_UNSUPPORTED (error cleared) for shapes it does not
// take. ye / wprev null: the first layer (no combine).
bool combine_route_ok(const DevLayer &L, int n) {
    const int CE = L.router.dt == MH_DT_Q8R ? 16 : 4;
    const int chunks = L.router.dt == MH_DT_Q8R ? cr_chunks<MH_DT_Q8R>() : cr_chunks<MH_DT_F32>();
    return (L.router.dt == MH_DT_Q8R || L.router.dt == MH_DT_F32) && n >= 1 && n <= 16 &&
           n * L.top_k <= kMaxOrder && L.hidden <= kCRMaxH && L.hidden % CE == 0 &&
           L.hidden / CE <= 64 * chunks && L.n_experts <= kMaxExperts && (uintptr_t)L.router.data % 16 == 0 &&
           (uint64_t)L.n_experts * (uint64_t)L.hidden * (L.router.dt == MH_DT_Q8R ? 1u : 4u) < (1ull << 32);
}

int launch_combine_route(const DevLayer &L, float *x, const float *ye, const float *wprev, int n, float *xb,
                         float *rl, int32_t *sel, float *w, uint32_t *usage, int32_t *order, hipStream_t s) {
    if (!combine_route_ok(L, n)) return MH_E_UNSUPPORTED;
    void *cp = nullptr;
    bool fresh = false;
    MH_TRY(scratch(S_CROUTE, sizeof(unsigned) * 17, &cp, &fresh));
    if (fresh) {
        MH_LAUNCH("zero_counters", k_zero_u32, dim3(1), dim3(64), 0, s, (uint32_t *)cp, 17);
        MH_TRY(hip_check(hipGetLastError(), "counter clear"));
    }
    CombineRouteArgs A;
    A.x = x;
    A.ye = ye;
    A.wprev = wprev;
    A.H = L.hidden;
    A.k = L.top_k;
    A.nw = L.mlp_norm;
    A.eps = L.norm_eps;
    A.xb = xb;
    A.rw = L.router.data;
    A.rs = (const float *)L.router.scales;
    A.rb = L.router_b;
    A.E = L.n_experts;
    A.router_norm = L.router_norm;
    A.unfilled = -1;
    A.n = n;
    A.rl = rl;
    A.sel = sel;
    A.w = w;
    A.usage = usage;
    A.order = order;
    A.cnt = (unsigned *)cp;
    const dim3 grid((unsigned)n, (unsigned)((L.n_experts + kCRRows - 1) / kCRRows));
#define CR_LAUNCH(DT, PER) MH_LAUNCH("combine_route", (k_combine_route<DT, PER>), grid, dim3(1024), 0, s, A)
    if (L.router.dt == MH_DT_Q8R) {
        if (L.n_experts <= 128) CR_LAUNCH(MH_DT_Q8R, 2);
        else if (L.n_experts <= 256) CR_LAUNCH(MH_DT_Q8R, 4);
        else CR_LAUNCH(MH_DT_Q8R, kMaxExperts / 64);
    } else {
        if (L.n_experts <= 128) CR_LAUNCH(MH_DT_F32, 2);
        else if (L.n_experts <= 256) CR_LAUNCH(MH_DT_F32, 4);
        else CR_LAUNCH(MH_DT_F32, kMaxExperts / 64);
    }
#undef CR_LAUNCH
    return hip_check(hipGetLastError(), "combine/route launch");
}

// Scratch for a layer call of n tokens.
struct LayerBufs {
    float *xb, *rl, *h, *ye;
    int32_t *sel;
    float *w;
    int32_t *order;   // [2 n k] expert-sorted assignments (n <= 16), else null
};

int layer_bufs(const DevLayer &L, int n, LayerBufs *b) {
    void *p;
    MH_TRY(scratch(S_XB, (uint64_t)n * L.hidden * 4, &p));
    b->xb = (float *)p;
    MH_TRY(scratch(S_RL, (uint64_t)n * L.n_experts * 4, &p));
    b->rl = (float *)p;
    MH_TRY(scratch(S_H, (uint64_t)n * L.top_k * L.ffn * 4, &p));
    b->h = (float *)p;
    MH_TRY(scratch(S_YE, (uint64_t)n * L.top_k * L.hidden * 4, &p));
    b->ye = (float *)p;
    MH_TRY(scratch(S_SEL, (uint64_t)n * L.top_k * 4, &p));
    b->sel = (int32_t *)p;
    MH_TRY(scratch(S_W, (uint64_t)n * L.top_k * 4, &p));
    b->w = (float *)p;
    b->order = nullptr;
    if (n <= 16) {
        MH_TRY(scratch(S_ORD, (uint64_t)2 * n * L.top_k * 4, &p));
        b->order = (int32_t *)p;
    }
    return MH_OK;
}

// Router (rmsnorm, logits, top-k) for n tokens into b->xb / b->sel / b->w
// (and the expert-sorted order into `order` when it is not null).
// x null: b.xb already holds rmsnorm(x) of this layer (k_combine_norm).
int run_router(const DevLayer &L, const float *x, int n, int unfilled, const LayerBufs &b, uint32_t *usage,
               int32_t *order, hipStream_t s) {
    if (x) MH_TRY(launch_rmsnorm(x, L.mlp_norm, b.xb, L.hidden, L.norm_eps, n, s));
    MH_TRY(launch_gemv(L.router, b.xb, b.rl, n, s));
    return launch_topk(b.rl, L.router_b, n, L.n_experts, L.top_k, L.router_norm, unfilled, b.sel, b.w, usage, order,
                       s);
}

// few: the layer's MXFP4 scales are known to be f16-exact (a stack's plan
// scanned them), so 2-16 tokens take the expert-grouped matrix-core kernels
// (each routed expert read once for its tokens); the BATCH_GEMV switch, or
// a layer they cannot run, keeps the per-assignment GEMVs.
// have_xb: b.xb holds this layer's normed input already; next: the next
// layer, whose RMSNorm is fused into this layer's combine (or null).
int run_decode_layer(const DevLayer &L, float *x, int n, const LayerBufs &b, uint32_t *usage, hipStream_t s,
                     bool few = false, bool have_xb = false, const DevLayer *next = nullptr) {
    MH_TRY(run_router(L, have_xb ? nullptr : x, n, -1, b, usage, b.order, s));
    if (few && b.order && !sw(SW_BATCH_GEMV) && grouped_ok(L, n))
        MH_TRY(launch_grouped(L, n, b.order, b.xb, b.h, b.ye, s));
    else
        MH_TRY(launch_experts(L, n * L.top_k, b.sel, b.order, b.xb, b.h, b.ye, s));
    if (next) {
        MH_LAUNCH("combine_norm", k_combine_norm, dim3((unsigned)n), dim3(1024), 0, s, x, b.ye, b.w, L.hidden, L.top_k,
                  next->mlp_norm, next->norm_eps, b.xb);
    } else {
        MH_LAUNCH("combine_decode", k_combine_decode, dim3((unsigned)((L.hidden + 255) / 256), (unsigned)n), dim3(256),
                  0, s, x, b.ye, b.w, L.hidden, L.top_k);
    }
    return hip_check(hipGetLastError(), "combine launch");
}

// The scaled-MFMA grouped GEMM takes a chunk once its experts average at
// least this many assignments: its 32-token tiles are then at least a
// quarter full. Below that the per-assignment GEMVs do no more work, and
// they keep f32 arithmetic (the GEMM carries activations as three fp6 terms,
// ~12 significant bits, and its instruction cuts each product to ~2^-13 of
// the largest one it sums; a small, sharply peaked model can amplify that
// to a few 1e-4 of relative error in its logits).
constexpr int kMfmaMinPerExpert = 8;

int run_expert_major(const DevLayer &L, int n, const float *xb, const int32_t *sel, const float *w, float *x,
                     const LayerBufs &b, hipStream_t s) {
    if (prefill_mfma_ok(L) && (int64_t)n * L.top_k >= (int64_t)kMfmaMinPerExpert * L.n_experts)
        MH_TRY(run_expert_major_mfma(L, n, xb, sel, b.ye, s));
    else MH_TRY(launch_experts(L, n * L.top_k, sel, nullptr, xb, b.h, b.ye, s));
    if (L.hidden % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)b.ye % 16 == 0)
        MH_LAUNCH("combine_prefill", k_combine_prefill4, dim3((unsigned)((L.hidden / 4 + 255) / 256), (unsigned)n),
                  dim3(256), 0, s, x, b.ye, sel, w, L.hidden, L.top_k, L.n_experts);
    else
        MH_LAUNCH("combine_prefill", k_combine_prefill, dim3((unsigned)((L.hidden + 255) / 256), (unsigned)n), dim3(256), 0,
                  s, x, b.ye, sel, w, L.hidden, L.top_k, L.n_experts);
    return hip_check(hipGetLastError(), "prefill combine launch");
}

int check_tokens(int n, const char *what) {
    if (n < 1 || n > 65535) return fail(MH_E_ARG, "%s: token count %d out of range [1, 65535]", what, n);
    return MH_OK;
}

}  // namespace

int validate_layer(const mh_moe_layer *L) {
    if (!L) return fail(MH_E_ARG, "NULL layer");
    if (L->hidden < 1 || L->ffn < 1 || L->n_experts < 1)
        return fail(MH_E_ARG, "layer: hidden=%lld ffn=%lld experts=%d", (long long)L->hidden, (long long)L->ffn,
                    L->n_experts);
    if (L->top_k < 1 || L->top_k > kMaxTopK || L->top_k > L->n_experts)
        return fail(MH_E_ARG, "layer: top_k=%d must be in [1, min(16, experts=%d)]", L->top_k, L->n_experts);
    if (L->n_experts > kMaxExperts) return fail(MH_E_UNSUPPORTED, "layer: %d experts > %d", L->n_experts, kMaxExperts);
    // the layout must be wt_expert_layout()'s (engine/mten.h:136-150)
    uint64_t off[9], pos = 0;
    int64_t rows[3] = {L->ffn, L->ffn, L->hidden}, cols[3] = {L->hidden, L->hidden, L->ffn};
    for (int m = 0; m < 3; m++) {
        uint64_t db, sb;
        MH_TRY(wt_bytes(L->expert_dt, rows[m], cols[m], &db, &sb));
        off[3 * m] = pos;
        pos = (pos + db + 63) & ~63ull;
        off[3 * m + 1] = pos;
        pos = (pos + sb + 63) & ~63ull;
        off[3 * m + 2] = pos;
        pos = (pos + (uint64_t)rows[m] * 4 + 63) & ~63ull;
    }
    for (int i = 0; i < 9; i++)
        if (off[i] != L->off[i])
            return fail(MH_E_ARG, "layer: off[%d]=%llu, expected %llu from the expert layout", i,
                        (unsigned long long)L->off[i], (unsigned long long)off[i]);
    if (L->expert_stride != ((pos + 63) & ~63ull))
        return fail(MH_E_ARG, "layer: expert_stride=%llu, expected %llu", (unsigned long long)L->expert_stride,
                    (unsigned long long)((pos + 63) & ~63ull));
    if (L->expert_stride > 0xFFFFFFFFull)   // the kernels address an expert with 32-bit offsets
        return fail(MH_E_UNSUPPORTED, "layer: expert_stride=%llu exceeds 4 GiB", (unsigned long long)L->expert_stride);
    // elements per chunk of the GEMV engine (gemv_chunk<DT>::E)
    const int ce = (L->expert_dt == MH_DT_F32) ? 4 : 32;
    if (L->hidden % ce || L->ffn % ce || L->hidden / ce > kGemvThreads || L->ffn / ce > kGemvThreads)
        return fail(MH_E_UNSUPPORTED, "layer: hidden=%lld / ffn=%lld not a multiple of %d elements or wider "
                    "than %d chunks", (long long)L->hidden, (long long)L->ffn, ce, kGemvThreads);
    if (L->router.rows != L->n_experts || L->router.cols != L->hidden)
        return fail(MH_E_ARG, "layer: router is %lld x %lld, expected %d x %lld", (long long)L->router.rows,
                    (long long)L->router.cols, L->n_experts, (long long)L->hidden);
    return MH_OK;
}

int resolve_layer(const mh_moe_layer *L, DevLayer *out) {
    MH_TRY(validate_layer(L));
    out->hidden = L->hidden;
    out->ffn = L->ffn;
    out->n_experts = L->n_experts;
    out->top_k = L->top_k;
    out->alpha = L->alpha;
    out->limit = L->limit;
    out->norm_eps = L->norm_eps;
    out->act_plain = L->act_plain ? 1 : 0;
    out->router_norm = L->router_norm ? 1 : 0;
    out->expert_dt = L->expert_dt;
    out->expert_stride = L->expert_stride;
    for (int i = 0; i < 9; i++) out->off[i] = L->off[i];
    const void *p;
    MH_TRY(resolve_weight(L->experts, L->expert_stride * (uint64_t)L->n_experts, &p, "layer experts"));
    out->experts = (const uint8_t *)p;
    MH_TRY(resolve_wt(&L->router, &out->router, "layer router"));
    MH_TRY(resolve_weight(L->router_b, (uint64_t)L->n_experts * 4, &p, "layer router_b"));
    out->router_b = (const float *)p;
    MH_TRY(resolve_weight(L->mlp_norm, (uint64_t)L->hidden * 4, &p, "layer mlp_norm"));
    out->mlp_norm = (const float *)p;
    return MH_OK;
}

}  // namespace mh

struct mh_stack {
    std::vector<mh::DevLayer> layers;
    int max_batch;
    mh::StepPlan *plan = nullptr;   // one-launch batch-1 path (null/ineligible -> per-layer launches)
};

namespace mh {

// Layer l of a stack for one token on device x (the one-launch kernel when
// the plan holds, else the per-layer launches); sel, w (device [k]) and
// usage (device [E]) are this layer's rows, or null.
int stack_decode_layer(mh_stack *st, int l, float *x, int32_t *sel, float *w, uint32_t *usage) {
    hipStream_t s = stream();
    if (!sw(SW_NO_FUSED) && step_plan_ok(st->plan)) {
        int rc = step_run(st->plan, st->layers.data(), l, 1, x, sel, w, usage, s);
        if (rc != MH_E_UNSUPPORTED) return rc;
        clear_error();
    }
    const DevLayer &L = st->layers[(size_t)l];
    LayerBufs b;
    MH_TRY(layer_bufs(L, 1, &b));
    if (sel) b.sel = sel;
    if (w) b.w = w;
    return run_decode_layer(L, x, 1, b, usage, s);
}

// One-layer plans of the one-launch decode kernel for the layers that
// mh_moe and mh_moe_dev see at batch 1, keyed by the resolved layer (its
// device pointers and parameters): made on a layer's first call (the plan
// scans the layer's down scales once), kept until mh_shutdown releases them
// (the cache is dropped when the initialisation changes) or the cache is
// full (then its oldest plan goes). A layer no plan can run keeps a null
// entry and takes the per-layer launches.
struct LayerPlanKey {
    const void *experts, *router, *router_s, *router_b, *norm;
    int64_t hidden, ffn;
    int E, k, rdt, edt, act_plain, router_norm;
    float alpha, limit, eps;
    uint64_t stride;
    bool operator==(const LayerPlanKey &o) const {
        return experts == o.experts && router == o.router && router_s == o.router_s && router_b == o.router_b &&
               norm == o.norm && hidden == o.hidden && ffn == o.ffn && E == o.E && k == o.k && rdt == o.rdt &&
               edt == o.edt && act_plain == o.act_plain && router_norm == o.router_norm && alpha == o.alpha &&
               limit == o.limit && eps == o.eps && stride == o.stride;
    }
};
struct LayerPlans {
    uint64_t epoch = 0;
    std::vector<std::pair<LayerPlanKey, StepPlan *>> plans;
};
LayerPlans g_lplans;
constexpr size_t kLayerPlans = 256;

StepPlan *layer_plan(const DevLayer &L) {
    if (g_lplans.epoch != init_epoch()) {
        // plans of an earlier initialisation: mh_shutdown released their memory
        for (auto &e : g_lplans.plans) step_plan_destroy(e.second);
        g_lplans.plans.clear();
        g_lplans.epoch = init_epoch();
    }
    const LayerPlanKey key{L.experts,    L.router.data, L.router.scales, L.router_b, L.mlp_norm,
                           L.hidden,     L.ffn,         L.n_experts,     L.top_k,    L.router.dt,
                           L.expert_dt,  L.act_plain,   L.router_norm,   L.alpha,    L.limit,
                           L.norm_eps,   L.expert_stride};
    for (auto &e : g_lplans.plans)
        if (e.first == key) return e.second;
    StepPlan *p = nullptr;
    if (step_plan_create(&L, 1, &p) != MH_OK || !step_plan_ok(p)) {
        clear_error();
        if (p) step_plan_destroy(p);
        p = nullptr;
    }
    if (g_lplans.plans.size() >= kLayerPlans) {
        step_plan_destroy(g_lplans.plans.front().second);
        g_lplans.plans.erase(g_lplans.plans.begin());
    }
    g_lplans.plans.push_back({key, p});
    return p;
}

// moe() for one token on device x through the layer's one-launch plan:
// MH_E_UNSUPPORTED (error cleared) when no plan runs this layer.
int one_launch_layer(const DevLayer &L, float *x, int32_t *sel, float *w, hipStream_t s) {
    StepPlan *p = sw(SW_NO_FUSED) ? nullptr : layer_plan(L);
    if (!p) return MH_E_UNSUPPORTED;
    const int rc = step_run(p, &L, 0, 1, x, sel, w, nullptr, s);
    if (rc == MH_E_UNSUPPORTED) clear_error();
    return rc;
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_moe_dev(const mh_moe_layer *Lh, float *x, int batch, int32_t *sel, float *w) {
    clear_error();
    MH_TRY(check_tokens(batch, "mh_moe_dev"));
    MH_TRY(validate_layer(Lh));
    MH_TRY(require_init());
    DevLayer L;
    MH_TRY(resolve_layer(Lh, &L));
    MH_TRY(resolve_dev(x, (uint64_t)batch * L.hidden * 4, "mh_moe_dev x"));
    if (sel) MH_TRY(resolve_dev(sel, (uint64_t)batch * L.top_k * 4, "mh_moe_dev sel"));
    if (w) MH_TRY(resolve_dev(w, (uint64_t)batch * L.top_k * 4, "mh_moe_dev w"));
    LayerBufs b;
    MH_TRY(layer_bufs(L, batch, &b));
    hipStream_t s = stream();
    if (batch == 1) {   // the one-launch kernel when a plan runs the layer
        const int rc = one_launch_layer(L, x, sel ? sel : b.sel, w ? w : b.w, s);
        if (rc != MH_E_UNSUPPORTED) return rc;
    }
    MH_TRY(run_decode_layer(L, x, batch, b, nullptr, s));
    if (sel) MH_HIP(hipMemcpyAsync(sel, b.sel, (size_t)batch * L.top_k * 4, hipMemcpyDeviceToDevice, s));
    if (w) MH_HIP(hipMemcpyAsync(w, b.w, (size_t)batch * L.top_k * 4, hipMemcpyDeviceToDevice, s));
    return MH_OK;
}

int mh_moe(const mh_moe_layer *Lh, float *x, int32_t *sel, float *w) {
    clear_error();
    if (!x) return fail(MH_E_ARG, "mh_moe: NULL x");
    MH_TRY(validate_layer(Lh));
    MH_TRY(require_init());
    DevLayer L;
    MH_TRY(resolve_layer(Lh, &L));
    void *dx;
    MH_TRY(scratch(S_X, (uint64_t)L.hidden * 4, &dx));
    LayerBufs b;
    MH_TRY(layer_bufs(L, 1, &b));
    hipStream_t s = stream();
    MH_HIP(hipMemcpyAsync(dx, x, (size_t)L.hidden * 4, hipMemcpyHostToDevice, s));
    // the one-launch kernel when a plan runs the layer, else the per-layer launches
    const int rc = one_launch_layer(L, (float *)dx, b.sel, b.w, s);
    if (rc == MH_E_UNSUPPORTED) MH_TRY(run_decode_layer(L, (float *)dx, 1, b, nullptr, s));
    else if (rc) return rc;
    MH_HIP(hipMemcpyAsync(x, dx, (size_t)L.hidden * 4, hipMemcpyDeviceToHost, s));
    if (sel) MH_HIP(hipMemcpyAsync(sel, b.sel, (size_t)L.top_k * 4, hipMemcpyDeviceToHost, s));
    if (w) MH_HIP(hipMemcpyAsync(w, b.w, (size_t)L.top_k * 4, hipMemcpyDeviceToHost, s));
    return sync_checked(s);
}

int mh_topk_dev(const float *logits, int n, int E, int k, int router_norm, int32_t *sel, float *w) {
    clear_error();
    MH_TRY(check_tokens(n, "mh_topk_dev"));
    if (E < 1 || E > kMaxExperts) return fail(MH_E_ARG, "mh_topk_dev: experts=%d out of [1, %d]", E, kMaxExperts);
    if (k < 1 || k > kMaxTopK || k > E) return fail(MH_E_ARG, "mh_topk_dev: k=%d out of [1, min(16, %d)]", k, E);
    MH_TRY(require_init());
    MH_TRY(resolve_dev(logits, (uint64_t)n * E * 4, "mh_topk_dev logits"));
    MH_TRY(resolve_dev(sel, (uint64_t)n * k * 4, "mh_topk_dev sel"));
    MH_TRY(resolve_dev(w, (uint64_t)n * k * 4, "mh_topk_dev w"));
    return launch_topk(logits, nullptr, n, E, k, router_norm ? 1 : 0, 0, sel, w, nullptr, nullptr, stream());
}

int mh_expert_major_dev(const mh_moe_layer *Lh, int n, const float *xb, const int32_t *sel, const float *w,
                        float *x) {
    clear_error();
    MH_TRY(check_tokens(n, "mh_expert_major_dev"));
    MH_TRY(validate_layer(Lh));
    MH_TRY(require_init());
    DevLayer L;
    MH_TRY(resolve_layer(Lh, &L));
    MH_TRY(resolve_dev(xb, (uint64_t)n * L.hidden * 4, "mh_expert_major_dev xb"));
    MH_TRY(resolve_dev(sel, (uint64_t)n * L.top_k * 4, "mh_expert_major_dev sel"));
    MH_TRY(resolve_dev(w, (uint64_t)n * L.top_k * 4, "mh_expert_major_dev w"));
    MH_TRY(resolve_dev(x, (uint64_t)n * L.hidden * 4, "mh_expert_major_dev x"));
    LayerBufs b;
    MH_TRY(layer_bufs(L, n, &b));
    return run_expert_major(L, n, xb, sel, w, x, b, stream());
}

int mh_moe_prefill_dev(const mh_moe_layer *Lh, int n, float *x, int32_t *sel, float *w) {
    clear_error();
    MH_TRY(check_tokens(n, "mh_moe_prefill_dev"));
    MH_TRY(validate_layer(Lh));
    MH_TRY(require_init());
    DevLayer L;
    MH_TRY(resolve_layer(Lh, &L));
    MH_TRY(resolve_dev(x, (uint64_t)n * L.hidden * 4, "mh_moe_prefill_dev x"));
    if (sel) MH_TRY(resolve_dev(sel, (uint64_t)n * L.top_k * 4, "mh_moe_prefill_dev sel"));
    if (w) MH_TRY(resolve_dev(w, (uint64_t)n * L.top_k * 4, "mh_moe_prefill_dev w"));
    LayerBufs b;
    MH_TRY(layer_bufs(L, n, &b));
    hipStream_t s = stream();
    MH_TRY(run_router(L, x, n, 0, b, nullptr, nullptr, s));
    MH_TRY(run_expert_major(L, n, b.xb, b.sel, b.w, x, b, s));
    if (sel) MH_HIP(hipMemcpyAsync(sel, b.sel, (size_t)n * L.top_k * 4, hipMemcpyDeviceToDevice, s));
    if (w) MH_HIP(hipMemcpyAsync(w, b.w, (size_t)n * L.top_k * 4, hipMemcpyDeviceToDevice, s));
    return MH_OK;
}

int mh_moe_prefill(const mh_moe_layer *Lh, int n, float *x, int32_t *sel, float *w) {
    clear_error();
    MH_TRY(check_tokens(n, "mh_moe_prefill"));
    if (!x) return fail(MH_E_ARG, "mh_moe_prefill: NULL x");
    MH_TRY(validate_layer(Lh));
    MH_TRY(require_init());
    DevLayer L;
    MH_TRY(resolve_layer(Lh, &L));
    void *dx;
    MH_TRY(scratch(S_X, (uint64_t)n * L.hidden * 4, &dx));
    LayerBufs b;
    MH_TRY(layer_bufs(L, n, &b));
    hipStream_t s = stream();
    const size_t xbytes = (size_t)n * L.hidden * 4, kbytes = (size_t)n * L.top_k * 4;
    MH_HIP(hipMemcpyAsync(dx, x, xbytes, hipMemcpyHostToDevice, s));
    MH_TRY(run_router(L, (float *)dx, n, 0, b, nullptr, nullptr, s));
    MH_TRY(run_expert_major(L, n, b.xb, b.sel, b.w, (float *)dx, b, s));
    MH_HIP(hipMemcpyAsync(x, dx, xbytes, hipMemcpyDeviceToHost, s));
    if (sel) MH_HIP(hipMemcpyAsync(sel, b.sel, kbytes, hipMemcpyDeviceToHost, s));
    if (w) MH_HIP(hipMemcpyAsync(w, b.w, kbytes, hipMemcpyDeviceToHost, s));
    return sync_checked(s);
}

int mh_stack_create(const mh_moe_layer *layers, int n_layers, int max_batch, mh_stack **out) {
    clear_error();
    if (!layers || !out || n_layers < 1) return fail(MH_E_ARG, "mh_stack_create: NULL layers/out or n_layers < 1");
    MH_TRY(check_tokens(max_batch, "mh_stack_create"));
    for (int i = 0; i < n_layers; i++) MH_TRY(validate_layer(&layers[i]));
    MH_TRY(require_init());
    mh_stack *st = new mh_stack();
    st->max_batch = max_batch;
    st->layers.resize((size_t)n_layers);
    for (int i = 0; i < n_layers; i++) {
        int rc = resolve_layer(&layers[i], &st->layers[(size_t)i]);
        if (rc) {
            delete st;
            return rc;
        }
        const DevLayer &a = st->layers[0], &b = st->layers[(size_t)i];
        if (b.hidden != a.hidden || b.top_k != a.top_k || b.n_experts != a.n_experts || b.ffn != a.ffn) {
            delete st;
            return fail(MH_E_ARG, "mh_stack_create: layer %d shape differs from layer 0", i);
        }
    }
    int rc = step_plan_create(st->layers.data(), n_layers, &st->plan);
    if (rc) {
        step_plan_destroy(st->plan);
        delete st;
        return rc;
    }
    *out = st;
    return MH_OK;
}

int mh_stack_decode(mh_stack *st, float *x, int batch, int32_t *sel, float *w, uint32_t *usage) {
    clear_error();
    if (!st) return fail(MH_E_ARG, "mh_stack_decode: NULL stack");
    if (batch < 1 || batch > st->max_batch)
        return fail(MH_E_ARG, "mh_stack_decode: batch %d outside [1, %d]", batch, st->max_batch);
    MH_TRY(require_init());
    const DevLayer &L0 = st->layers[0];
    const int nl = (int)st->layers.size(), k = L0.top_k;
    MH_TRY(resolve_dev(x, (uint64_t)batch * L0.hidden * 4, "mh_stack_decode x"));
    if (sel) MH_TRY(resolve_dev(sel, (uint64_t)nl * batch * k * 4, "mh_stack_decode sel"));
    if (w) MH_TRY(resolve_dev(w, (uint64_t)nl * batch * k * 4, "mh_stack_decode w"));
    if (usage) MH_TRY(resolve_dev(usage, (uint64_t)nl * L0.n_experts * 4, "mh_stack_decode usage"));
    hipStream_t s = stream();
    if (batch == 1 && !sw(SW_NO_FUSED) && step_plan_ok(st->plan)) {
        int rc = step_run(st->plan, st->layers.data(), 0, nl, x, sel, w, usage, s);
        if (rc != MH_E_UNSUPPORTED) return rc;
        clear_error();   // shape this device cannot run in one launch: per-layer launches below
    }
    LayerBufs b;
    MH_TRY(layer_bufs(L0, batch, &b));
    const bool few = step_plan_few(st->plan);
    bool fuse = b.order != nullptr && !sw(SW_SPLIT_ROUTE);
    for (int l = 0; l < nl && fuse; l++) fuse = combine_route_ok(st->layers[(size_t)l], batch);
    if (fuse) {
        // each layer boundary (the previous layer's combine, this layer's
        // norm, router and top-k) in one launch; the sel / w of a layer in
        // the caller's rows or, without them, in place in the scratch (a
        // token's weights are rewritten only after every block of the token
        // has read the previous layer's)
        auto lsel = [&](int l) { return sel ? sel + (size_t)l * batch * k : b.sel; };
        auto lw = [&](int l) { return w ? w + (size_t)l * batch * k : b.w; };
        auto luse = [&](int l) { return usage ? usage + (size_t)l * L0.n_experts : nullptr; };
        MH_TRY(launch_combine_route(L0, x, nullptr, nullptr, batch, b.xb, b.rl, lsel(0), lw(0), luse(0), b.order, s));
        for (int l = 0; l < nl; l++) {
            const DevLayer &L = st->layers[(size_t)l];
            if (few && !sw(SW_BATCH_GEMV) && grouped_ok(L, batch))
                MH_TRY(launch_grouped(L, batch, b.order, b.xb, b.h, b.ye, s));
            else
                MH_TRY(launch_experts(L, batch * k, lsel(l), b.order, b.xb, b.h, b.ye, s));
            if (l + 1 < nl) {
                MH_TRY(launch_combine_route(st->layers[(size_t)l + 1], x, b.ye, lw(l), batch, b.xb, b.rl, lsel(l + 1),
                                            lw(l + 1), luse(l + 1), b.order, s));
            } else {
                MH_LAUNCH("combine_decode", k_combine_decode, dim3((unsigned)((L.hidden + 255) / 256), (unsigned)batch),
                          dim3(256), 0, s, x, b.ye, lw(l), L.hidden, L.top_k);
                MH_TRY(hip_check(hipGetLastError(), "combine launch"));
            }
        }
        return MH_OK;
    }
    for (int l = 0; l < nl; l++) {
        LayerBufs bl = b;
        if (sel) bl.sel = sel + (size_t)l * batch * k;
        if (w) bl.w = w + (size_t)l * batch * k;
        // every layer after the first takes its normed input from the
        // previous layer's combine
        MH_TRY(run_decode_layer(st->layers[(size_t)l], x, batch, bl,
                                usage ? usage + (size_t)l * L0.n_experts : nullptr, s, few, l > 0,
                                l + 1 < nl ? &st->layers[(size_t)l + 1] : nullptr));
    }
    return MH_OK;
}

int mh_stack_apply_dev(mh_stack *st, int layer, const float *xb, const int32_t *sel, const float *w, float *x) {
    clear_error();
    if (!st) return fail(MH_E_ARG, "mh_stack_apply_dev: NULL stack");
    const int nl = (int)st->layers.size();
    if (layer < 0 || layer >= nl) return fail(MH_E_ARG, "mh_stack_apply_dev: layer %d outside [0, %d)", layer, nl);
    MH_TRY(require_init());
    const DevLayer &L = st->layers[(size_t)layer];
    MH_TRY(resolve_dev(xb, (uint64_t)L.hidden * 4, "mh_stack_apply_dev xb"));
    MH_TRY(resolve_dev(sel, (uint64_t)L.top_k * 4, "mh_stack_apply_dev sel"));
    MH_TRY(resolve_dev(w, (uint64_t)L.top_k * 4, "mh_stack_apply_dev w"));
    MH_TRY(resolve_dev(x, (uint64_t)L.hidden * 4, "mh_stack_apply_dev x"));
    hipStream_t s = stream();
    if (!sw(SW_NO_FUSED) && step_plan_ok(st->plan)) {
        int rc = step_run(st->plan, st->layers.data(), layer, 1, x, nullptr, nullptr, nullptr, s, xb, sel, w);
        if (rc != MH_E_UNSUPPORTED) return rc;
        clear_error();   // per-layer launches below
    }
    LayerBufs b;
    MH_TRY(layer_bufs(L, 1, &b));
    return run_expert_major(L, 1, xb, sel, w, x, b, s);
}

int mh_stack_destroy(mh_stack *st) {
    clear_error();
    if (st) {
        if (st->plan) (void)hipStreamSynchronize(stream());
        step_plan_destroy(st->plan);
    }
    delete st;
    return MH_OK;
}

}  // extern "C"
