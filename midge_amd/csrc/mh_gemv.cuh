// mh_gemv.cuh — the block-level GEMV engine shared by every matvec-shaped
// kernel in libmidge_hip (plain GEMV, expert gate/up, expert down).
//
// Layout of work inside a block ("lanes own column chunks"):
//   A row of `cols` elements is C = cols / E 16-byte chunks (E elements per
//   chunk: 32 for the 4-bit types, 16 for int8, 4 for f32). Thread t owns
//   chunk c = t % C of row slot s = t / C, with ns = floor(blockDim / C)
//   slots. Each thread keeps x[c*E .. c*E+E) in registers for the whole
//   block, so every weight byte is loaded exactly once, with 16-byte vector
//   loads that are contiguous across the C lanes of a slot (one row).
//   A step processes ns * U flat rows (U row-iterations in flight per thread);
//   per-thread partial dot products go to LDS and one wave per row sums them
//   in a fixed order (deterministic). The block's results land in `res`.
#pragma once
#include "mh_internal.h"

namespace mh {

constexpr int kGemvU = 4;          // row iterations in flight per thread
constexpr int kGemvThreads = 1024;

// Slots per block for C chunks per row and the thread count that covers them.
inline void gemv_shape(int C, int *ns, int *nt) {
    int s = kGemvThreads / C;
    if (s < 1) s = 1;
    int t = ((s * C + 63) / 64) * 64;
    *ns = s;
    *nt = t;
}

// LDS floats needed by block_gemv for ns slots of C chunks.
inline size_t gemv_lds_floats(int ns, int C) { return (size_t)kGemvU * ns * C; }

// Row source for block_gemv: flat row f -> (data pointer, scale pointer).
// `scale` is the f16 group scales for 4-bit types, unused otherwise.
struct RowRef {
    const uint8_t *data;
    const uint16_t *scale;
};

// Computes res[f] = sum over chunks of dot(row f, x) for f in [0, nf).
// For 4-bit types the f16 group scale is applied per chunk (exact: powers of
// two commute with rounding; non-power-of-two scales multiply the group's
// partial sum once, as the reference does). For int8 the per-row scale is the
// caller's. `xr` holds this thread's E elements of x; `red` is LDS of
// gemv_lds_floats(ns, C); `res` is LDS of at least nf floats.
// Must be called by every thread of the block.
template <int DT, class RowFn>
__device__ __forceinline__ void block_gemv(RowFn rowref, int nf, int C, int ns, const float *xr,
                                           float *red, float *res) {
    const int t = threadIdx.x;
    const int slot = t / C, c = t - slot * C;
    const bool active = slot < ns;
    const int nw = blockDim.x >> 6, wave = t >> 6, lane = t & 63;
    for (int f0 = 0; f0 < nf; f0 += ns * kGemvU) {
        mh_u4 q[kGemvU];
        float sc[kGemvU];
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            int f = f0 + u * ns + slot;
            q[u] = mh_u4{0u, 0u, 0u, 0u};
            sc[u] = 0.f;
            if (active && f < nf) {
                RowRef rr = rowref(f);
                q[u] = __builtin_nontemporal_load((const mh_u4 *)(rr.data + (size_t)c * 16));
                if constexpr (DT == MH_DT_MXFP4 || DT == MH_DT_Q4G32) sc[u] = mh_f16(rr.scale[c]);
                else sc[u] = 1.f;
            }
        }
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            float p = mh_dot_chunk<DT>(q[u], xr) * sc[u];
            if (active) red[(u * ns + slot) * C + c] = p;
        }
        __syncthreads();
        const int items = kGemvU * ns;
        for (int it = wave; it < items; it += nw) {
            int f = f0 + it;   // it = u * ns + slot, f = f0 + u * ns + slot
            if (f >= nf) continue;
            float s = 0.f;
            for (int cc = lane; cc < C; cc += 64) s += red[it * C + cc];
            s = mh_wave_sum(s);
            if (lane == 0) res[f] = s;
        }
        __syncthreads();
    }
}

// Load this thread's E elements of x (zeros for idle threads).
template <int DT>
__device__ __forceinline__ void load_x(const float *x, int C, int ns, float *xr) {
    constexpr int E = mh_chunk<DT>::E;
    const int t = threadIdx.x;
    const int slot = t / C, c = t - slot * C;
    if (slot < ns) {
        const float4 *p = (const float4 *)(x + (size_t)c * E);
#pragma unroll
        for (int i = 0; i < E / 4; ++i) {
            float4 v = p[i];
            xr[4 * i + 0] = v.x;
            xr[4 * i + 1] = v.y;
            xr[4 * i + 2] = v.z;
            xr[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < E; ++i) xr[i] = 0.f;
    }
}

}  // namespace mh
