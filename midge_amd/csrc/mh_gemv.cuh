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
    for (int f0 = 0; f0 < nf; f0 += ns * kGemvU) {
        // Branch-free loads: rows past nf and idle slots re-read a row the
        // block loads anyway (a cache hit) and are masked out below. Scales
        // stay raw f16 bits here: converting inside this loop would make
        // every iteration wait for its load.
        mh_u4 q[kGemvU];
        uint32_t sb[kGemvU];
        const int sl = active ? slot : ns - 1;
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            const int f = min(f0 + u * ns + sl, nf - 1);
            const RowRef rr = rowref(f);
            q[u] = mh_load16(mh_global(rr.data + (size_t)c * 16));
            if constexpr (DT == MH_DT_MXFP4 || DT == MH_DT_Q4G32) sb[u] = mh_load_u16(mh_global(rr.scale + c));
            else sb[u] = 0x3C00u;   // f16 1.0: int8 / f32 rows are scaled by the caller
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            const bool valid = active && f0 + u * ns + slot < nf;
            const float p = mh_dot_chunk<DT>(q[u], xr) * (valid ? mh_f16((uint16_t)sb[u]) : 0.f);
            if (active) red[(u * ns + slot) * C + c] = p;
        }
        __syncthreads();
        // row it = u * ns + slot is flat row f0 + it
        block_reduce_rows(red, C, kGemvU * ns, res + f0, [&](int it) { return f0 + it < nf; });
        __syncthreads();
    }
}

// Sums each row of red[nrows][C] (row-major) into out[row]. A wave takes 8
// rows at a time: 8 lanes per row each add every 8th partial, then three
// xor-shuffles combine them (a fixed order, so results are deterministic).
// Rows in `skip` (out[row] untouched) are those the caller marks invalid.
template <class Keep>
__device__ __forceinline__ void block_reduce_rows(const float *red, int C, int nrows, float *out, Keep keep) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int rl = lane >> 3, part = lane & 7;
    for (int r0 = wave * 8; r0 < nrows; r0 += nw * 8) {
        const int r = r0 + rl;
        float s = 0.f;
        if (r < nrows)
            for (int cc = part; cc < C; cc += 8) s += red[r * C + cc];
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        s += __shfl_xor(s, 4, 64);
        if (part == 0 && r < nrows && keep(r)) out[r] = s;
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
