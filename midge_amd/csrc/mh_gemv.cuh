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

constexpr int kGemvU = 4;          // 16-byte words in flight per thread per step
constexpr int kGemvThreads = 512;
constexpr int kGemvNB = 2;         // register sets: loads run NB - 1 steps ahead of the math

// A thread's share of a row: W 16-byte words (2 for int8, so that a chunk is
// 32 elements and a 2880-wide row is 90 chunks, as for the 4-bit types:
// 5 row slots per 512-thread block instead of 2), E elements; U row
// iterations in flight, so that U * W words are in flight per thread.
template <int DT>
struct gemv_chunk {
    static constexpr int W = DT == MH_DT_Q8R ? 2 : 1;
    static constexpr int E = mh_chunk<DT>::E * W;
    static constexpr int U = kGemvU / W;
};

// Slots per block for C chunks per row and the thread count that covers them.
inline void gemv_shape(int C, int *ns, int *nt) {
    int s = kGemvThreads / C;
    if (s < 1) s = 1;
    int t = ((s * C + 63) / 64) * 64;
    *ns = s;
    *nt = t;
}

// LDS floats needed by block_gemv for ns slots of C chunks (two buffers).
inline size_t gemv_lds_floats(int ns, int C) { return (size_t)2 * kGemvU * ns * C; }

// Buffer resources: the engine addresses rows by 32-bit byte offsets from a
// block-uniform base (buffer loads), so a row's address costs a 24-bit
// multiply-add, not 64-bit pointer arithmetic. Reads past `bytes` return 0.
typedef __amdgpu_buffer_rsrc_t mh_rsrc;
constexpr int kGemvNT = 2;   // cache-policy bits of weight loads: nontemporal
__device__ __forceinline__ mh_rsrc gemv_rsrc(const void *p, uint32_t bytes) {
    const uint64_t v = (uint64_t)p;   // made scalar: the resource is uniform
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    void *u = (void *)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// a * b for a, b < 2^24 (full-rate v_mul_u32_u24), low 32 bits of the product
__device__ __forceinline__ uint32_t mul24(uint32_t a, uint32_t b) { return (uint32_t)__umul24(a, b); }

// Row source for block_gemv: flat row f -> byte offsets of its data (in the
// data resource) and of its f16 group scales (in the scale resource; 4-bit
// types only).
struct RowOff {
    uint32_t data, scale;
};

// Sums each row of red[nrows][C] (row-major) into out[row]. A wave takes 8
// rows at a time: 8 lanes per row each add every 8th partial in column order,
// then lane 0 of the 8 adds the others' sums as ((p0 + p1) + (p2 + p3)) +
// ((p4 + p5) + (p6 + p7)): a fixed order, so results are deterministic. A
// lane's partials are read in batches of 12 issued together (a read-add
// loop would wait for each read in turn), then added in the same order.
// Rows in `skip` (out[row] untouched) are those the caller marks invalid.
// nw is the block's wave count, passed in: reading blockDim inside a
// pipelined loop is a memory load whose wait also waits for every weight
// load in flight.
template <class Keep>
__device__ __forceinline__ void block_reduce_rows(const float *red, int C, int nrows, int nw, float *out,
                                                  Keep keep) {
    constexpr int kB = 12;   // partials read per batch
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rl = lane >> 3, part = lane & 7;
    for (int r0 = wave * 8; r0 < nrows; r0 += nw * 8) {
        const int r = r0 + rl;
        float s = 0.f;
        if (r < nrows) {
            const float *rr = red + r * C;
            int cc = part;
            for (; cc + 8 * (kB - 1) < C; cc += 8 * kB) {
                float v[kB];
#pragma unroll
                for (int i = 0; i < kB; ++i) v[i] = rr[cc + 8 * i];
#pragma unroll
                for (int i = 0; i < kB; ++i) s += v[i];
            }
            float v[kB];
#pragma unroll
            for (int i = 0; i < kB; ++i) v[i] = cc + 8 * i < C ? rr[cc + 8 * i] : 0.f;
#pragma unroll
            for (int i = 0; i < kB; ++i)
                if (cc + 8 * i < C) s += v[i];
        }
        s += dpp_x1(s);
        s += dpp_x2(s);
        s += dpp_shl<4>(s);
        if (part == 0 && r < nrows && keep(r)) out[r] = s;
    }
}

// One step's loads: U row iterations of this thread's chunk (branch-free:
// rows past nf and idle slots re-read the block's last row, a cache hit,
// and are masked out in the math). Scale bits stay raw f16 here: converting
// inside the load loop would make every iteration wait for its load.
// Weight loads are non-temporal, except for int8 rows (two words a chunk):
// there one instruction covers every other 16 bytes of its lines, and a
// non-temporal line fetched for the first word was fetched again for the
// second (int8 lm_head 201088 x 2880 at batch 1: 125 -> 112 us cached).
template <int DT, int U, class RowFn>
__device__ __forceinline__ void gemv_load(mh_rsrc rd, mh_rsrc rs, RowFn rowoff, int f0, int nf, int c, int sl,
                                          int ns, mh_u4 *q, uint32_t *sb) {
    constexpr int W = gemv_chunk<DT>::W;
    const uint32_t cw = (uint32_t)c * (16u * W), cs = (uint32_t)c * 2u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const RowOff o = rowoff(min(f0 + u * ns + sl, nf - 1));
#pragma unroll
        for (int w = 0; w < W; ++w)
            q[u * W + w] = __builtin_amdgcn_raw_buffer_load_b128(rd, o.data + cw + 16u * w, 0, W == 2 ? 0 : kGemvNT);
        if constexpr (DT == MH_DT_MXFP4 || DT == MH_DT_Q4G32)
            sb[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, o.scale + cs, 0, kGemvNT);
        else
            sb[u] = 0x3C00u;   // f16 1.0: int8 / f32 rows are scaled by the caller
    }
}

// One step's math: partial dot products of this thread's chunk into red.
template <int DT, int U>
__device__ __forceinline__ void gemv_math(const mh_u4 *q, const uint32_t *sb, const float *xr, int f0, int nf,
                                          int slot, int c, int C, int ns, bool active, float *red) {
    constexpr int W = gemv_chunk<DT>::W, WE = mh_chunk<DT>::E;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool valid = active && f0 + u * ns + slot < nf;
        float d = mh_dot_chunk<DT>(q[u * W], xr);
#pragma unroll
        for (int w = 1; w < W; ++w) d += mh_dot_chunk<DT>(q[u * W + w], xr + w * WE);
        const float p = d * (valid ? mh_f16((uint16_t)sb[u]) : 0.f);
        if (active) red[(u * ns + slot) * C + c] = p;
    }
}

// Computes res[f] = sum over chunks of dot(row f, x) for f in [0, nf), rows
// addressed through rowoff(f) in the resources rd (data) and rs (scales).
// For 4-bit types the f16 group scale is applied per chunk (exact: powers of
// two commute with rounding; non-power-of-two scales multiply the group's
// partial sum once, as the reference does). For int8 the per-row scale is the
// caller's. `xr` holds this thread's E elements of x; `red` is LDS of
// gemv_lds_floats(ns, C) (two buffers); `res` is LDS of at least nf floats.
// Software-pipelined NB deep: while step i (U rows per slot) is computed,
// synchronised and reduced, the loads of steps i + 1 .. i + NB - 1 are in
// flight. Must be called by every thread.
template <int DT, int U = gemv_chunk<DT>::U, int NB = kGemvNB, class RowFn>
__device__ __forceinline__ void block_gemv(mh_rsrc rd, mh_rsrc rs, RowFn rowoff, int nf, int C, int ns,
                                           const float *xr, float *red, float *res) {
    constexpr int WW = gemv_chunk<DT>::W;
    const int t = threadIdx.x;
    const int slot = t / C, c = t - slot * C;
    const bool active = slot < ns;
    const int sl = active ? slot : ns - 1;
    const int step = ns * U;
    const int per = U * ns * C;   // floats of one red buffer
    const int nw = (ns * C + 63) >> 6;   // the launch's waves (gemv_shape)
    mh_u4 q[NB][U * WW];
    uint32_t sc[NB][U];
    if (nf <= 0) return;
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) gemv_load<DT, U>(rd, rs, rowoff, j * step, nf, c, sl, ns, q[j], sc[j]);
    // step j of a group of NB: loads of step fj + NB - 1 (rows clamped, so
    // steps past the end re-read the last row), then the math of step fj
    auto stepj = [&](int j, int fj) {
        gemv_load<DT, U>(rd, rs, rowoff, fj + (NB - 1) * step, nf, c, sl, ns, q[(j + NB - 1) % NB],
                         sc[(j + NB - 1) % NB]);
        __builtin_amdgcn_sched_barrier(0);
        float *rb = red + ((fj / step) & 1) * per;
        gemv_math<DT, U>(q[j], sc[j], xr, fj, nf, slot, c, C, ns, active, rb);
        __syncthreads();
        block_reduce_rows(rb, C, step, nw, res + fj, [&](int it) { return fj + it < nf; });
    };
    // whole groups without exits (an exit inside the unrolled group makes the
    // compiler wait for every load in flight at the loop edge), then the rest
    int f0 = 0;
    for (; f0 + (NB - 1) * step < nf; f0 += NB * step) {
#pragma unroll
        for (int j = 0; j < NB; ++j) stepj(j, f0 + j * step);
    }
#pragma unroll
    for (int j = 0; j < NB - 1; ++j)
        if (f0 + j * step < nf) stepj(j, f0 + j * step);
    __syncthreads();
}

// Load this thread's E elements of x (zeros for idle threads).
template <int DT>
__device__ __forceinline__ void load_x(const float *x, int C, int ns, float *xr) {
    constexpr int E = gemv_chunk<DT>::E;
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
