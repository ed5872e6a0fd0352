// mh_attn.hip — the trunk's attention for one decode token, attention()
// (engine/midge.c:341-400), on the device: the next component of the
// decode step beside the MoE layers.
//
//   rmsnorm, q, k, v one launch on the GEMV engine (k_gemv3), any weight
//                    dtype: every block forms xb = rmsnorm(x) * w for its
//                    own chunks of x; k_rmsnorm and three launch_gemv calls
//                    where the shapes differ
//   k_attn_split     per query head and split of the cached positions:
//                    biases, per-head RMSNorm (the reference's sequential
//                    sum), RoPE from the given tables, the current k and v
//                    rounded to f16 as wk_to_f16 does (and written to the
//                    cache slot pos % cap by one block of the kv head); the
//                    scores over the cached positions, softmax with the
//                    optional sink logit in the denominator, the weighted
//                    sum of the cached v (splits combined by the last one
//                    to finish when a head has more than one)
//   o                the GEMV engine with the residual in its epilogue
//                    (k_gemv_res: + bias, x += o); GEMV + k_attn_residual
//                    where the shape needs the general kernel
#include "mh_gemv.cuh"
#include "mh_xchg.cuh"

namespace mh {
namespace {

constexpr int kAttnThreads = 256;

// The attention RMSNorm and q, k and v in one launch: the three matrices
// (same dtype and width) as consecutive block ranges of one grid, each block
// a k_gemv block over rows of one of them (block-uniform choice), into
// y[m] = W[m] xb with xb = x * inv * w, inv = 1 / sqrt(mean(x^2) + eps)
// (engine/mkern.h:238-243). Every block sums x^2 over the distinct chunks in
// the same fixed order, so all reach the same inv.
struct Gemv3Args {
    const uint8_t *W[3];
    const void *S[3];
    float *Y[3];
    int rows[3], nb[3];
    const float *x, *nw;
    float eps;
    int cols, ns, rpb;
};

template <int DT>
__global__ void __launch_bounds__(kGemvThreads) k_gemv3(Gemv3Args A) {
    constexpr int E = gemv_chunk<DT>::E;
    extern __shared__ float lds[];
    int b = blockIdx.x, m = 0;
    if (b >= A.nb[0]) {
        b -= A.nb[0];
        m = 1;
        if (b >= A.nb[1]) {
            b -= A.nb[1];
            m = 2;
        }
    }
    const uint8_t *W = m == 0 ? A.W[0] : m == 1 ? A.W[1] : A.W[2];
    const void *S = m == 0 ? A.S[0] : m == 1 ? A.S[1] : A.S[2];
    float *Y = m == 0 ? A.Y[0] : m == 1 ? A.Y[1] : A.Y[2];
    const int rows = m == 0 ? A.rows[0] : m == 1 ? A.rows[1] : A.rows[2];
    const int C = A.cols / E;
    float *res = lds, *red = lds + A.rpb;
    const int r0 = b * A.rpb, nf = min(A.rpb, rows - r0);
    const uint32_t rowbytes = (uint32_t)C * 16u * gemv_chunk<DT>::W;
    float xr[E];
    load_x<DT>(A.x, C, A.ns, xr);
    {
        __shared__ float part[kGemvThreads / 64];
        const int t = threadIdx.x, slot = t / C, c = t - slot * C;
        float ss = 0.f;
        if (slot == 0)   // each chunk once
#pragma unroll
            for (int j = 0; j < E; ++j) ss = __builtin_fmaf(xr[j], xr[j], ss);
        ss = mh_wave_sum(ss);
        if ((t & 63) == 0) part[t >> 6] = ss;
        __syncthreads();
        ss = 0.f;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) ss += part[w];
        const float inv = 1.0f / sqrtf(ss / (float)A.cols + A.eps);
        if (slot < A.ns) {
            const float4 *wp = (const float4 *)(A.nw + (size_t)c * E);
#pragma unroll
            for (int i = 0; i < E / 4; ++i) {
                const float4 w4 = wp[i];
                xr[4 * i + 0] = xr[4 * i + 0] * inv * w4.x;
                xr[4 * i + 1] = xr[4 * i + 1] * inv * w4.y;
                xr[4 * i + 2] = xr[4 * i + 2] * inv * w4.z;
                xr[4 * i + 3] = xr[4 * i + 3] * inv * w4.w;
            }
        }
    }
    const mh_rsrc rd = gemv_rsrc(W + (size_t)r0 * rowbytes, (uint32_t)nf * rowbytes);
    const mh_rsrc rs = gemv_rsrc((const uint16_t *)S + (size_t)r0 * C, (uint32_t)nf * (uint32_t)C * 2u);
    block_gemv<DT>(
        rd, rs, [&](int f) { return RowOff{mul24((uint32_t)f, rowbytes), mul24((uint32_t)f, 2u * C)}; }, nf, C,
        A.ns, xr, red, res);
    for (int f = threadIdx.x; f < nf; f += blockDim.x) {
        float v = res[f];
        if constexpr (DT == MH_DT_Q8R) v *= ((const float *)S)[r0 + f];
        Y[r0 + f] = v;
    }
}

// The o projection with the residual in its epilogue:
// x[r] = x[r] + ((Wo ao)[r] + bo[r]) (two roundings, as wk_addbias then
// the residual loop of attention()).
template <int DT>
__global__ void __launch_bounds__(kGemvThreads)
k_gemv_res(const uint8_t *__restrict__ W, const void *__restrict__ S, const float *__restrict__ ao,
           const float *__restrict__ bo, float *__restrict__ x, int rows, int cols, int ns, int rpb) {
#pragma clang fp contract(off)
    constexpr int E = gemv_chunk<DT>::E;
    extern __shared__ float lds[];
    const int C = cols / E;
    float *res = lds, *red = lds + rpb;
    const int r0 = blockIdx.x * rpb, nf = min(rpb, rows - r0);
    const uint32_t rowbytes = (uint32_t)C * 16u * gemv_chunk<DT>::W;
    float xr[E];
    load_x<DT>(ao, C, ns, xr);
    const mh_rsrc rd = gemv_rsrc(W + (size_t)r0 * rowbytes, (uint32_t)nf * rowbytes);
    const mh_rsrc rs = gemv_rsrc((const uint16_t *)S + (size_t)r0 * C, (uint32_t)nf * (uint32_t)C * 2u);
    block_gemv<DT>(
        rd, rs, [&](int f) { return RowOff{mul24((uint32_t)f, rowbytes), mul24((uint32_t)f, 2u * C)}; }, nf, C,
        ns, xr, red, res);
    for (int f = threadIdx.x; f < nf; f += blockDim.x) {
        float v = res[f];
        if constexpr (DT == MH_DT_Q8R) v *= ((const float *)S)[r0 + f];
        const float y = v + bo[r0 + f];
        x[r0 + f] = x[r0 + f] + y;
    }
}

template <int DT>
int launch_o_res_t(const DevWT &w, const float *ao, const float *bo, float *x, hipStream_t s, bool *done) {
    constexpr int E = gemv_chunk<DT>::E;
    *done = false;
    if (w.cols % E != 0 || w.cols / E > kGemvThreads || ((uintptr_t)w.data % 16) != 0 || ((uintptr_t)ao % 16) != 0 ||
        w.rows > INT32_MAX)
        return MH_OK;
    const int C = (int)(w.cols / E);
    int ns, nt;
    gemv_shape(C, &ns, &nt);
    const int64_t target = (int64_t)device_cus() * 2;
    int64_t rpb = (w.rows + target - 1) / target;
    rpb = ((rpb + ns - 1) / ns) * ns;
    if (rpb < ns) rpb = ns;
    if (rpb > 4096) rpb = 4096;
    const int64_t nblk = (w.rows + rpb - 1) / rpb;
    const size_t lds = ((size_t)rpb + gemv_lds_floats(ns, C)) * sizeof(float);
    MH_LAUNCH("gemv_o_res", k_gemv_res<DT>, dim3((unsigned)nblk), dim3(nt), lds, s, w.data, w.scales, ao, bo, x,
              (int)w.rows, (int)w.cols, ns, (int)rpb);
    *done = true;
    return hip_check(hipGetLastError(), "o projection launch");
}

// One launch for the RMSNorm and q, k, v when their dtype and layout allow
// the GEMV engine's chunked kernel; *done = false leaves them to k_rmsnorm
// and three launch_gemv.
template <int DT>
int launch_qkv_t(const DevWT *w, const float *x, const float *nw, float eps, float *const *y, hipStream_t s,
                 bool *done) {
    constexpr int E = gemv_chunk<DT>::E;
    const int64_t cols = w[0].cols;
    *done = false;
    for (int m = 0; m < 3; ++m)
        if (w[m].dt != DT || w[m].cols != cols || ((uintptr_t)w[m].data % 16) != 0 || w[m].rows > INT32_MAX)
            return MH_OK;
    if (cols % E != 0 || cols / E > kGemvThreads || ((uintptr_t)x % 16) != 0 || ((uintptr_t)nw % 16) != 0)
        return MH_OK;
    const int C = (int)(cols / E);
    int ns, nt;
    gemv_shape(C, &ns, &nt);
    const int64_t total = w[0].rows + w[1].rows + w[2].rows, target = (int64_t)device_cus() * 2;
    int64_t rpb = (total + target - 1) / target;
    rpb = ((rpb + ns - 1) / ns) * ns;
    if (rpb < ns) rpb = ns;
    if (rpb > 4096) rpb = 4096;
    Gemv3Args A;
    int nblk = 0;
    for (int m = 0; m < 3; ++m) {
        A.W[m] = w[m].data;
        A.S[m] = w[m].scales;
        A.Y[m] = y[m];
        A.rows[m] = (int)w[m].rows;
        A.nb[m] = (int)((w[m].rows + rpb - 1) / rpb);
        nblk += A.nb[m];
    }
    A.x = x;
    A.nw = nw;
    A.eps = eps;
    A.cols = (int)cols;
    A.ns = ns;
    A.rpb = (int)rpb;
    const size_t lds = ((size_t)rpb + gemv_lds_floats(ns, C)) * sizeof(float);
    MH_LAUNCH("gemv_qkv", k_gemv3<DT>, dim3((unsigned)nblk), dim3(nt), lds, s, A);
    *done = true;
    return hip_check(hipGetLastError(), "q/k/v launch");
}

// The cache's f16 as wk_to_f16 (engine/mkern.h:261-273) makes it: the
// hardware's round-to-nearest-even conversion (which already overflows to
// inf from 65520 up), except that magnitudes below the f16 normal range
// become a signed zero and NaN becomes a signed inf.
__device__ __forceinline__ uint16_t to_f16_ref(float f) {
    const float a = fabsf(f);
    const uint16_t sign = (uint16_t)((__float_as_uint(f) >> 16) & 0x8000u);
    if (!(a >= 0x1p-14f)) return a != a ? (uint16_t)(sign | 0x7c00u) : sign;
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float block_max_f(float v, float *part) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = part[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, part[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_sum_f(float v, float *part) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += part[i];
    __syncthreads();
    return r;
}

// The decode attention of one token in one launch: prep and heads split
// over the cached positions. Block (h, s) takes query head h and positions
// [P s, P s + P) of the nctx cached ones (P = 256 on 256 threads up to 256
// positions, else 2048 on 1024 threads: contexts up to 2048 need no
// combine):
//   prep     q of head h and the current token's k, v of its kv head
//            (biases, per-head RMSNorm with the reference's sequential sum
//            of squares, RoPE, k and v rounded to f16 as wk_to_f16 does),
//            every global value loaded in one round; every block of a kv
//            head computes the same k, v and uses them for the current
//            slot, and block (first head of the group, split 0) writes them
//            to the cache slot, so no block waits for another
//   scores   the reference's sequential f16 dot per position (16-byte
//            loads, all of a thread's positions in flight), times scale
//   partial  m = the split's maximum score, l = sum of e = expf(score - m),
//            o = sum of e * v (head_dim 64: threads of 8 dims x a position
//            group with 16-byte loads, the groups added in order; else
//            waves over positions, lanes over dims)
//   combine  in the block when the head has one split; else the last split
//            of head h to finish (a per-head counter it resets) reads the
//            others' partials: M = max(m over splits, sink), den = sum of l *
//            expf(m - M) (+ expf(sink - M)), ao = sum of o * expf(m - M) /
//            den. The factors round differently from the reference's single
//            pass over expf(score - max); the result stays within its own
//            AVX2-vs-scalar divergence.
constexpr int kSplitT = 1024;     // threads per block
constexpr int kSplitP = 2;        // positions per thread: 2048 positions per split
constexpr int kMaxSplits = 1024;  // splits per head (cached positions <= 2^21)

struct SplitArgs {
    const float *q, *k, *v;
    const float *bq, *bk, *bv, *qn, *kn, *co, *si, *sink;
    uint16_t *kc, *vc;
    float *part;      // [nh][S][hd + 2]: o, m, l
    unsigned *cnt;    // [nh] arrivals (zero between calls)
    float *ao;        // [nh][hd]
    int nh, hd, gq, kvd, nctx, slot, S, sinks, qk_norm, kvec;
    float scale, eps;
};

__device__ __forceinline__ float f16_at(const uint16_t *p) { return mh_f16(*p); }

template <int T, int PPT>
__global__ void __launch_bounds__(T) k_attn_split(SplitArgs A) {
#pragma clang fp contract(off)
    constexpr int P = T * PPT;   // positions per split
    __shared__ float uq[256], uk[256];
    __shared__ __attribute__((aligned(16))) uint16_t kcur[256], vcur[256];
    __shared__ float s_inv[2];
    __shared__ float sc[P];
    __shared__ float red[T / 64];
    // o partials: per wave [T / 64][256], or per position group [T / 8][64]
    __shared__ float ob[T / 8 * 64 > T / 64 * 256 ? T / 8 * 64 : T / 64 * 256];
    __shared__ int s_last;
    __shared__ float s_m[kMaxSplits], s_l[kMaxSplits];
    const int h = blockIdx.x / A.S, s = blockIdx.x - h * A.S;
    const int kh = h / A.gq, hd = A.hd, half = hd / 2, i = threadIdx.x, lane = i & 63, wv = i >> 6;
    // ---------------------------------------------------------- prep
    // every global value the prep needs, loaded in one round
    float xq = 0.f, xk = 0.f, xv = 0.f, cs = 0.f, sn = 0.f, wq = 0.f, wk = 0.f;
    if (i < hd) {
        xq = A.q[(size_t)h * hd + i] + A.bq[(size_t)h * hd + i];
        xk = A.k[(size_t)kh * hd + i] + A.bk[(size_t)kh * hd + i];
        xv = A.v[(size_t)kh * hd + i] + A.bv[(size_t)kh * hd + i];
        if (A.qk_norm) {
            wq = A.qn[i];
            wk = A.kn[i];
        }
    }
    if (i < half) {
        cs = A.co[i];
        sn = A.si[i];
    }
    if (i < hd) {
        uq[i] = xq;
        uk[i] = xk;
    }
    __syncthreads();
    if (A.qk_norm) {
        if (i == 0 || i == 64) {   // the reference's sequential sums of squares
            const float *u = i == 0 ? uq : uk;
            float ss = 0.f;
            for (int j = 0; j < hd; ++j) ss += u[j] * u[j];
            s_inv[i == 0 ? 0 : 1] = 1.0f / sqrtf(ss / (float)hd + A.eps);
        }
        __syncthreads();
        const float vq = i < hd ? uq[i] * s_inv[0] * wq : 0.f;
        const float vk = i < hd ? uk[i] * s_inv[1] * wk : 0.f;
        __syncthreads();
        if (i < hd) {
            uq[i] = vq;
            uk[i] = vk;
        }
        __syncthreads();
    }
    float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f;
    if (i < half) {
        const float a = uq[i], c = uq[i + half], b = uk[i], d = uk[i + half];
        q0 = a * cs - c * sn;
        q1 = c * cs + a * sn;
        k0 = b * cs - d * sn;
        k1 = d * cs + b * sn;
    }
    __syncthreads();
    if (i < half) {
        uq[i] = q0;
        uq[i + half] = q1;
        uk[i] = k0;
        uk[i + half] = k1;
    }
    __syncthreads();
    if (i < hd) {
        kcur[i] = to_f16_ref(uk[i]);
        vcur[i] = to_f16_ref(xv);
        if (h % A.gq == 0 && s == 0) {
            const size_t o = (size_t)A.slot * A.kvd + (size_t)kh * hd + i;
            A.kc[o] = kcur[i];
            A.vc[o] = vcur[i];
        }
    }
    __syncthreads();
    // ---------------------------------------------------------- scores
    // positions t0 + i + T r, r < PPT (one 16-byte load per 8 cached values,
    // every load of the thread's positions issued before the sums, which
    // keep the reference's order within a position)
    const int t0 = P * s;
    float dd[PPT];
    if (A.kvec && hd == 64) {
        uint4 kw[PPT][8];
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int t = t0 + i + T * r;
            const bool cur = t == A.slot || t >= A.nctx;
            const uint16_t *kt = cur ? kcur : A.kc + (size_t)t * A.kvd + (size_t)kh * hd;
#pragma unroll
            for (int c = 0; c < 8; ++c) kw[r][c] = *(const uint4 *)(kt + 8 * c);
        }
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            float d = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t ww[4] = {kw[r][c].x, kw[r][c].y, kw[r][c].z, kw[r][c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    d += uq[8 * c + 2 * j] * mh_f16((uint16_t)(ww[j] & 0xffffu));
                    d += uq[8 * c + 2 * j + 1] * mh_f16((uint16_t)(ww[j] >> 16));
                }
            }
            dd[r] = d;
        }
    } else {
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const int t = t0 + i + T * r;
            float d = 0.f;
            if (t < A.nctx) {
                const uint16_t *kt = t == A.slot ? kcur : A.kc + (size_t)t * A.kvd + (size_t)kh * hd;
                for (int j = 0; j < hd; ++j) d += uq[j] * f16_at(kt + j);
            }
            dd[r] = d;
        }
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < PPT; ++r) {
        dd[r] = t0 + i + T * r < A.nctx ? dd[r] * A.scale : -INFINITY;
        mloc = fmaxf(mloc, dd[r]);
    }
    const float m = block_max_f(mloc, red);
    float el = 0.f;
#pragma unroll
    for (int r = 0; r < PPT; ++r) {
        const float e = t0 + i + T * r < A.nctx ? expf(dd[r] - m) : 0.f;
        sc[i + T * r] = e;
        el += e;
    }
    const float l = block_sum_f(el, red);   // (its barriers also order the sc writes)
    const int np = min(P, A.nctx - t0);
    if (A.kvec && hd == 64) {
        // 16-byte loads: thread (position group pg, dims 8 dc .. 8 dc + 7)
        // takes positions pg, pg + NG, ... (all its loads in flight), then
        // the groups' sums are added in order
        constexpr int NG = T / 8, NPT = P / NG;
        const int pg = i >> 3, dc = i & 7;
        float o8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        uint4 w8[NPT];
#pragma unroll
        for (int u = 0; u < NPT; ++u) {
            const int j = pg + NG * u, tt = t0 + j;
            w8[u] = (j < np && tt != A.slot) ? *(const uint4 *)(A.vc + (size_t)tt * A.kvd + (size_t)kh * hd + 8 * dc)
                                             : *(const uint4 *)(vcur + 8 * dc);
        }
#pragma unroll
        for (int u = 0; u < NPT; ++u) {
            const int j = pg + NG * u;
            if (j < np) {
                const float e = sc[j];
                const uint32_t ww[4] = {w8[u].x, w8[u].y, w8[u].z, w8[u].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    o8[2 * q] += e * mh_f16((uint16_t)(ww[q] & 0xffffu));
                    o8[2 * q + 1] += e * mh_f16((uint16_t)(ww[q] >> 16));
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) ob[pg * 64 + 8 * dc + q] = o8[q];
        __syncthreads();
        float o = 0.f;
        if (i < 64)
            for (int g2 = 0; g2 < NG; ++g2) o += ob[g2 * 64 + i];
        __syncthreads();
        // as the per-wave layout below: wave 0's row holds the sums, the
        // other rows zero
        for (int q = i; q < T / 64 * 256; q += T) ob[q] = 0.f;
        __syncthreads();
        if (i < 64) ob[i] = o;
    } else {
        // waves over positions (stride T / 64), lanes over dims; eight
        // positions' loads issued before their products, which are still
        // added in position order
        constexpr int NW = T / 64, U = 8;
        for (int i0 = 0; i0 < hd; i0 += 64) {
            const int dm = i0 + lane;
            float o = 0.f;
            if (dm < hd) {
                const uint16_t *vb = A.vc + (size_t)kh * hd + dm;
                const float vslot = mh_f16(vcur[dm]);
                int j = wv;
                for (; j + NW * (U - 1) < np; j += NW * U) {
                    float vv[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int tt = t0 + j + NW * u;
                        vv[u] = tt == A.slot ? vslot : mh_f16(vb[(size_t)tt * A.kvd]);
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u) o += sc[j + NW * u] * vv[u];
                }
                for (; j < np; j += NW) {
                    const int tt = t0 + j;
                    o += sc[j] * (tt == A.slot ? vslot : mh_f16(vb[(size_t)tt * A.kvd]));
                }
            }
            if (dm < 256) ob[wv * 256 + dm] = dm < hd ? o : 0.f;
        }
    }
    __syncthreads();
    if (A.S == 1) {   // one split: the combine's arithmetic without the memory round trip
        float M = m;
        const float sinkv = A.sinks ? A.sink[h] : -1e30f;
        if (sinkv > M) M = sinkv;
        const float f = expf(m - M);
        float den = l * f;
        if (A.sinks) den += expf(sinkv - M);
        const float inv = 1.0f / den;
        for (int dm = i; dm < hd; dm += T) {
            float o = 0.f;
#pragma unroll
            for (int w = 0; w < T / 64; ++w) o += ob[w * 256 + dm];
            A.ao[(size_t)h * hd + dm] = o * f * inv;
        }
        return;
    }
    float *pp = A.part + ((size_t)h * A.S + s) * (hd + 2);
    for (int dm = i; dm < hd; dm += T) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < T / 64; ++w) o += ob[w * 256 + dm];
        __hip_atomic_store(pp + dm, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (i == 0) {
        __hip_atomic_store(pp + hd, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + hd + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // ---------------------------------------------------------- combine
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (i == 0) {
        // one thread's acquire serves the block: its invalidation covers the
        // CU's cache and the L2 every wave reads through, and the barrier
        // orders the other waves' loads after it
        const bool last =
            __hip_atomic_fetch_add(&A.cnt[h], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)A.S - 1u;
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(&A.cnt[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // after the acquire, plain loads in one round: every split's m and l
    // into LDS, then each thread's o values
    const float *ph = A.part + (size_t)h * A.S * (hd + 2);
    for (int q = i; q < A.S; q += T) {
        s_m[q] = ph[(size_t)q * (hd + 2) + hd];
        s_l[q] = ph[(size_t)q * (hd + 2) + hd + 1];
    }
    __syncthreads();
    float M = -1e30f;
    for (int q = 0; q < A.S; ++q) M = fmaxf(M, s_m[q]);
    const float sinkv = A.sinks ? A.sink[h] : -1e30f;
    if (sinkv > M) M = sinkv;
    float den = 0.f;
    for (int q = 0; q < A.S; ++q) den += s_l[q] * expf(s_m[q] - M);
    if (A.sinks) den += expf(sinkv - M);
    const float inv = 1.0f / den;
    for (int dm = i; dm < hd; dm += T) {
        float o = 0.f;
        for (int q = 0; q < A.S; ++q) o += ph[(size_t)q * (hd + 2) + dm] * expf(s_m[q] - M);
        A.ao[(size_t)h * hd + dm] = o * inv;
    }
}

// ------------------------------------------------ attention in one launch
//
// The whole of attention() for one token in one persistent grid of NB blocks
// (one per CU at most, all resident: every wait is a bounded poll on a
// tagged word, and a timeout raises the error flag instead of hanging), for
// int8 (q8r) projections:
//   1  every block owning q/k/v rows reads x, forms xb = rmsnorm(x) * w in
//      LDS (the same fixed-order sum of squares in every block), computes
//      its RQ rows of [q; k; v] = W xb (* row scale, + bias) and publishes
//      them as tagged words;
//   2  block (head h, split s) for h < nh, s < S gathers q of head h and k,
//      v of its kv head and runs k_attn_split's per-head arithmetic over its
//      positions (per-head RMSNorm with the reference's sequential sums,
//      RoPE, k and v rounded to f16 as wk_to_f16 does and written to the
//      cache slot by one block of the kv head, the f16 dots in position
//      order, the softmax partials); with S > 1 block (h, 0) combines the
//      splits' partials; the head's output is published in kAR copies;
//   3  every block gathers the attention output and computes its RO rows of
//      o = Wo ao (* scale, + bias) and x[r] = x[r] + o[r] (two roundings, as
//      wk_addbias then the residual loop).
// x is read in phase 1 and written in phase 3: a block writes only after it
// has gathered every head's output, which needs every block's q/k/v rows,
// each published after that block read x. Every block owns q/k/v rows
// (NB = ceil(QR / RQ)).
constexpr int kA1Threads = 512;
constexpr int kA1HMax = 3072;     // hidden size
constexpr int kA1QMax = 4096;     // n_heads * head_dim
constexpr int kA1UQ = 4;          // row iterations per thread of phase 1 (q, k, v)
constexpr int kA1UO = 4;          // row iterations per thread of phase 3 (o)
constexpr int kA1PPT = 2;         // positions per thread and split: 1024 per split
constexpr int kA1P = kA1Threads * kA1PPT;
constexpr int kA1MaxS = 8;        // splits per head
constexpr int kAR = 8;            // copies of the attention output (each polled by NB / kAR blocks)

struct Attn1Args {
    const int8_t *w[4];        // q, k, v, o rows
    const float *ws[4];        // their row scales
    const float *b[4];         // biases
    const float *an, *qn, *kn, *co, *si, *sink;
    uint16_t *kc, *vc;
    float *x;                  // [H], updated in place
    uint64_t *qkv;             // [QR] tagged rows of q, k, v (with biases)
    uint64_t *part;            // [nh][S][hd + 2] tagged split partials: o, m, l
    uint64_t *ao;              // [kAR][aos] tagged attention output
    unsigned *err;
    int H, nh, hd, gq, qd, kvd, QR, nctx, slot, S, sinks, qk_norm, kvec, RQ, RO, aos;
    float eps, scale;
    unsigned tag;
};

// Rows [0, nr) of a block's share of int8 rows of C 32-element chunks (row
// j at rowp(j)) times v (LDS, 32-float groups padded to 33): thread (slot,
// chunk c) takes rows slot + ns u, u < U. a1_issue loads them (2 x 16 bytes
// a row and thread) so that they can be in flight long before a1_math uses
// them; a1_math forms the chunk partials and the per-row sums in a fixed
// order into out[0 .. nr). red: LDS of U * kA1Threads floats.
template <int U, class RowP>
__device__ __forceinline__ void a1_issue(RowP rowp, int nr, int C, mh_u4 (&q)[U][2]) {
    const int t = threadIdx.x, ns = kA1Threads / C;
    const int slot = t / C, c = t - slot * C;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = slot + ns * u;
        if (slot < ns && j < nr) {
            const int8_t *p = rowp(j) + (size_t)c * 32;
            q[u][0] = *(const mh_u4 *)p;
            q[u][1] = *(const mh_u4 *)(p + 16);
        } else {
            q[u][0] = q[u][1] = mh_u4{0u, 0u, 0u, 0u};
        }
    }
}

template <int U>
__device__ __forceinline__ void a1_math(const mh_u4 (&q)[U][2], int nr, int C, const float *v, float *red,
                                        float *out) {
    const int t = threadIdx.x, ns = kA1Threads / C;
    const int slot = t / C, c = t - slot * C;
    const bool act = slot < ns;
    float xr[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) xr[j] = act ? v[c * 33 + j] : 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = slot + ns * u;
        float d = 0.f;
        const uint32_t ww[8] = {q[u][0].x, q[u][0].y, q[u][0].z, q[u][0].w, q[u][1].x, q[u][1].y, q[u][1].z, q[u][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int bt = 0; bt < 4; ++bt)
                d = __builtin_fmaf((float)(int8_t)(ww[e] >> (8 * bt)), xr[4 * e + bt], d);
        if (act && j < nr) red[j * C + c] = d;
    }
    __syncthreads();
    // row sums: 8 lanes per row in column order, then a fixed combine
    block_reduce_rows(red, C, nr, kA1Threads / 64, out, [](int) { return true; });
    __syncthreads();
}

__global__ void __launch_bounds__(kA1Threads) k_attn1(Attn1Args A) {
#pragma clang fp contract(off)
    __shared__ float s_x[kA1HMax];
    __shared__ float s_v[kA1QMax / 32 * 33];     // xb (phase 1), then the attention output (phase 3)
    __shared__ float red[kA1UQ * kA1Threads];
    __shared__ float s_out[512];
    __shared__ float s_part[16];
    __shared__ float uq[256], uk[256];
    __shared__ __attribute__((aligned(16))) uint16_t kcur[256], vcur[256];
    __shared__ float s_inv[2];
    __shared__ float sc[kA1P];
    __shared__ float ob[kA1Threads / 8 * 64 > kA1Threads / 64 * 256 ? kA1Threads / 8 * 64 : kA1Threads / 64 * 256];
    __shared__ float s_m[kA1MaxS], s_l[kA1MaxS];
    __shared__ int s_late;
    const int b = blockIdx.x, t = threadIdx.x, NB = gridDim.x;
    const int H = A.H, hd = A.hd, C1 = H / 32, C3 = A.qd / 32;
    const unsigned tag = A.tag;
    if (t == 0) s_late = 0;
    // ------------------------------------------------------------ 1: q, k, v
    // the weight rows of phases 1 and 3 are issued first: they depend on
    // nothing, and land while x is read and normalized and the heads run
    const int q0 = A.RQ * b, nq = max(0, min(A.QR - q0, A.RQ));
    const int o0 = A.RO * b, no = max(0, min(H - o0, A.RO));
    auto qkv_row = [&](int j) __attribute__((always_inline)) {
        const int gr = q0 + j;
        const int m = gr < A.qd ? 0 : gr < A.qd + A.kvd ? 1 : 2;
        const int lr = gr - (m == 0 ? 0 : m == 1 ? A.qd : A.qd + A.kvd);
        return (m == 0 ? A.w[0] : m == 1 ? A.w[1] : A.w[2]) + (size_t)lr * (size_t)H;
    };
    mh_u4 wq1[kA1UQ][2], wo3[kA1UO][2];
    a1_issue<kA1UQ>(qkv_row, nq, C1, wq1);
    a1_issue<kA1UO>([&](int j) __attribute__((always_inline)) { return A.w[3] + (size_t)(o0 + j) * (size_t)A.qd; },
                    no, C3, wo3);
    {
        float ss = 0.f;
        for (int i = t; i < H; i += kA1Threads) {
            const float xv = A.x[i];
            s_x[i] = xv;
            ss = __builtin_fmaf(xv, xv, ss);
        }
        ss = mh_wave_sum(ss);
        if ((t & 63) == 0) s_part[t >> 6] = ss;
        __syncthreads();
        ss = 0.f;
        for (int w = 0; w < kA1Threads / 64; ++w) ss += s_part[w];
        const float inv = 1.0f / sqrtf(ss / (float)H + A.eps);
        for (int i = t; i < H; i += kA1Threads) s_v[(i >> 5) * 33 + (i & 31)] = s_x[i] * inv * A.an[i];
        __syncthreads();
        a1_math<kA1UQ>(wq1, nq, C1, s_v, red, s_out);
        for (int j = t; j < nq; j += kA1Threads) {
            const int gr = q0 + j;
            const int m = gr < A.qd ? 0 : gr < A.qd + A.kvd ? 1 : 2;
            const int lr = gr - (m == 0 ? 0 : m == 1 ? A.qd : A.qd + A.kvd);
            const float y = s_out[j] * A.ws[m][lr];
            st_tag(A.qkv + gr, tag, y + A.b[m][lr]);
        }
    }
    // ------------------------------------------------------------ 2: heads
    if (b < A.nh * A.S) {
        constexpr int T = kA1Threads, PPT = kA1PPT, P = kA1P;
        const int h = b / A.S, s = b - h * A.S;
        const int kh = h / A.gq, half = hd / 2, i = t, lane = t & 63, wv = t >> 6;
        float xq = 0.f, xk = 0.f, xv = 0.f, cs = 0.f, sn = 0.f, wq = 0.f, wk = 0.f;
        if (i < hd) {
            const uint64_t *pq = A.qkv + (size_t)h * hd + i, *pk = A.qkv + A.qd + (size_t)kh * hd + i;
            const uint64_t *pv = A.qkv + A.qd + A.kvd + (size_t)kh * hd + i;
            uint64_t a = ld_tag(pq), c = ld_tag(pk), d = ld_tag(pv);
            for (unsigned spins = 0; !(tag_is(a, tag) && tag_is(c, tag) && tag_is(d, tag)); ++spins) {
                if (spins > kSpinLimit) {
                    s_late = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                if (!tag_is(a, tag)) a = ld_tag(pq);
                if (!tag_is(c, tag)) c = ld_tag(pk);
                if (!tag_is(d, tag)) d = ld_tag(pv);
            }
            xq = tag_val(a);
            xk = tag_val(c);
            xv = tag_val(d);
            if (A.qk_norm) {
                wq = A.qn[i];
                wk = A.kn[i];
            }
            uq[i] = xq;
            uk[i] = xk;
        }
        if (i < half) {
            cs = A.co[i];
            sn = A.si[i];
        }
        __syncthreads();
        if (s_late) {
            if (t == 0) raise_err(A.err);
            return;
        }
        if (A.qk_norm) {
            if (i == 0 || i == 64) {   // the reference's sequential sums of squares
                const float *u = i == 0 ? uq : uk;
                float ssq = 0.f;
                for (int j = 0; j < hd; ++j) ssq += u[j] * u[j];
                s_inv[i == 0 ? 0 : 1] = 1.0f / sqrtf(ssq / (float)hd + A.eps);
            }
            __syncthreads();
            const float vq = i < hd ? uq[i] * s_inv[0] * wq : 0.f;
            const float vk = i < hd ? uk[i] * s_inv[1] * wk : 0.f;
            __syncthreads();
            if (i < hd) {
                uq[i] = vq;
                uk[i] = vk;
            }
            __syncthreads();
        }
        float r0 = 0.f, r1 = 0.f, k0 = 0.f, k1 = 0.f;
        if (i < half) {
            const float a = uq[i], c = uq[i + half], bb = uk[i], d = uk[i + half];
            r0 = a * cs - c * sn;
            r1 = c * cs + a * sn;
            k0 = bb * cs - d * sn;
            k1 = d * cs + bb * sn;
        }
        __syncthreads();
        if (i < half) {
            uq[i] = r0;
            uq[i + half] = r1;
            uk[i] = k0;
            uk[i + half] = k1;
        }
        __syncthreads();
        if (i < hd) {
            kcur[i] = to_f16_ref(uk[i]);
            vcur[i] = to_f16_ref(xv);
            if (h % A.gq == 0 && s == 0) {
                const size_t o = (size_t)A.slot * A.kvd + (size_t)kh * hd + i;
                A.kc[o] = kcur[i];
                A.vc[o] = vcur[i];
            }
        }
        __syncthreads();
        // scores: positions t0 + i + T r, the reference's f16 dot order
        const int t0 = P * s;
        float dd[PPT];
        if (A.kvec) {   // head_dim 64: one 16-byte load per 8 cached values
            uint4 kw[PPT][8];
#pragma unroll
            for (int r = 0; r < PPT; ++r) {
                const int tt = t0 + i + T * r;
                const bool cur = tt == A.slot || tt >= A.nctx;
                const uint16_t *kt = cur ? kcur : A.kc + (size_t)tt * A.kvd + (size_t)kh * hd;
#pragma unroll
                for (int c = 0; c < 8; ++c) kw[r][c] = *(const uint4 *)(kt + 8 * c);
            }
#pragma unroll
            for (int r = 0; r < PPT; ++r) {
                float d = 0.f;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const uint32_t ww[4] = {kw[r][c].x, kw[r][c].y, kw[r][c].z, kw[r][c].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        d += uq[8 * c + 2 * j] * mh_f16((uint16_t)(ww[j] & 0xffffu));
                        d += uq[8 * c + 2 * j + 1] * mh_f16((uint16_t)(ww[j] >> 16));
                    }
                }
                dd[r] = d;
            }
        } else {
#pragma unroll
            for (int r = 0; r < PPT; ++r) {
                const int tt = t0 + i + T * r;
                float d = 0.f;
                if (tt < A.nctx) {
                    const uint16_t *kt = tt == A.slot ? kcur : A.kc + (size_t)tt * A.kvd + (size_t)kh * hd;
                    for (int j = 0; j < hd; ++j) d += uq[j] * f16_at(kt + j);
                }
                dd[r] = d;
            }
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            dd[r] = t0 + i + T * r < A.nctx ? dd[r] * A.scale : -INFINITY;
            mloc = fmaxf(mloc, dd[r]);
        }
        const float m = block_max_f(mloc, s_part);
        float el = 0.f;
#pragma unroll
        for (int r = 0; r < PPT; ++r) {
            const float e = t0 + i + T * r < A.nctx ? expf(dd[r] - m) : 0.f;
            sc[i + T * r] = e;
            el += e;
        }
        const float l = block_sum_f(el, s_part);   // (its barriers also order the sc writes)
        const int np = min(P, A.nctx - t0);
        if (A.kvec) {
            constexpr int NG = T / 8, NPT = P / NG;
            const int pg = i >> 3, dc = i & 7;
            float o8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            uint4 w8[NPT];
#pragma unroll
            for (int u = 0; u < NPT; ++u) {
                const int j = pg + NG * u, tt = t0 + j;
                w8[u] = (j < np && tt != A.slot) ? *(const uint4 *)(A.vc + (size_t)tt * A.kvd + (size_t)kh * hd + 8 * dc)
                                                 : *(const uint4 *)(vcur + 8 * dc);
            }
#pragma unroll
            for (int u = 0; u < NPT; ++u) {
                const int j = pg + NG * u;
                if (j < np) {
                    const float e = sc[j];
                    const uint32_t ww[4] = {w8[u].x, w8[u].y, w8[u].z, w8[u].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        o8[2 * q] += e * mh_f16((uint16_t)(ww[q] & 0xffffu));
                        o8[2 * q + 1] += e * mh_f16((uint16_t)(ww[q] >> 16));
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) ob[pg * 64 + 8 * dc + q] = o8[q];
            __syncthreads();
            float o = 0.f;
            if (i < 64)
                for (int g2 = 0; g2 < NG; ++g2) o += ob[g2 * 64 + i];
            __syncthreads();
            for (int q = i; q < T / 64 * 256; q += T) ob[q] = 0.f;
            __syncthreads();
            if (i < 64) ob[i] = o;
        } else {
            constexpr int NW = T / 64, U = 8;
            for (int i0 = 0; i0 < hd; i0 += 64) {
                const int dm = i0 + lane;
                float o = 0.f;
                if (dm < hd) {
                    const uint16_t *vb = A.vc + (size_t)kh * hd + dm;
                    const float vslot = mh_f16(vcur[dm]);
                    int j = wv;
                    for (; j + NW * (U - 1) < np; j += NW * U) {
                        float vvv[U];
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const int tt = t0 + j + NW * u;
                            vvv[u] = tt == A.slot ? vslot : mh_f16(vb[(size_t)tt * A.kvd]);
                        }
#pragma unroll
                        for (int u = 0; u < U; ++u) o += sc[j + NW * u] * vvv[u];
                    }
                    for (; j < np; j += NW) {
                        const int tt = t0 + j;
                        o += sc[j] * (tt == A.slot ? vslot : mh_f16(vb[(size_t)tt * A.kvd]));
                    }
                }
                if (dm < 256) ob[wv * 256 + dm] = dm < hd ? o : 0.f;
            }
        }
        __syncthreads();
        const float sinkv = A.sinks ? A.sink[h] : -1e30f;
        if (A.S == 1) {
            float M = m;
            if (sinkv > M) M = sinkv;
            const float f = expf(m - M);
            float den = l * f;
            if (A.sinks) den += expf(sinkv - M);
            const float inv = 1.0f / den;
            for (int dm = i; dm < hd; dm += T) {
                float o = 0.f;
#pragma unroll
                for (int w = 0; w < T / 64; ++w) o += ob[w * 256 + dm];
                const float ov = o * f * inv;
#pragma unroll
                for (int cp = 0; cp < kAR; ++cp) st_tag(A.ao + (size_t)cp * A.aos + (size_t)h * hd + dm, tag, ov);
            }
        } else {
            uint64_t *pp = A.part + ((size_t)h * A.S + s) * (hd + 2);
            for (int dm = i; dm < hd; dm += T) {
                float o = 0.f;
#pragma unroll
                for (int w = 0; w < T / 64; ++w) o += ob[w * 256 + dm];
                st_tag(pp + dm, tag, o);
            }
            if (i == 0) {
                st_tag(pp + hd, tag, m);
                st_tag(pp + hd + 1, tag, l);
            }
            if (s == 0) {
                // split 0 combines: every split's m and l, then its o values
                if (i < A.S) {
                    const uint64_t *ps = A.part + ((size_t)h * A.S + i) * (hd + 2);
                    uint64_t wm = ld_tag(ps + hd), wl = ld_tag(ps + hd + 1);
                    for (unsigned spins = 0; !(tag_is(wm, tag) && tag_is(wl, tag)); ++spins) {
                        if (spins > kSpinLimit) {
                            s_late = 1;
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                        if (!tag_is(wm, tag)) wm = ld_tag(ps + hd);
                        if (!tag_is(wl, tag)) wl = ld_tag(ps + hd + 1);
                    }
                    s_m[i] = tag_val(wm);
                    s_l[i] = tag_val(wl);
                }
                __syncthreads();
                if (s_late) {
                    if (t == 0) raise_err(A.err);
                    return;
                }
                float M = sinkv;
                for (int q = 0; q < A.S; ++q) M = fmaxf(M, s_m[q]);
                float den = 0.f;
                for (int q = 0; q < A.S; ++q) den += s_l[q] * expf(s_m[q] - M);
                if (A.sinks) den += expf(sinkv - M);
                const float inv = 1.0f / den;
                // the head's output into ob (its partials were read above),
                // published only once every split's words have arrived
                for (int dm = i; dm < hd; dm += T) {
                    float o = 0.f;
                    for (int q = 0; q < A.S; ++q) {
                        const uint64_t *po = A.part + ((size_t)h * A.S + q) * (hd + 2) + dm;
                        uint64_t wo = ld_tag(po);
                        for (unsigned spins = 0; !tag_is(wo, tag); ++spins) {
                            if (spins > kSpinLimit) {
                                s_late = 1;
                                break;
                            }
                            __builtin_amdgcn_s_sleep(1);
                            wo = ld_tag(po);
                        }
                        o += tag_val(wo) * expf(s_m[q] - M);
                    }
                    ob[dm] = o * inv;
                }
                __syncthreads();
                if (s_late) {
                    if (t == 0) raise_err(A.err);
                    return;
                }
                for (int dm = i; dm < hd; dm += T) {
                    const float ov = ob[dm];
#pragma unroll
                    for (int cp = 0; cp < kAR; ++cp) st_tag(A.ao + (size_t)cp * A.aos + (size_t)h * hd + dm, tag, ov);
                }
            }
        }
    }
    // ------------------------------------------------------------ 3: o + residual
    if (no > 0) {
        // every word of the thread's share loaded at once, then only the
        // late ones polled again
        constexpr int NA = kA1QMax / kA1Threads;
        const uint64_t *src = A.ao + (size_t)(b % kAR) * A.aos;
        const int tt = opaque(t);
        uint64_t w[NA];
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int i = tt + k * kA1Threads;
            w[k] = i < A.qd ? ld_tag(src + i) : (uint64_t)tag << 32;
        }
        bool late = false;
        for (unsigned spins = 0;; ++spins) {
            bool ready = true;
#pragma unroll
            for (int k = 0; k < NA; ++k) ready = ready && tag_is(w[k], tag);
            if (ready) break;
            if (spins > kSpinLimit) {
                late = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int k = 0; k < NA; ++k) {
                const int i = tt + k * kA1Threads;
                if (i < A.qd && !tag_is(w[k], tag)) w[k] = ld_tag(src + i);
            }
        }
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            const int i = t + k * kA1Threads;
            if (i < A.qd) s_v[(i >> 5) * 33 + (i & 31)] = tag_val(w[k]);
        }
        if (__syncthreads_or(late)) {
            if (t == 0) raise_err(A.err);
            return;
        }
        a1_math<kA1UO>(wo3, no, C3, s_v, red, s_out);
        for (int j = t; j < no; j += kA1Threads) {
            const float y = s_out[j] * A.ws[3][o0 + j] + A.b[3][o0 + j];
            A.x[o0 + j] = s_x[o0 + j] + y;
        }
    }
    (void)NB;
}

__global__ void k_attn_clear(unsigned *p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// y = o + bias; x += y (two roundings, as wk_addbias then the residual loop)
__global__ void __launch_bounds__(kAttnThreads)
k_attn_residual(float *__restrict__ x, const float *__restrict__ o, const float *__restrict__ bo, int64_t H) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < H) {
        const float y = o[i] + bo[i];
        x[i] = x[i] + y;
    }
}

}  // namespace
}  // namespace mh

using namespace mh;

extern "C" {

int mh_attention_dev(const mh_attn_layer *L, float *x, int pos) {
    clear_error();
    if (!L || !x) return fail(MH_E_ARG, "mh_attention_dev: NULL layer or x");
    const int64_t H = L->hidden;
    const int nh = L->n_heads, nkv = L->n_kv_heads, hd = L->head_dim;
    if (H < 1 || nh < 1 || nkv < 1 || nh % nkv != 0 || hd < 2 || hd % 2 != 0 || hd > 256 || L->ctx < 1)
        return fail(MH_E_ARG, "mh_attention_dev: shape (hidden %lld, heads %d/%d, head_dim %d, ctx %d)", (long long)H,
                    nh, nkv, hd, L->ctx);
    if (pos < 0 || pos >= L->ctx) return fail(MH_E_ARG, "mh_attention_dev: position %d outside [0, %d)", pos, L->ctx);
    if ((int64_t)std::min(L->ctx, L->window > 0 ? L->window : L->ctx) > (int64_t)kSplitT * kSplitP * kMaxSplits)
        return fail(MH_E_UNSUPPORTED, "mh_attention_dev: more than %d cached positions", kSplitT * kSplitP * kMaxSplits);
    if (L->qk_norm && (!L->qn || !L->kn)) return fail(MH_E_ARG, "mh_attention_dev: qk_norm without weights");
    if (L->sinks && !L->sink) return fail(MH_E_ARG, "mh_attention_dev: sinks without values");
    const int kvd = nkv * hd, qd = nh * hd;
    if (L->wq.rows != qd || L->wq.cols != H || L->wk.rows != kvd || L->wk.cols != H || L->wv.rows != kvd ||
        L->wv.cols != H || L->wo.rows != H || L->wo.cols != qd)
        return fail(MH_E_ARG, "mh_attention_dev: projection shapes do not match the heads");
    MH_TRY(require_init());
    const int cap = (L->window > 0 && L->window < L->ctx) ? L->window : L->ctx;
    DevWT wq, wk, wv, wo;
    MH_TRY(resolve_wt(&L->wq, &wq, "attention wq"));
    MH_TRY(resolve_wt(&L->wk, &wk, "attention wk"));
    MH_TRY(resolve_wt(&L->wv, &wv, "attention wv"));
    MH_TRY(resolve_wt(&L->wo, &wo, "attention wo"));
    const void *bq, *bk, *bv, *bo, *an, *qn = nullptr, *kn = nullptr, *sk = nullptr, *co, *si;
    MH_TRY(resolve_weight(L->bq, (uint64_t)qd * 4, &bq, "attention bq"));
    MH_TRY(resolve_weight(L->bk, (uint64_t)kvd * 4, &bk, "attention bk"));
    MH_TRY(resolve_weight(L->bv, (uint64_t)kvd * 4, &bv, "attention bv"));
    MH_TRY(resolve_weight(L->bo, (uint64_t)H * 4, &bo, "attention bo"));
    MH_TRY(resolve_weight(L->attn_norm, (uint64_t)H * 4, &an, "attention norm"));
    if (L->qk_norm) {
        MH_TRY(resolve_weight(L->qn, (uint64_t)hd * 4, &qn, "attention q norm"));
        MH_TRY(resolve_weight(L->kn, (uint64_t)hd * 4, &kn, "attention k norm"));
    }
    if (L->sinks) MH_TRY(resolve_weight(L->sink, (uint64_t)nh * 4, &sk, "attention sinks"));
    const uint64_t tab = (uint64_t)L->ctx * (hd / 2) * 4;
    MH_TRY(resolve_weight(L->rope_cos, tab, &co, "rope cos"));
    MH_TRY(resolve_weight(L->rope_sin, tab, &si, "rope sin"));
    MH_TRY(resolve_dev(L->kc, (uint64_t)cap * kvd * 2, "attention k cache"));
    MH_TRY(resolve_dev(L->vc, (uint64_t)cap * kvd * 2, "attention v cache"));
    MH_TRY(resolve_dev(x, (uint64_t)H * 4, "mh_attention_dev x"));
    // scratch: the heads' arrival counters [nh] (zeroed when the slot is
    // (re)allocated; every call leaves them zero), xb / o [H], q [qd], k, v
    // [kvd], the splits' partials [nh][S][hd + 2], ao [qd]
    const int nctx = pos + 1 < cap ? pos + 1 : cap;
    // up to 256 cached positions (the sliding layers): 256-thread blocks,
    // one position per thread; beyond: 1024 threads, two positions each
    const bool small = nctx <= 256;
    const int P = small ? 256 : kSplitT * kSplitP;
    const int S = (nctx + P - 1) / P;
    const size_t oc = 0, ox = ((size_t)nh * 4 + 255) & ~(size_t)255;
    const size_t oq = ox + (((size_t)H * 4 + 255) & ~(size_t)255), ok = oq + (((size_t)qd * 4 + 255) & ~(size_t)255);
    const size_t ov = ok + (((size_t)kvd * 4 + 255) & ~(size_t)255), op = ov + (((size_t)kvd * 4 + 255) & ~(size_t)255);
    const size_t oo = op + (((size_t)nh * S * (hd + 2) * 4 + 255) & ~(size_t)255), total = oo + (size_t)qd * 4;
    // sized for the longest context, so the slot is not reallocated as the
    // context grows
    const int Smax = (cap + kSplitT * kSplitP - 1) / (kSplitT * kSplitP);
    const size_t total_max = total + (size_t)nh * (Smax - S) * (hd + 2) * 4 + 256;
    void *p;
    bool fresh = false;
    MH_TRY(scratch(S_ATTN, total_max, &p, &fresh));
    static int cleared_nh = 0;   // heads whose counters the slot holds zeroed (0 after a (re)allocation)
    if (fresh) cleared_nh = 0;
    uint8_t *b8 = (uint8_t *)p;
    unsigned *cnt = (unsigned *)(b8 + oc);
    if (nh > cleared_nh) {
        MH_LAUNCH("attn_clear", k_attn_clear, dim3(1), dim3(256), 0, stream(), cnt, nh);
        cleared_nh = nh;
    }
    float *xb = (float *)(b8 + ox), *q = (float *)(b8 + oq), *k = (float *)(b8 + ok), *v = (float *)(b8 + ov);
    float *part = (float *)(b8 + op), *ao = (float *)(b8 + oo);
    hipStream_t s = stream();
    {
        // the one-launch kernel when its limits hold (int8 projections, the
        // LDS capacities, every head's splits in the grid, one block per CU
        // resident); the ATTN_SPLIT switch keeps the separate launches, so
        // callers can compare the two
        const int cus = device_cus(), QR = qd + 2 * kvd;
        const int RQ = (QR + cus - 1) / cus, NB = (QR + RQ - 1) / RQ;
        const int C1 = (int)(H / 32), C3 = qd / 32;
        const int ns1 = C1 >= 1 ? kA1Threads / C1 : 0, ns3 = C3 >= 1 ? kA1Threads / C3 : 0;
        const int RO = (int)((H + NB - 1) / NB), S1 = (nctx + kA1P - 1) / kA1P;
        bool ok1 = !sw(SW_ATTN_SPLIT);
        for (const DevWT *w : {&wq, &wk, &wv, &wo})
            ok1 = ok1 && w->dt == MH_DT_Q8R && w->scales && (uintptr_t)w->data % 16 == 0;
        ok1 = ok1 && H % 32 == 0 && H <= kA1HMax && qd % 32 == 0 && qd <= kA1QMax && ns1 >= 1 && ns3 >= 1 &&
              RQ <= std::min(512, ns1 * kA1UQ) && RO <= std::min(512, ns3 * kA1UO) && hd <= 256 && S1 <= kA1MaxS &&
              nh * S1 <= NB;
        static int occ_dev = -1, occ = 0;
        if (ok1) {
            int dev = 0;
            MH_HIP(hipGetDevice(&dev));
            if (dev != occ_dev) {
                MH_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)k_attn1, kA1Threads, 0));
                occ_dev = dev;
            }
            ok1 = occ >= 1;
        }
        if (ok1) {
            unsigned *err_dev = nullptr;
            MH_TRY(async_flag(F_ATTN1, "attention: an exchange timed out (blocks not co-resident)", &err_dev));
            // exchange words: q/k/v rows, the splits' partials, kAR copies of
            // the attention output (zeroed when the slot is (re)allocated: a
            // launch's tag is never 0 and never repeats)
            const size_t aos = ((size_t)qd + 15) / 16 * 16 + 32;
            const size_t wqkv = ((size_t)QR + 31) / 32 * 32, wpart = ((size_t)nh * kA1MaxS * (hd + 2) + 31) / 32 * 32;
            const size_t words = wqkv + wpart + kAR * aos;
            const size_t words_max = words;
            void *p1;
            bool fresh1 = false;
            MH_TRY(scratch(S_ATTN1, words_max * 8, &p1, &fresh1));
            // launch tags count up from 1 over words zeroed when the slot is
            // (re)allocated or grows; before the count could wrap to 0 the
            // words are zeroed again and the count restarts (a word left
            // from an older launch then never matches a later tag)
            static size_t zeroed_words = 0;
            static unsigned tag = 0;
            if (fresh1) zeroed_words = 0;
            if (words > zeroed_words || tag >= 0xF0000000u) {
                MH_LAUNCH("attn_clear", k_attn_clear, dim3(64), dim3(256), 0, s, (unsigned *)p1, (int)(2 * words_max));
                zeroed_words = words_max;
                tag = 0;
            }
            Attn1Args A;
            A.w[0] = (const int8_t *)wq.data;
            A.w[1] = (const int8_t *)wk.data;
            A.w[2] = (const int8_t *)wv.data;
            A.w[3] = (const int8_t *)wo.data;
            A.ws[0] = (const float *)wq.scales;
            A.ws[1] = (const float *)wk.scales;
            A.ws[2] = (const float *)wv.scales;
            A.ws[3] = (const float *)wo.scales;
            A.b[0] = (const float *)bq;
            A.b[1] = (const float *)bk;
            A.b[2] = (const float *)bv;
            A.b[3] = (const float *)bo;
            A.an = (const float *)an;
            A.qn = (const float *)qn;
            A.kn = (const float *)kn;
            A.co = (const float *)co + (size_t)pos * (hd / 2);
            A.si = (const float *)si + (size_t)pos * (hd / 2);
            A.sink = (const float *)sk;
            A.kc = L->kc;
            A.vc = L->vc;
            A.x = x;
            A.qkv = (uint64_t *)p1;
            A.part = A.qkv + wqkv;
            A.ao = A.part + wpart;
            A.err = err_dev;
            A.H = (int)H;
            A.nh = nh;
            A.hd = hd;
            A.gq = nh / nkv;
            A.qd = qd;
            A.kvd = kvd;
            A.QR = QR;
            A.nctx = nctx;
            A.slot = pos % cap;
            A.S = S1;
            A.sinks = L->sinks ? 1 : 0;
            A.qk_norm = L->qk_norm ? 1 : 0;
            A.kvec = hd == 64 && (uintptr_t)L->kc % 16 == 0 && (uintptr_t)L->vc % 16 == 0;
            A.RQ = RQ;
            A.RO = RO;
            A.aos = (int)aos;
            A.eps = L->norm_eps;
            A.scale = L->attn_scale;
            A.tag = ++tag;
            MH_LAUNCH("attn1", k_attn1, dim3((unsigned)NB), dim3(kA1Threads), 0, s, A);
            return hip_check(hipGetLastError(), "attention launch");
        }
    }
    {
        const DevWT w3[3] = {wq, wk, wv};
        float *const y3[3] = {q, k, v};
        const float *nw = (const float *)an;
        bool done = false;
        switch (wq.dt) {
        case MH_DT_F32: MH_TRY(launch_qkv_t<MH_DT_F32>(w3, x, nw, L->norm_eps, y3, s, &done)); break;
        case MH_DT_Q8R: MH_TRY(launch_qkv_t<MH_DT_Q8R>(w3, x, nw, L->norm_eps, y3, s, &done)); break;
        case MH_DT_Q4G32: MH_TRY(launch_qkv_t<MH_DT_Q4G32>(w3, x, nw, L->norm_eps, y3, s, &done)); break;
        case MH_DT_MXFP4: MH_TRY(launch_qkv_t<MH_DT_MXFP4>(w3, x, nw, L->norm_eps, y3, s, &done)); break;
        }
        if (!done) {
            MH_TRY(launch_rmsnorm(x, nw, xb, H, L->norm_eps, 1, s));
            MH_TRY(launch_gemv(wq, xb, q, 1, s));
            MH_TRY(launch_gemv(wk, xb, k, 1, s));
            MH_TRY(launch_gemv(wv, xb, v, 1, s));
        }
    }
    const int kvec = hd % 8 == 0 && (uintptr_t)L->kc % 16 == 0 && (uintptr_t)L->vc % 16 == 0;
    SplitArgs A{q, k, v, (const float *)bq, (const float *)bk, (const float *)bv, (const float *)qn, (const float *)kn,
                (const float *)co + (size_t)pos * (hd / 2), (const float *)si + (size_t)pos * (hd / 2),
                (const float *)sk, L->kc, L->vc, part, cnt, ao, nh, hd, nh / nkv, kvd, nctx, pos % cap, S,
                L->sinks ? 1 : 0, L->qk_norm ? 1 : 0, kvec, L->attn_scale, L->norm_eps};
    if (small) MH_LAUNCH("attn_split", (k_attn_split<256, 1>), dim3((unsigned)(nh * S)), dim3(256), 0, s, A);
    else MH_LAUNCH("attn_split", (k_attn_split<kSplitT, kSplitP>), dim3((unsigned)(nh * S)), dim3(kSplitT), 0, s, A);
    bool fused = false;
    switch (wo.dt) {
    case MH_DT_F32: MH_TRY(launch_o_res_t<MH_DT_F32>(wo, ao, (const float *)bo, x, s, &fused)); break;
    case MH_DT_Q8R: MH_TRY(launch_o_res_t<MH_DT_Q8R>(wo, ao, (const float *)bo, x, s, &fused)); break;
    case MH_DT_Q4G32: MH_TRY(launch_o_res_t<MH_DT_Q4G32>(wo, ao, (const float *)bo, x, s, &fused)); break;
    case MH_DT_MXFP4: MH_TRY(launch_o_res_t<MH_DT_MXFP4>(wo, ao, (const float *)bo, x, s, &fused)); break;
    }
    if (!fused) {
        MH_TRY(launch_gemv(wo, ao, xb, 1, s));
        MH_LAUNCH("attn_residual", k_attn_residual, dim3((unsigned)((H + kAttnThreads - 1) / kAttnThreads)),
                  dim3(kAttnThreads), 0, s, x, xb, (const float *)bo, H);
    }
    return hip_check(hipGetLastError(), "attention launch");
}

}  // extern "C"
