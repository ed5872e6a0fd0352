// mh_attn.hip — the trunk's attention for one decode token, attention()
// (engine/midge.c:341-400), on the device: the next component of the
// decode step beside the MoE layers.
//
//   rmsnorm          launch_rmsnorm (k_rmsnorm)
//   q, k, v          one launch on the GEMV engine (k_gemv3), any weight
//                    dtype; three launch_gemv calls where the shapes differ
//   k_attn_prep      one block per head, one thread per element: biases,
//                    per-head RMSNorm (the reference's sequential sum), RoPE
//                    from the given tables, k and v to the f16 cache slot
//                    pos % cap with the reference's conversion (wk_to_f16)
//   k_attn_heads     one block per query head: scores over the cached
//                    positions, softmax with the optional sink logit in the
//                    denominator, the weighted sum of the cached v
//   o                the GEMV engine with the residual in its epilogue
//                    (k_gemv_res: + bias, x += o); GEMV + k_attn_residual
//                    where the shape needs the general kernel
#include "mh_gemv.cuh"

namespace mh {
namespace {

constexpr int kAttnThreads = 256;

// q, k and v in one launch: the three matrices (same dtype and width) as
// consecutive block ranges of one grid, each block a k_gemv block over rows
// of one of them (block-uniform choice), into y[m] = W[m] x.
struct Gemv3Args {
    const uint8_t *W[3];
    const void *S[3];
    float *Y[3];
    int rows[3], nb[3];
    const float *x;
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

// One launch for q, k, v when their dtype and layout allow the GEMV
// engine's chunked kernel; *done = false leaves them to three launch_gemv.
template <int DT>
int launch_qkv_t(const DevWT *w, const float *x, float *const *y, hipStream_t s, bool *done) {
    constexpr int E = gemv_chunk<DT>::E;
    const int64_t cols = w[0].cols;
    *done = false;
    for (int m = 0; m < 3; ++m)
        if (w[m].dt != DT || w[m].cols != cols || ((uintptr_t)w[m].data % 16) != 0 || w[m].rows > INT32_MAX)
            return MH_OK;
    if (cols % E != 0 || cols / E > kGemvThreads || ((uintptr_t)x % 16) != 0) return MH_OK;
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
    A.cols = (int)cols;
    A.ns = ns;
    A.rpb = (int)rpb;
    const size_t lds = ((size_t)rpb + gemv_lds_floats(ns, C)) * sizeof(float);
    MH_LAUNCH("gemv_qkv", k_gemv3<DT>, dim3((unsigned)nblk), dim3(nt), lds, s, A);
    *done = true;
    return hip_check(hipGetLastError(), "q/k/v launch");
}
constexpr int kHeadThreads = 1024;   // per query head: positions, then head_dim x position groups

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

struct PrepArgs {
    float *q, *k, *v;
    const float *bq, *bk, *bv, *qn, *kn, *co, *si;
    uint16_t *kc, *vc;
    int nh, nkv, hd, slot, qk_norm;
    float eps;
};

// Block h: query head h (h < nh) or key/value head h - nh, one thread per
// element, the vector in LDS: + bias, RMSNorm with the head norm weights (if
// enabled; the reference's sequential sum of squares, in one thread), RoPE;
// q goes back to memory, k and v (+ bias) to the cache slot as f16.
__global__ void __launch_bounds__(256) k_attn_prep(PrepArgs A) {
#pragma clang fp contract(off)
    __shared__ float u[256];
    __shared__ float s_inv;
    const int h = blockIdx.x, i = threadIdx.x, hd = A.hd, half = hd / 2;
    const bool isq = h < A.nh;
    const int g = isq ? h : h - A.nh;
    float *src = isq ? A.q + (size_t)h * hd : A.k + (size_t)g * hd;
    const float *b = isq ? A.bq + (size_t)h * hd : A.bk + (size_t)g * hd;
    if (i < hd) u[i] = src[i] + b[i];
    __syncthreads();
    if (A.qk_norm) {
        const float *w = isq ? A.qn : A.kn;
        if (i == 0) {
            float ss = 0.f;
            for (int j = 0; j < hd; ++j) ss += u[j] * u[j];
            s_inv = 1.0f / sqrtf(ss / (float)hd + A.eps);
        }
        __syncthreads();
        const float val = i < hd ? u[i] * s_inv * w[i] : 0.f;
        __syncthreads();
        if (i < hd) u[i] = val;
        __syncthreads();
    }
    float r0 = 0.f, r1 = 0.f;
    if (i < half) {
        const float a = u[i], c = u[i + half];
        r0 = a * A.co[i] - c * A.si[i];
        r1 = c * A.co[i] + a * A.si[i];
    }
    __syncthreads();
    if (i < half) {
        u[i] = r0;
        u[i + half] = r1;
    }
    __syncthreads();
    if (i >= hd) return;
    if (isq) {
        src[i] = u[i];
    } else {
        const size_t o = (size_t)A.slot * A.nkv * hd + (size_t)g * hd + i;
        A.kc[o] = to_f16_ref(u[i]);
        A.vc[o] = to_f16_ref(A.v[(size_t)g * hd + i] + A.bv[(size_t)g * hd + i]);
    }
}

struct HeadArgs {
    const float *q, *sink;
    const uint16_t *kc, *vc;
    float *att, *ao;
    int hd, gq, kvd, nctx, cap, sinks;
    int kvec;   // 1: cached keys read 16 bytes at a time (hd % 8 == 0, 16-byte aligned cache)
    float scale;
};

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

// Block h = query head h over the nctx cached positions. Scores are the
// reference's sequential f16 dot (one position per thread); the softmax sum
// and the weighted sum of v are split over the block (hd dims x 1024 / hd
// position groups), so they round in a different order than the
// reference's loops.
__global__ void __launch_bounds__(kHeadThreads) k_attn_heads(HeadArgs A) {
#pragma clang fp contract(off)
    __shared__ float part[kHeadThreads / 64];
    __shared__ float qs[256];
    __shared__ float acc[kHeadThreads];
    const int h = blockIdx.x, kh = h / A.gq, hd = A.hd;
    const float *qh = A.q + (size_t)h * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) qs[i] = qh[i];
    __syncthreads();
    float *sc = A.att + (size_t)h * A.cap;
    float mx = -1e30f;
    for (int t = threadIdx.x; t < A.nctx; t += blockDim.x) {
        const uint16_t *kt = A.kc + (size_t)t * A.kvd + (size_t)kh * hd;
        float d = 0.f;
        if (A.kvec) {   // 16-byte loads of 8 cached values, summed in order
            for (int i0 = 0; i0 < hd; i0 += 8) {
                const uint4 w = *(const uint4 *)(kt + i0);
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    d += qs[i0 + 2 * j] * mh_f16((uint16_t)(ww[j] & 0xffffu));
                    d += qs[i0 + 2 * j + 1] * mh_f16((uint16_t)(ww[j] >> 16));
                }
            }
        } else {
            for (int i = 0; i < hd; ++i) d += qs[i] * mh_f16(kt[i]);
        }
        d *= A.scale;
        sc[t] = d;
        mx = fmaxf(mx, d);
    }
    mx = block_max_f(mx, part);
    const float sinkv = A.sinks ? A.sink[h] : -1e30f;
    if (sinkv > mx) mx = sinkv;
    float s = 0.f;
    for (int t = threadIdx.x; t < A.nctx; t += blockDim.x) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        s += e;
    }
    const float den = (A.sinks ? expf(sinkv - mx) : 0.f) + block_sum_f(s, part);
    const float inv = 1.0f / den;
    // thread (group j, dim i): positions j, j + nq, ... of dim i
    const int i = threadIdx.x % hd, j = threadIdx.x / hd, nq = blockDim.x / hd;
    float o = 0.f;
    if (j < nq)
        for (int t = j; t < A.nctx; t += nq)
            o += (sc[t] * inv) * mh_f16(A.vc[(size_t)t * A.kvd + (size_t)kh * hd + i]);
    if (j < nq) acc[j * hd + i] = o;
    __syncthreads();
    if (threadIdx.x < hd) {
        float r = 0.f;
        for (int q = 0; q < nq; ++q) r += acc[q * hd + threadIdx.x];
        A.ao[(size_t)h * hd + threadIdx.x] = r;
    }
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
    // scratch: xb / o [H], q [qd], k, v [kvd], scores [nh][cap], ao [qd]
    const size_t oq = ((size_t)H * 4 + 255) & ~(size_t)255, ok = oq + (((size_t)qd * 4 + 255) & ~(size_t)255);
    const size_t ov = ok + (((size_t)kvd * 4 + 255) & ~(size_t)255), oa = ov + (((size_t)kvd * 4 + 255) & ~(size_t)255);
    const size_t oo = oa + (((size_t)nh * cap * 4 + 255) & ~(size_t)255), total = oo + (size_t)qd * 4;
    void *p;
    MH_TRY(scratch(S_ATTN, total, &p));
    uint8_t *b8 = (uint8_t *)p;
    float *xb = (float *)b8, *q = (float *)(b8 + oq), *k = (float *)(b8 + ok), *v = (float *)(b8 + ov);
    float *att = (float *)(b8 + oa), *ao = (float *)(b8 + oo);
    hipStream_t s = stream();
    MH_TRY(launch_rmsnorm(x, (const float *)an, xb, H, L->norm_eps, 1, s));
    {
        const DevWT w3[3] = {wq, wk, wv};
        float *const y3[3] = {q, k, v};
        bool done = false;
        switch (wq.dt) {
        case MH_DT_F32: MH_TRY(launch_qkv_t<MH_DT_F32>(w3, xb, y3, s, &done)); break;
        case MH_DT_Q8R: MH_TRY(launch_qkv_t<MH_DT_Q8R>(w3, xb, y3, s, &done)); break;
        case MH_DT_Q4G32: MH_TRY(launch_qkv_t<MH_DT_Q4G32>(w3, xb, y3, s, &done)); break;
        case MH_DT_MXFP4: MH_TRY(launch_qkv_t<MH_DT_MXFP4>(w3, xb, y3, s, &done)); break;
        }
        if (!done) {
            MH_TRY(launch_gemv(wq, xb, q, 1, s));
            MH_TRY(launch_gemv(wk, xb, k, 1, s));
            MH_TRY(launch_gemv(wv, xb, v, 1, s));
        }
    }
    PrepArgs P{q, k, v, (const float *)bq, (const float *)bk, (const float *)bv, (const float *)qn, (const float *)kn,
               (const float *)co + (size_t)pos * (hd / 2), (const float *)si + (size_t)pos * (hd / 2), L->kc, L->vc,
               nh, nkv, hd, pos % cap, L->qk_norm ? 1 : 0, L->norm_eps};
    MH_LAUNCH("attn_prep", k_attn_prep, dim3((unsigned)(nh + nkv)), dim3((unsigned)((hd + 63) / 64 * 64)), 0, s, P);
    const int kvec = hd % 8 == 0 && (uintptr_t)L->kc % 16 == 0;
    HeadArgs A{q, (const float *)sk, L->kc, L->vc, att, ao, hd, nh / nkv, kvd, pos + 1 < cap ? pos + 1 : cap, cap,
               L->sinks ? 1 : 0, kvec, L->attn_scale};
    MH_LAUNCH("attn_heads", k_attn_heads, dim3((unsigned)nh), dim3(kHeadThreads), 0, s, A);
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
