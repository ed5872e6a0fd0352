// mh_sample.hip — sample() (engine/midge.c:654-679) on device logits: the
// token after the lm_head GEMV, without copying the vocabulary's logits to
// the host.
//
//   temp <= 0   the first maximum (a strictly larger value wins, so equal
//               maxima go to the lowest index; NaN never wins, and a NaN at
//               index 0 makes the answer 0, as the reference's loop gives)
//   temp > 0    p[i] = expf((l[i] - max) / temp) / (float)sum (f64 sum);
//               tokens by falling p (stable: equal p in index order); the
//               smallest prefix whose f64 sum reaches topp; the first token
//               where the running sum reaches u * (float)(prefix sum).
//
// u is the caller's uniform draw (the reference draws rng_f() at that point
// of sample(), and only when temp > 0).
#include <hipcub/hipcub.hpp>

#include "mh_internal.h"

namespace mh {
namespace {

constexpr int kSampThreads = 256;
constexpr int kSampBlocks = 256;    // partial reductions per pass
constexpr int kScanThreads = 1024;  // the nucleus scan (one block)

struct MaxIdx {
    float v;
    int i;
};

// the reference loop's order: a larger value wins, equal values go to the
// lower index, NaN never wins
__device__ __forceinline__ MaxIdx max_of(MaxIdx a, MaxIdx b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ __forceinline__ MaxIdx wave_max(MaxIdx m) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        MaxIdx n;
        n.v = __shfl_xor(m.v, o, 64);
        n.i = __shfl_xor(m.i, o, 64);
        m = max_of(m, n);
    }
    return m;
}

// block-wide max of one value per thread (all threads get it)
__device__ MaxIdx block_max(MaxIdx m) {
    __shared__ float sv[16];
    __shared__ int si[16];
    m = wave_max(m);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = m.v;
        si[w] = m.i;
    }
    __syncthreads();
    MaxIdx r{-INFINITY, INT32_MAX};
    for (int i = 0; i < nw; ++i) r = max_of(r, MaxIdx{sv[i], si[i]});
    __syncthreads();
    return r;
}

// per-block maxima of logits[V] (grid-stride)
__global__ void __launch_bounds__(kSampThreads)
k_samp_max(const float *__restrict__ lg, int V, MaxIdx *__restrict__ part) {
    MaxIdx m{-INFINITY, INT32_MAX};
    for (int i = blockIdx.x * kSampThreads + threadIdx.x; i < V; i += gridDim.x * kSampThreads)
        m = max_of(m, MaxIdx{lg[i], i});
    m = block_max(m);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// the maximum over the partials, with the reference loop's index-0 rule
__device__ __forceinline__ MaxIdx final_max(const float *lg, const MaxIdx *part) {
    MaxIdx m{-INFINITY, INT32_MAX};
    for (int b = threadIdx.x; b < kSampBlocks; b += blockDim.x) m = max_of(m, part[b]);
    m = block_max(m);
    if (__builtin_isnan(lg[0]) || m.i == INT32_MAX) m = MaxIdx{lg[0], 0};
    return m;
}

__global__ void __launch_bounds__(kSampThreads)
k_samp_greedy(const float *__restrict__ lg, const MaxIdx *__restrict__ part, int32_t *__restrict__ out) {
    const MaxIdx m = final_max(lg, part);
    if (threadIdx.x == 0) *out = m.i;
}

// p[i] = expf((l[i] - max) / temp), ids[i] = i; per-block f64 sums
__global__ void __launch_bounds__(kSampThreads)
k_samp_exp(const float *__restrict__ lg, int V, float temp, const MaxIdx *__restrict__ part, float *__restrict__ p,
           int *__restrict__ ids, double *__restrict__ dsum) {
    __shared__ double sd[kSampThreads / 64];
    const float mx = final_max(lg, part).v;
    double s = 0;
    for (int i = blockIdx.x * kSampThreads + threadIdx.x; i < V; i += gridDim.x * kSampThreads) {
        const float e = expf((lg[i] - mx) / temp);
        p[i] = e;
        ids[i] = i;
        s += e;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) sd[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0;
        for (int w = 0; w < kSampThreads / 64; ++w) t += sd[w];
        dsum[blockIdx.x] = t;
    }
}

// p[i] /= (float)den, den the f64 sum of the partials (fixed order)
__global__ void __launch_bounds__(kSampThreads)
k_samp_norm(float *__restrict__ p, int V, const double *__restrict__ dsum) {
    __shared__ float s_den;
    if (threadIdx.x == 0) {
        double den = 0;
        for (int b = 0; b < kSampBlocks; ++b) den += dsum[b];
        s_den = (float)den;
    }
    __syncthreads();
    const float den = s_den;
    for (int i = blockIdx.x * kSampThreads + threadIdx.x; i < V; i += gridDim.x * kSampThreads) p[i] = p[i] / den;
}

// inclusive f64 scan of one value per thread over the block; returns the
// thread's prefix and sets *total to the block's sum
__device__ double block_scan(double v, double *total) {
    __shared__ double ws[kScanThreads / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    if (lane == 63) ws[w] = v;
    __syncthreads();
    double before = 0, all = 0;
    for (int i = 0; i < kScanThreads / 64; ++i) {
        if (i < w) before += ws[i];
        all += ws[i];
    }
    __syncthreads();
    *total = all;
    return before + v;
}

// The nucleus and the pick over the sorted probabilities ps (falling) and
// their tokens is: one block, 1024 sorted entries per round, running f64
// sums kept in pre[] for the pick.
__global__ void __launch_bounds__(kScanThreads)
k_samp_pick(const float *__restrict__ ps, const int *__restrict__ is, int V, float topp, float u,
            double *__restrict__ pre, int32_t *__restrict__ out) {
    __shared__ int s_n;
    __shared__ double s_cum;
    if (threadIdx.x == 0) s_n = INT32_MAX;
    __syncthreads();
    double carry = 0;
    int n = V;
    for (int base = 0; base < V; base += kScanThreads) {
        const int i = base + threadIdx.x;
        double total;
        const double c = carry + block_scan(i < V ? (double)ps[i] : 0.0, &total);
        if (i < V) {
            pre[i] = c;
            if (c >= (double)topp) atomicMin(&s_n, i + 1);
        }
        carry += total;
        __syncthreads();
        if (s_n != INT32_MAX) {
            n = s_n;
            break;
        }
    }
    if (threadIdx.x == 0) s_cum = pre[n - 1];
    __syncthreads();
    const float r = u * (float)s_cum;
    if (threadIdx.x == 0) s_n = INT32_MAX;
    __syncthreads();
    for (int base = 0; base < n; base += kScanThreads) {
        const int i = base + threadIdx.x;
        if (i < n && (double)r <= pre[i]) atomicMin(&s_n, i);
        __syncthreads();
        if (s_n != INT32_MAX) break;
    }
    if (threadIdx.x == 0) *out = is[s_n != INT32_MAX ? s_n : n - 1];
}

}  // namespace
}  // namespace mh

using namespace mh;

extern "C" {

int mh_sample_dev(const float *logits, int64_t V, float temp, float topp, float u, int32_t *out) {
    clear_error();
    if (!logits || !out) return fail(MH_E_ARG, "mh_sample_dev: NULL logits or out");
    if (V < 1 || V > (int64_t)INT32_MAX / 2) return fail(MH_E_ARG, "mh_sample_dev: vocabulary %lld out of range", (long long)V);
    MH_TRY(require_init());
    MH_TRY(resolve_dev(logits, (uint64_t)V * 4, "mh_sample_dev logits"));
    MH_TRY(resolve_dev(out, 4, "mh_sample_dev out"));
    hipStream_t s = stream();
    const int n = (int)V;
    // scratch: maxima and f64 partials, p and token ids, their sorted copies,
    // the running sums, then the sort's temporary storage
    size_t sort_bytes = 0;
    MH_HIP(hipcub::DeviceRadixSort::SortPairsDescending(nullptr, sort_bytes, (const float *)nullptr, (float *)nullptr,
                                                        (const int *)nullptr, (int *)nullptr, n, 0, 32, s));
    const size_t a_part = 0, a_dsum = a_part + kSampBlocks * sizeof(MaxIdx);
    const size_t a_p = (a_dsum + kSampBlocks * sizeof(double) + 255) & ~(size_t)255;
    const size_t a_ids = (a_p + (size_t)n * 4 + 255) & ~(size_t)255;
    const size_t a_ps = (a_ids + (size_t)n * 4 + 255) & ~(size_t)255;
    const size_t a_is = (a_ps + (size_t)n * 4 + 255) & ~(size_t)255;
    const size_t a_pre = (a_is + (size_t)n * 4 + 255) & ~(size_t)255;
    const size_t a_sort = (a_pre + (size_t)n * 8 + 255) & ~(size_t)255;
    void *base;
    MH_TRY(scratch(S_SAMPLE, a_sort + sort_bytes, &base));
    uint8_t *b8 = (uint8_t *)base;
    MaxIdx *part = (MaxIdx *)(b8 + a_part);
    double *dsum = (double *)(b8 + a_dsum);
    float *p = (float *)(b8 + a_p), *ps = (float *)(b8 + a_ps);
    int *ids = (int *)(b8 + a_ids), *is = (int *)(b8 + a_is);
    double *pre = (double *)(b8 + a_pre);
    MH_LAUNCH("sample_max", k_samp_max, dim3(kSampBlocks), dim3(kSampThreads), 0, s, logits, n, part);
    if (temp <= 0.f) {
        MH_LAUNCH("sample_greedy", k_samp_greedy, dim3(1), dim3(kSampThreads), 0, s, logits, part, out);
        return hip_check(hipGetLastError(), "sample launch");
    }
    MH_LAUNCH("sample_exp", k_samp_exp, dim3(kSampBlocks), dim3(kSampThreads), 0, s, logits, n, temp, part, p, ids,
              dsum);
    MH_LAUNCH("sample_norm", k_samp_norm, dim3(kSampBlocks), dim3(kSampThreads), 0, s, p, n, dsum);
    MH_HIP(hipcub::DeviceRadixSort::SortPairsDescending(b8 + a_sort, sort_bytes, p, ps, ids, is, n, 0, 32, s));
    MH_LAUNCH("sample_pick", k_samp_pick, dim3(1), dim3(kScanThreads), 0, s, ps, is, n, topp, u, pre, out);
    return hip_check(hipGetLastError(), "sample launch");
}

}  // extern "C"
