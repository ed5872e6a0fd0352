// mh_sample.hip — sample() (engine/midge.c:654-679) on device logits: the
// token after the lm_head GEMV, without copying the vocabulary's logits to
// the host.
//
//   temp <= 0   the first maximum (a strictly larger value wins, so equal
//               maxima go to the lowest index; NaN never wins, and a NaN at
//               index 0 makes the answer 0, as the reference's loop gives)
//   temp > 0    p[i] = expf((l[i] - max) / temp) / (float)sum (f64 sum);
//               tokens by falling p (equal p in index order); the smallest
//               prefix whose f64 sum reaches topp; the first token where the
//               running sum reaches u * (float)(prefix sum).
//
// u is the caller's uniform draw (the reference draws rng_f() at that point
// of sample(), and only when temp > 0).
//
// Only the nucleus is ever ordered. Three launches (one when greedy); the
// last block of a launch to finish does the launch's single-block step
// (blocks publish with device-scope stores, the last one is found by a
// counter it resets):
//   k_samp_max      per-block maxima; last block: the maximum (greedy: the
//                   answer). Block 0 also clears the histogram.
//   k_samp_exp      e = expf((l - max) / temp): per-block f64 sums and a
//                   histogram of the nonzero e over their top 12 bits
//                   (count, f32 mass). Last block: den = (float) of the f64
//                   sum, and the candidate threshold T: the highest bin
//                   whose mass from the top reaches topp * den by a margin
//                   that covers the histogram's f32 rounding; p >= RN(lower
//                   edge / den) then holds every token of those bins
//                   (division is monotone).
//   k_samp_select   the ids of the tokens with p >= T (a prefix of the
//                   sorted order whatever the ids, so it holds the nucleus
//                   if its mass reaches topp). Last block: if they fit
//                   (<= kCap) they are sorted in LDS (bitonic, by falling p
//                   then id), scanned in f64, and the nucleus and the pick
//                   read off. Otherwise (a flat distribution, or topp close
//                   to 1, where every block has stored p instead) an exact
//                   radix select over all V: four histogram levels over p's
//                   bits with f64 masses (one histogram per wave, then added
//                   in a fixed order) find where the running sum crosses
//                   topp, then u * cum; a count over index order finds the
//                   token among equal p.
//
// Rounding: the reference adds the sorted probabilities one by one in f64;
// here the f64 sums run in another order, which moves a sum by a few units
// of 2^-53 relative, so a pick can differ only when u * cum or topp falls
// that close to a running sum.
#include "mh_internal.h"

namespace mh {
namespace {

constexpr int kSampThreads = 256;
constexpr int kSampBlocks = 256;   // blocks of the first two launches
constexpr int kSelThreads = 1024;  // the select launch and its last block
constexpr int kSelBlocks = 64;
constexpr int kBins = 1024;        // e histogram: bits(e) >> 20, e in [0, 1]
constexpr int kCap = 8192;         // candidates the one-block sort takes
constexpr int kRadixBins = 256;    // bins per radix level (8 bits)

struct MaxIdx {
    float v;
    int i;
};

// The workspace of one sample call (device memory): a fixed head, then p
// (V floats) when the radix select needs it.
struct SampWs {
    uint64_t part[kSampBlocks];   // per-block maxima (MaxIdx as bits)
    double dsum[kSampBlocks];     // per-block f64 sums of e
    unsigned hcnt[kBins];         // nonzero e per bin
    float hmass[kBins];           // their mass (f32: only steers T)
    float mx;                     // the maximum logit
    float den;                    // (float) of the f64 sum of e
    float tp;                     // the candidate threshold T
    int radix;                    // 1: the candidates cannot fit; p is stored
    unsigned done[3];             // last-block counters, one per launch
    unsigned ncand;               // tokens with p >= T
    unsigned pad[56];
    int cand[kCap];               // their ids (the first kCap)
    float p[1];                   // [V] (only when radix)
};
constexpr uint64_t kWsHead = offsetof(SampWs, p);

// device-scope stores and loads of data that other blocks of the same
// launch read (no cache on the way can hold a stale copy)
template <class T>
__device__ __forceinline__ void st_agent(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_agent(const T *p) {
    return __hip_atomic_load((T *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True in the launch's last block to get here. Every thread's stores have
// completed before its block counts itself in; the last block then drops
// what its caches hold (acquire), resets the counter for the next call and
// goes on alone.
__device__ bool last_block(unsigned *done) {
    __shared__ bool s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!s_last) return false;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (threadIdx.x == 0) st_agent(done, 0u);
    return true;
}

// the reference loop's order: a larger value wins, equal values go to the
// lower index, NaN never wins
__device__ __forceinline__ MaxIdx max_of(MaxIdx a, MaxIdx b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ uint64_t pack(MaxIdx m) {
    return (uint64_t)__float_as_uint(m.v) | ((uint64_t)(uint32_t)m.i << 32);
}
__device__ __forceinline__ MaxIdx unpack(uint64_t w) { return MaxIdx{__uint_as_float((uint32_t)w), (int)(w >> 32)}; }

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

// e of one logit: every kernel evaluates this same expression
__device__ __forceinline__ float samp_e(float l, float mx, float temp) { return expf((l - mx) / temp); }

// Scans over the block (all threads get the block total). The f64 scan
// returns the inclusive sum and sets *excl to the exclusive one, computed
// so that a thread's exclusive sum is bit for bit the previous thread's
// inclusive one (the intervals (excl, incl] tile (0, total]).
__device__ double block_scan_f64(double v, double *excl, double *total) {
    __shared__ double ws[kSelThreads / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    const double prev = __shfl_up(v, 1, 64);
    if (lane == 63) ws[w] = v;
    __syncthreads();
    double before = 0, all = 0;
    for (int i = 0; i < nw; ++i) {
        if (i < w) before += ws[i];
        all += ws[i];
    }
    __syncthreads();
    *total = all;
    *excl = lane == 0 ? before : before + prev;
    return before + v;
}
__device__ int block_scan_int(int v, int *total) {
    __shared__ int ws[kSelThreads / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    if (lane == 63) ws[w] = v;
    __syncthreads();
    int before = 0, all = 0;
    for (int i = 0; i < nw; ++i) {
        if (i < w) before += ws[i];
        all += ws[i];
    }
    __syncthreads();
    *total = all;
    return before + v;
}

// ---------------------------------------------------------------- launches

// Per-block maxima of logits[V] (grid-stride); the last block takes the
// maximum, with the reference loop's index-0 rule, and writes the greedy
// answer. Block 0 clears the histogram and the candidate count.
__global__ void __launch_bounds__(kSampThreads) k_samp_max(const float *__restrict__ lg, int V, SampWs *ws,
                                                           int32_t *__restrict__ greedy_out) {
    if (blockIdx.x == 0) {
        for (int b = threadIdx.x; b < kBins; b += kSampThreads) {
            ws->hcnt[b] = 0;
            ws->hmass[b] = 0.f;
        }
        if (threadIdx.x == 0) ws->ncand = 0;
    }
    MaxIdx m{-INFINITY, INT32_MAX};
    for (int i = blockIdx.x * kSampThreads + threadIdx.x; i < V; i += gridDim.x * kSampThreads)
        m = max_of(m, MaxIdx{lg[i], i});
    m = block_max(m);
    if (threadIdx.x == 0) st_agent(&ws->part[blockIdx.x], pack(m));
    if (!last_block(&ws->done[0])) return;
    MaxIdx r{-INFINITY, INT32_MAX};
    for (int b = threadIdx.x; b < (int)gridDim.x; b += kSampThreads) r = max_of(r, unpack(ld_agent(&ws->part[b])));
    r = block_max(r);
    if (__builtin_isnan(lg[0]) || r.i == INT32_MAX) r = MaxIdx{lg[0], 0};
    if (threadIdx.x == 0) {
        ws->mx = r.v;
        if (greedy_out) *greedy_out = r.i;
    }
}

// e, its per-block f64 sums and the e histogram (per block in LDS, then
// added to the global one); the last block: den and the threshold.
__global__ void __launch_bounds__(kSampThreads) k_samp_exp(const float *__restrict__ lg, int V, float temp,
                                                           float topp, SampWs *ws) {
    __shared__ unsigned s_cnt[kBins];
    __shared__ float s_mass[kBins];
    __shared__ double sd[kSampThreads / 64];
    for (int b = threadIdx.x; b < kBins; b += kSampThreads) {
        s_cnt[b] = 0;
        s_mass[b] = 0.f;
    }
    const float mx = ws->mx;
    __syncthreads();
    double s = 0;
    for (int i = blockIdx.x * kSampThreads + threadIdx.x; i < V; i += gridDim.x * kSampThreads) {
        const float e = samp_e(lg[i], mx, temp);
        s += e;
        if (e != 0.f) {
            const int b = min((int)(__float_as_uint(e) >> 20), kBins - 1);   // (NaN: the top bin)
            atomicAdd(&s_cnt[b], 1u);
            atomicAdd(&s_mass[b], e);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) sd[threadIdx.x >> 6] = s;
    __syncthreads();
    for (int b = threadIdx.x; b < kBins; b += kSampThreads) {
        if (s_cnt[b]) {
            atomicAdd(&ws->hcnt[b], s_cnt[b]);
            atomicAdd(&ws->hmass[b], s_mass[b]);
        }
    }
    if (threadIdx.x == 0) {
        double t = 0;
        for (int w = 0; w < kSampThreads / 64; ++w) t += sd[w];
        st_agent(&ws->dsum[blockIdx.x], t);
    }
    if (!last_block(&ws->done[1]) || threadIdx.x >= 64) return;
    // the first wave: den (lane l adds blocks l, l + 64, ... in order, then a
    // butterfly: every lane gets the same bits)
    const int lane = threadIdx.x;
    double d = 0;
    for (int b = lane; b < (int)gridDim.x; b += 64) d += ld_agent(&ws->dsum[b]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) d += __shfl_xor(d, o, 64);
    const float den = (float)d;
    // the threshold: lane l holds bins kBins-1-16l .. falling
    constexpr int kPer = kBins / 64;
    const double target = (double)topp * (double)den * (1.0 + 1e-4);
    double m[kPer];
    unsigned c[kPer];
    double tot = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int b = kBins - 1 - (kPer * lane + j);
        m[j] = (double)ld_agent(&ws->hmass[b]);
        c[j] = ld_agent(&ws->hcnt[b]);
        tot += m[j];
    }
    double incl = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double n = __shfl_up(incl, o, 64);
        if (lane >= o) incl += n;
    }
    double run = incl - tot;
    int hit = -1;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        run += m[j];
        if (hit < 0 && run >= target) hit = kBins - 1 - (kPer * lane + j);
    }
    const unsigned long long any = __ballot(hit >= 0);
    const int B = any ? __shfl(hit, __ffsll((long long)any) - 1, 64) : 0;
    // at least the tokens of bins >= B are candidates (all V if B = 0)
    unsigned n = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) n += kBins - 1 - (kPer * lane + j) >= B ? c[j] : 0u;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) n += __shfl_xor(n, o, 64);
    if (lane == 0) {
        ws->den = den;
        ws->tp = __uint_as_float((uint32_t)B << 20) / den;
        ws->radix = (B == 0 ? V : (int)n) > kCap ? 1 : 0;
    }
}

// ------------------------------------------------------- the select launch

// LDS of the select launch's last block: the sort's keys, ids and running
// sums, or the radix select's per-wave histograms
union SelLds {
    struct {
        float p[kCap];
        int id[kCap];
        double pre[kCap];
    } sort;
    struct {
        unsigned cnt[kSelThreads / 64][kRadixBins];
        double mass[kSelThreads / 64][kRadixBins];
    } hist;
};

// "a comes before b": falling p, equal p by id
__device__ __forceinline__ bool before(float pa, int ia, float pb, int ib) {
    return pa > pb || (pa == pb && ia < ib);
}

struct Probs {   // p of token i: stored (radix) or as the other kernels compute it
    const float *lg, *ps;
    float mx, temp, den;
    __device__ __forceinline__ float operator()(int i) const {
        return ps ? ps[i] : samp_e(lg[i], mx, temp) / den;
    }
};

// Where the running sum of the sorted p first reaches X (> 0): p's bits key
// k*, the tokens before the group of p == k* (above, their mass above_mass),
// the group's size; found is false if the total stays below X (total then
// holds it). Four 8-bit levels over p's 31 bits.
struct Select {
    bool found;
    uint32_t key;
    int above, ties;
    double above_mass, total;
};
__device__ Select radix_select(const Probs &P, int V, double X, SelLds &L) {
    __shared__ int s_b, s_above, s_low, s_ties;
    __shared__ double s_mass, s_total;
    const int t = threadIdx.x, w = t >> 6;
    Select r{false, 0u, 0, 0, 0.0, 0.0};
    uint32_t prefix = 0;
    constexpr int kSh[4] = {23, 15, 7, 0}, kW[4] = {8, 8, 8, 7};
    for (int lv = 0; lv < 4; ++lv) {
        const int sh = kSh[lv], nb = 1 << kW[lv];
        for (int j = t; j < (kSelThreads / 64) * kRadixBins; j += kSelThreads) {
            (&L.hist.cnt[0][0])[j] = 0;
            (&L.hist.mass[0][0])[j] = 0.0;
        }
        if (t == 0) {
            s_b = -1;
            s_low = INT32_MAX;
        }
        __syncthreads();
        for (int i = t; i < V; i += kSelThreads) {
            const float p = P(i);
            const uint32_t k = __float_as_uint(p);
            if (lv == 0 || (k >> (sh + kW[lv])) == prefix) {
                const int b = (int)((k >> sh) & (uint32_t)(nb - 1));
                atomicAdd(&L.hist.cnt[w][b], 1u);
                atomicAdd(&L.hist.mass[w][b], (double)p);
            }
        }
        __syncthreads();
        // thread t < nb takes bin nb-1-t (the waves' copies added in order);
        // the running sums' intervals (lo, hi] tile (above_mass, total], so
        // exactly one bin holds X if any does
        const int b = nb - 1 - t;
        double m = 0;
        int c = 0;
        if (b >= 0) {
            for (int q = 0; q < kSelThreads / 64; ++q) {
                m += L.hist.mass[q][b];
                c += (int)L.hist.cnt[q][b];
            }
        }
        double tot, ex;
        const double in = block_scan_f64(m, &ex, &tot);
        int ctot;
        const int cin = block_scan_int(c, &ctot);
        const double lo = r.above_mass + ex, hi = r.above_mass + in;
        if (b >= 0 && c > 0 && lo < X && X <= hi) {
            s_b = b;
            s_mass = lo;
            s_above = r.above + cin - c;
        }
        if (b >= 0 && c > 0) atomicMin(&s_low, b);
        if (t == 0) s_total = r.above_mass + tot;
        __syncthreads();
        if (s_b < 0 && lv == 0) {   // X beyond the total
            r.total = s_total;
            return r;
        }
        if (s_b < 0 && b == s_low) {
            // X past this prefix's sum by a rounding (its mass at the level
            // above was summed in another order): the prefix's last bin
            s_b = b;
            s_mass = r.above_mass + (tot - m);
            s_above = r.above + ctot - c;
        }
        __syncthreads();
        if (b >= 0 && b == s_b) s_ties = c;
        __syncthreads();
        r.above_mass = s_mass;
        r.above = s_above;
        r.ties = s_ties;
        prefix = (prefix << kW[lv]) | (uint32_t)s_b;
        __syncthreads();
    }
    r.found = true;
    r.key = prefix;
    return r;
}

// The 1-based place j in the group of equal p (= v, `ties` of them) where
// above_mass + j v first reaches X.
__device__ int tie_place(double above_mass, float v, int ties, double X) {
    const double dv = (double)v;
    long long j = (long long)ceil((X - above_mass) / dv);
    j = max(1ll, min((long long)ties, j));
    while (j > 1 && above_mass + (double)(j - 1) * dv >= X) --j;
    while (j < ties && above_mass + (double)j * dv < X) ++j;
    return (int)j;
}

// The id of the (rank + 1)-th token in index order whose p has the bits
// key: each wave counts the matches of its contiguous segment (lanes on
// consecutive tokens), the segment holding the rank is searched again.
__device__ int id_of(const Probs &P, int V, uint32_t key, int rank) {
    __shared__ int s_cnt[kSelThreads / 64];
    __shared__ int s_id;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int nw = kSelThreads / 64;
    const int seg = ((V + nw - 1) / nw + 63) & ~63;
    const int lo = min(w * seg, V), hi = min(lo + seg, V);
    int c = 0;
    for (int i = lo; i < hi; i += 64) c += __popcll(__ballot(i + lane < hi && __float_as_uint(P(i + lane)) == key));
    if (lane == 0) s_cnt[w] = c;
    if (t == 0) s_id = -1;
    __syncthreads();
    int before = 0;
    for (int q = 0; q < w; ++q) before += s_cnt[q];
    if (rank >= before && rank < before + c) {
        int k = rank - before;
        for (int i = lo; i < hi; i += 64) {
            const unsigned long long bal = __ballot(i + lane < hi && __float_as_uint(P(i + lane)) == key);
            const int n = __popcll(bal);
            if (k < n) {
                unsigned long long m = bal;
                for (int j = 0; j < k; ++j) m &= m - 1;   // drop the k lowest matches
                if (lane == 0) s_id = i + (__ffsll((long long)m) - 1);
                break;
            }
            k -= n;
        }
    }
    __syncthreads();
    return s_id;
}

// The last token in the sorted order: the smallest p, the largest id among
// its equals.
__device__ int last_in_order(const Probs &P, int V) {
    __shared__ uint32_t s_key;
    __shared__ int s_id;
    const int t = threadIdx.x;
    if (t == 0) {
        s_key = 0xFFFFFFFFu;
        s_id = -1;
    }
    __syncthreads();
    uint32_t k = 0xFFFFFFFFu;
    for (int i = t; i < V; i += kSelThreads) k = min(k, __float_as_uint(P(i)));
    atomicMin(&s_key, k);
    __syncthreads();
    const uint32_t key = s_key;
    int id = -1;
    for (int i = t; i < V; i += kSelThreads)
        if (__float_as_uint(P(i)) == key) id = i;
    atomicMax(&s_id, id);
    __syncthreads();
    return s_id;
}

// The nucleus and the pick from the sorted candidates in LDS; false if the
// nucleus reaches past them.
__device__ bool pick_sorted(const Probs &P, int cnt, int V, float topp, float u, const int *cand, SelLds &L,
                            int32_t *out) {
    __shared__ int s_n, s_pick;
    const int t = threadIdx.x;
    // the candidates, padded to a power of two with entries that sort last
    int N2 = 64;
    while (N2 < cnt) N2 <<= 1;
    for (int i = t; i < N2; i += kSelThreads) {
        const int id = i < cnt ? ld_agent(&cand[i]) : INT32_MAX;
        L.sort.p[i] = i < cnt ? P(id) : -1.f;
        L.sort.id[i] = id;
    }
    __syncthreads();
    for (int k = 2; k <= N2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = t; i < N2; i += kSelThreads) {
                const int x = i ^ j;
                if (x > i) {
                    const float pa = L.sort.p[i], pb = L.sort.p[x];
                    const int ia = L.sort.id[i], ib = L.sort.id[x];
                    const bool swap = (i & k) == 0 ? before(pb, ib, pa, ia) : before(pa, ia, pb, ib);
                    if (swap) {
                        L.sort.p[i] = pb;
                        L.sort.p[x] = pa;
                        L.sort.id[i] = ib;
                        L.sort.id[x] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }
    // running f64 sums: thread t adds its run of C sorted entries in order
    const int C = (cnt + kSelThreads - 1) / kSelThreads;
    const int lo = min(t * C, cnt), hi = min(lo + C, cnt);
    double run = 0;
    for (int i = lo; i < hi; ++i) run += (double)L.sort.p[i];
    double tot, acc;
    (void)block_scan_f64(run, &acc, &tot);
    for (int i = lo; i < hi; ++i) {
        acc += (double)L.sort.p[i];
        L.sort.pre[i] = acc;
    }
    if (t == 0) s_n = INT32_MAX;
    __syncthreads();
    for (int i = lo; i < hi; ++i)
        if (L.sort.pre[i] >= (double)topp) {
            atomicMin(&s_n, i + 1);
            break;
        }
    __syncthreads();
    // the nucleus ends inside the list, or the list is the vocabulary
    int n = s_n;
    if (n == INT32_MAX && cnt == V) n = V;
    if (n == INT32_MAX) return false;
    const float r = u * (float)L.sort.pre[n - 1];
    if (t == 0) s_pick = n - 1;
    __syncthreads();
    const int hi2 = min(hi, n);
    for (int i = lo; i < hi2; ++i)
        if ((double)r <= L.sort.pre[i]) {
            atomicMin(&s_pick, i);
            break;
        }
    __syncthreads();
    if (t == 0) *out = L.sort.id[s_pick];
    return true;
}

// The nucleus and the pick over the whole vocabulary (radix select).
__device__ void pick_radix(const Probs &P, int V, float topp, float u, SelLds &L, int32_t *out) {
    const Select sn = radix_select(P, V, (double)topp, L);
    int n, jn = 0;
    double cum;
    if (sn.found) {
        jn = tie_place(sn.above_mass, __uint_as_float(sn.key), sn.ties, (double)topp);
        n = sn.above + jn;
        cum = sn.above_mass + (double)jn * (double)__uint_as_float(sn.key);
    } else {
        n = V;
        cum = sn.total;
    }
    const float r = u * (float)cum;
    int id = -1;
    if (r <= 0.f) {
        // the first token of the order: the largest p, the lowest id
        const Select s0 = radix_select(P, V, 1e-300, L);   // (a target below the largest p)
        id = id_of(P, V, s0.key, 0);
    } else {
        const Select sp = radix_select(P, V, (double)r, L);
        if (sp.found) {
            const int jp = tie_place(sp.above_mass, __uint_as_float(sp.key), sp.ties, (double)r);
            if (sp.above + jp <= n) id = id_of(P, V, sp.key, jp - 1);
        }
        if (id < 0) {   // past the nucleus: its last token
            if (sn.found) id = id_of(P, V, sn.key, jn - 1);
            else id = last_in_order(P, V);
        }
    }
    if (threadIdx.x == 0) *out = id >= 0 ? id : 0;   // (id >= 0: every pass counts the same tokens)
}

// The tokens with p >= T into the candidate list (the first kCap; the count
// goes on), or, when they cannot fit, p of every token into ws->p; then, in
// the last block, the nucleus and the pick.
__global__ void __launch_bounds__(kSelThreads) k_samp_select(const float *__restrict__ lg, int V, float temp,
                                                             float topp, float u, SampWs *ws,
                                                             int32_t *__restrict__ out) {
    __shared__ SelLds L;
    const float mx = ws->mx, den = ws->den, tp = ws->tp;
    const bool radix = ws->radix != 0;
    const int lane = threadIdx.x & 63;
    const int Vr = (V + 63) & ~63;   // whole waves take part in the ballots
    for (int i = blockIdx.x * kSelThreads + threadIdx.x; i < Vr; i += gridDim.x * kSelThreads) {
        const float p = i < V ? samp_e(lg[i], mx, temp) / den : 0.f;
        if (radix) {
            if (i < V) st_agent(&ws->p[i], p);
            continue;
        }
        const bool in = i < V && p >= tp;
        const unsigned long long bal = __ballot(in);
        if (!bal) continue;
        unsigned base = 0;
        const int lead = __ffsll((long long)bal) - 1;
        if (lane == lead) base = atomicAdd(&ws->ncand, (unsigned)__popcll(bal));
        base = __shfl(base, lead, 64);
        const unsigned pos = base + (unsigned)__popcll(bal & ((1ull << lane) - 1));
        if (in && pos < kCap) st_agent(&ws->cand[pos], i);
    }
    if (!last_block(&ws->done[2])) return;
    const int cnt = (int)ld_agent(&ws->ncand);
    if (!radix && cnt <= kCap) {
        const Probs P{lg, nullptr, mx, temp, den};
        if (pick_sorted(P, cnt, V, topp, u, ws->cand, L, out)) return;
        __syncthreads();
        pick_radix(P, V, topp, u, L, out);   // (the histogram fell short: recomputed p)
        return;
    }
    const Probs P{lg, radix ? ws->p : nullptr, mx, temp, den};
    pick_radix(P, V, topp, u, L, out);
}

// zeroes the workspace head (counters, histogram) of a fresh workspace
__global__ void k_samp_clear(uint32_t *w, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) w[i] = 0u;
}

// The library-owned workspace, its head zeroed whenever the slot is
// (re)allocated (a fill kernel, so that a caller's graph capture records no
// memset node).
int sample_scratch(uint64_t bytes, void **ws) {
    static void *cleared = nullptr;
    MH_TRY(scratch(S_SAMPLE, bytes, ws));
    if (*ws != cleared) {
        MH_LAUNCH("sample_clear", k_samp_clear, dim3(8), dim3(256), 0, stream(), (uint32_t *)*ws, (int)(kWsHead / 4));
        MH_TRY(hip_check(hipGetLastError(), "sample workspace clear"));
        cleared = *ws;
    }
    return MH_OK;
}

}  // namespace

// Workspace bytes of a sample call over V tokens.
uint64_t sample_ws_bytes(int64_t V) { return kWsHead + (uint64_t)V * 4; }

// The sampling launches on workspace ws (device, sample_ws_bytes(V) bytes;
// its last-block counters must be zero, as a fill to zero leaves them and
// every call leaves them). `prof` lets profiling bracket the launches with
// events (the allocation-free entry point passes false: event creation is
// not for it).
int sample_launch(const float *logits, int V, float temp, float topp, float u, void *ws_dev, int32_t *out,
                  hipStream_t s, bool prof) {
    SampWs *ws = (SampWs *)ws_dev;
    const bool greedy = temp <= 0.f;
#define SAMP_LAUNCH(name, kernel, grid, block, ...)                                  \
    do {                                                                             \
        if (prof) MH_LAUNCH(name, kernel, grid, block, 0, s, __VA_ARGS__);           \
        else hipLaunchKernelGGL(kernel, grid, block, 0, s, __VA_ARGS__);             \
    } while (0)
    SAMP_LAUNCH("sample_max", k_samp_max, dim3(kSampBlocks), dim3(kSampThreads), logits, V, ws,
                greedy ? out : nullptr);
    if (greedy) return hip_check(hipGetLastError(), "sample launch");
    SAMP_LAUNCH("sample_exp", k_samp_exp, dim3(kSampBlocks), dim3(kSampThreads), logits, V, temp, topp, ws);
    SAMP_LAUNCH("sample_select", k_samp_select, dim3(kSelBlocks), dim3(kSelThreads), logits, V, temp, topp, u, ws,
                out);
#undef SAMP_LAUNCH
    return hip_check(hipGetLastError(), "sample launch");
}

// ------------------------------------------ the fixed, allocation-free workspace

// Vocabularies up to 2^18 tokens (gpt-oss: 201088) fit the fixed workspace:
// about 1.05 MB of device memory per GPU, held until the process ends.
constexpr int64_t kStaticMaxV = 1 << 18;
static __device__ __align__(256) uint8_t samp_static_ws[kWsHead + kStaticMaxV * 4];

// The array's device address on each GPU (its host-side name is no device
// address), looked up once per device at initialisation.
constexpr int kMaxDevices = 64;
static void *g_static_ws[kMaxDevices];

int sample_static_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(MH_E_ARG, "device %d beyond the static workspace table", device);
    void *p = nullptr;
    MH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(samp_static_ws)));
    if (!p) return fail(MH_E_HIP, "hipGetSymbolAddress gave no address for the sampling workspace");
    // counters and histogram start at zero (a fill kernel: no memset node)
    hipLaunchKernelGGL(k_samp_clear, dim3(8), dim3(256), 0, stream(), (uint32_t *)p, (int)(kWsHead / 4));
    MH_HIP(hipGetLastError());
    g_static_ws[device] = p;
    return MH_OK;
}

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
    void *ws;
    MH_TRY(sample_scratch(sample_ws_bytes(V), &ws));
    return sample_launch(logits, (int)V, temp, topp, u, ws, out, stream(), true);
}

int mh_sample_dev_static(const float *logits, int64_t V, float temp, float topp, float u, int32_t *out) {
    clear_error();
    if (!logits || !out) return fail(MH_E_ARG, "mh_sample_dev_static: NULL logits or out");
    if (V < 1 || V > kStaticMaxV)
        return fail(MH_E_ARG, "mh_sample_dev_static: vocabulary %lld outside 1..%lld (the fixed workspace's limit)",
                    (long long)V, (long long)kStaticMaxV);
    MH_TRY(require_init());
    MH_TRY(resolve_dev(logits, (uint64_t)V * 4, "mh_sample_dev_static logits"));
    MH_TRY(resolve_dev(out, 4, "mh_sample_dev_static out"));
    const int dev = current_device();
    void *ws = dev >= 0 && dev < kMaxDevices ? g_static_ws[dev] : nullptr;
    if (!ws) return fail(MH_E_NOINIT, "mh_sample_dev_static: no workspace address for device %d", dev);
    return sample_launch(logits, (int)V, temp, topp, u, ws, out, stream(), false);
}

}  // extern "C"
