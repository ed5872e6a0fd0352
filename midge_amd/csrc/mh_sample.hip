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
//                   answer). Block 0 also clears the candidate counts.
//   k_samp_topp     every block: e = expf((l - max) / temp) of its tokens,
//                   their f64 sum, a histogram of e over its top 12 bits
//                   from 2^-40 up (count, f32 mass; stored per block), and
//                   the ids of its tokens with e >= tc = (1 - topp) / 2V,
//                   appended to the fast list. The last block: den =
//                   (float) of the f64 sum, then the fast path over the
//                   list (every token left out has p at most the list's
//                   smallest, so the list above that p is the head of the
//                   whole order; since den >= 1 and the tokens left out
//                   carry at most half of 1 - topp, it usually holds the
//                   nucleus):
//       <= 64 tokens  one wave: ranked with cross-lane reads, and the
//                     reference's own loops (the f64 running sum in order,
//                     the nucleus, the draw) in one lane;
//       <= kCapF      the block: a histogram of the list's p cuts it to the
//                     bins whose mass reaches topp, which are sorted in LDS.
//                   Taken when the nucleus ends above the list's smallest p.
//   k_samp_select   nothing if the fast path picked. Otherwise every block
//                   finds the candidate threshold T from the stored
//                   histograms (the highest bin whose mass from the top
//                   reaches topp * den by a margin that covers the f32
//                   rounding; p >= RN(lower edge / den) holds every token of
//                   those bins, division being monotone) and gathers its
//                   tokens with p >= T. Last block: if they fit (<= kCap)
//                   they are sorted in LDS (bitonic, by falling p then id),
//                   scanned in f64, and the nucleus and the pick read off.
//                   Otherwise (a flat distribution, or topp close to 1,
//                   where every block has stored p instead) an exact radix
//                   select over all V: four histogram levels over p's bits
//                   with f64 masses (one histogram per wave, then added in a
//                   fixed order) find where the running sum crosses topp,
//                   then u * cum; a count over index order finds the token
//                   among equal p.
//
// Rounding: the reference adds the sorted probabilities one by one in f64;
// so does the one-wave fast path, but elsewhere the f64 sums run in another
// order, which moves a sum by a few units
// of 2^-53 relative, so a pick can differ only when u * cum or topp falls
// that close to a running sum.
#include "mh_internal.h"

namespace mh {
namespace {

constexpr int kSampThreads = 256;
constexpr int kSampBlocks = 256;   // blocks of the max launch
constexpr int kSelThreads = 1024;  // the top-p launch and its last block
constexpr int kSelBlocks = 64;
constexpr int kHLo = 87 << 3;      // e histogram: bins bits(e) >> 20 from 2^-40 (e in [2^-40, 1])
constexpr int kHB = 1024 - kHLo;
constexpr int kCap = 8192;         // candidates the one-block sort takes
constexpr int kCapF = 1024;        // candidates the fast path ranks (one per thread)
constexpr int kRadixBins = 256;    // bins per radix level (8 bits)
constexpr const char *kSampleTimeout = "sampling: a radix-select barrier timed out (blocks not co-resident)";

struct MaxIdx {
    float v;
    int i;
};

// The radix select on the grid: per slot (one level of one select), the
// blocks' histograms summed by device atomics, and the blocks' arrivals.
// Slot 0 is level 0 (the same for every select); the nucleus select's
// levels 1-3 are slots 1-3, the draw's 4-6. The last arrival counter is the
// id search's, with its per-block match counts.
constexpr int kRSlots = 7;
struct SampRadix {
    double hm[kRSlots][kRadixBins];    // mass per bin
    unsigned hc[kRSlots][kRadixBins];  // tokens per bin
    unsigned arrive[kRSlots + 1];
    unsigned gcnt[kSelBlocks];
};

// The workspace of one sample call (device memory): a fixed head, then p
// (V floats) when the radix select needs it.
struct SampWs {
    uint64_t part[kSampBlocks];     // per-block maxima (MaxIdx as bits)
    double dsum[kSelBlocks];        // per-block f64 sums of e
    unsigned bcnt[kSelBlocks][kHB]; // per-block histograms of e: counts
    float bmass[kSelBlocks][kHB];   // and masses (f32: they only steer T)
    float mx;                       // the maximum logit
    float den;                      // (float) of the f64 sum of e
    int fast;                       // 1: the fast path picked (the select launch has nothing to do)
    unsigned done[3];               // last-block counters, one per launch
    unsigned ncand;                 // tokens with e >= tc (the fast list)
    unsigned nsel;                  // tokens with p >= T (the select launch's list)
    unsigned pad[56];
    SampRadix rx;                   // the radix select on the grid (zeroed by the top-p launch)
    int cand[kCap];                 // the fast list (the first kCapF), then the select launch's (the first kCap)
    alignas(16) float p[4];         // [V] (only when radix; 16-byte aligned for the block scans)
};
constexpr uint64_t kWsHead = offsetof(SampWs, p);
static_assert(kWsHead == 225312, "the workspace head size the headers state");

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
// goes on alone. One thread's acquire serves the block: its invalidation
// covers the CU's cache and the L2 that every wave of the block reads
// through, and the block barrier orders the other waves' loads after it
// (an invalidation per wave costs microseconds).
__device__ bool last_block(unsigned *done) {
    __shared__ bool s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
            st_agent(done, 0u);
        }
        s_last = last;
    }
    __syncthreads();
    return s_last;
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
// expf((l - max) / temp) of the reference, the argument formed in f32 as
// there, the exponential correctly rounded (f64 rounded once to f32):
// glibc's expf is within 0.502 ulp, so the two differ only where glibc's own
// result is not the nearest float. (A last-bit difference can reorder two
// tokens of nearly equal p, and with them a draw that falls between.)
__device__ __forceinline__ float samp_e(float l, float mx, float temp) {
    return (float)exp((double)((l - mx) / temp));
}

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
// answer. Block 0 clears the candidate counts.
__global__ void __launch_bounds__(kSampThreads) k_samp_max(const float *__restrict__ lg, int V, SampWs *ws,
                                                           int32_t *__restrict__ greedy_out) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        ws->ncand = 0;
        ws->nsel = 0;
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

// ------------------------------------------------------- the top-p launch

// LDS of the top-p launch's last block: the sort's keys, ids and running
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
    // p from the loaded value (a logit, or p itself when stored)
    __device__ __forceinline__ float of(float v) const { return ps ? v : samp_e(v, mx, temp) / den; }
    __device__ __forceinline__ float operator()(int i) const { return of(ps ? ps[i] : lg[i]); }
};

// f(i, p_i, ok) for every token i of [0, V), by the whole block: four
// tokens per 16-byte load and four loads in flight per thread (a scan by
// one block is bound by its loads in flight). Whole waves take every step
// (ok is false on the padding), so f may use wave-wide operations.
template <class F>
__device__ __forceinline__ void scan_p(const Probs &P, int V, F &&f) {
    const int t = threadIdx.x, lane = t & 63;
    const float *src = P.ps ? P.ps : P.lg;
    const int n4 = ((uintptr_t)src & 15) == 0 ? V >> 2 : 0;
    constexpr int U = 4;
    for (int c0 = t; c0 - lane < n4; c0 += U * kSelThreads) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * kSelThreads;
            v[u] = c < n4 ? ((const float4 *)src)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * kSelThreads;
            const bool ok = c < n4;
            f(4 * c + 0, P.of(v[u].x), ok);
            f(4 * c + 1, P.of(v[u].y), ok);
            f(4 * c + 2, P.of(v[u].z), ok);
            f(4 * c + 3, P.of(v[u].w), ok);
        }
    }
    // the last V mod 4 tokens (every token when the data is not 16-byte aligned)
    for (int i0 = 4 * n4 + t - lane; i0 < V; i0 += kSelThreads) {
        const int i = i0 + lane;
        const bool ok = i < V;
        f(i, ok ? P(i) : 0.f, ok);
    }
}

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
// One level of a radix select from its per-bin sums: thread t holds bin
// bb = nb-1-t's mass m and count c (bb < 0: none). The running sums'
// intervals (lo, hi] from the top tile (above_mass, total], so exactly one
// bin holds X if any does. Appends the bin to *prefix and updates r (the
// tokens above it, their mass, the bin's count); false when X lies beyond
// the total at level 0 (r.total then holds it).
__device__ bool level_choose(double m, int c, int bb, int lv, int kw, double X, Select &r, uint32_t *prefix) {
    __shared__ int s_b, s_above, s_low, s_ties;
    __shared__ double s_mass, s_total;
    if (threadIdx.x == 0) {
        s_b = -1;
        s_low = INT32_MAX;
    }
    double tot, ex;
    const double in = block_scan_f64(m, &ex, &tot);   // (its barriers order the reset above)
    int ctot;
    const int cin = block_scan_int(c, &ctot);
    const double lo = r.above_mass + ex, hi = r.above_mass + in;
    if (bb >= 0 && c > 0 && lo < X && X <= hi) {
        s_b = bb;
        s_mass = lo;
        s_above = r.above + cin - c;
    }
    if (bb >= 0 && c > 0) atomicMin(&s_low, bb);
    if (threadIdx.x == 0) s_total = r.above_mass + tot;
    __syncthreads();
    if (s_b < 0 && lv == 0) {   // X beyond the total
        r.total = s_total;
        __syncthreads();
        return false;
    }
    if (s_b < 0 && bb == s_low) {
        // X past this prefix's sum by a rounding (its mass at the level
        // above was summed in another order): the prefix's last bin
        s_b = bb;
        s_mass = r.above_mass + (tot - m);
        s_above = r.above + ctot - c;
    }
    __syncthreads();
    if (bb >= 0 && bb == s_b) s_ties = c;
    __syncthreads();
    r.above_mass = s_mass;
    r.above = s_above;
    r.ties = s_ties;
    *prefix = (*prefix << kw) | (uint32_t)s_b;
    __syncthreads();
    return true;
}

__device__ Select radix_select(const Probs &P, int V, double X, SelLds &L) {
    const int t = threadIdx.x, w = t >> 6;
    Select r{false, 0u, 0, 0, 0.0, 0.0};
    uint32_t prefix = 0;
    for (int lv = 0; lv < 4; ++lv) {
        // levels of 8, 8, 8 and 7 bits: p's bits 30-23, 22-15, 14-7, 6-0
        const int kw = lv < 3 ? 8 : 7, sh = lv < 3 ? 23 - 8 * lv : 0, nb = 1 << kw;
        for (int j = t; j < (kSelThreads / 64) * kRadixBins; j += kSelThreads) {
            (&L.hist.cnt[0][0])[j] = 0;
            (&L.hist.mass[0][0])[j] = 0.0;
        }
        __syncthreads();
        scan_p(P, V, [&](int, float p, bool ok) {
            const uint32_t k = __float_as_uint(p);
            if (ok && (lv == 0 || (k >> (sh + kw)) == prefix)) {
                const int b = (int)((k >> sh) & (uint32_t)(nb - 1));
                atomicAdd(&L.hist.cnt[w][b], 1u);
                atomicAdd(&L.hist.mass[w][b], (double)p);
            }
        });
        __syncthreads();
        // thread t < nb takes bin nb-1-t (the waves' copies added in order)
        const int b = nb - 1 - t;
        double m = 0;
        int c = 0;
        if (b >= 0) {
            for (int q = 0; q < kSelThreads / 64; ++q) {
                m += L.hist.mass[q][b];
                c += (int)L.hist.cnt[q][b];
            }
        }
        if (!level_choose(m, c, b, lv, kw, X, r, &prefix)) return r;
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
// consecutive tokens, four loads in flight), the segment holding the rank
// is searched again.
__device__ int id_of(const Probs &P, int V, uint32_t key, int rank) {
    __shared__ int s_cnt[kSelThreads / 64];
    __shared__ int s_id;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int nw = kSelThreads / 64, U = 4;
    const int seg = ((V + nw - 1) / nw + 63) & ~63;
    const int lo = min(w * seg, V), hi = min(lo + seg, V);
    int c = 0;
    for (int i = lo; i < hi; i += 64 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = i + 64 * u + lane;
            v[u] = j < hi ? (P.ps ? P.ps[j] : P.lg[j]) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = i + 64 * u + lane;
            c += __popcll(__ballot(j < hi && __float_as_uint(P.of(v[u])) == key));
        }
    }
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
    scan_p(P, V, [&](int, float p, bool ok) {
        if (ok) k = min(k, __float_as_uint(p));
    });
    atomicMin(&s_key, k);
    __syncthreads();
    const uint32_t key = s_key;
    int id = -1;
    scan_p(P, V, [&](int i, float p, bool ok) {
        if (ok && __float_as_uint(p) == key) id = max(id, i);
    });
    atomicMax(&s_id, id);
    __syncthreads();
    return s_id;
}

// The nucleus and the pick from the cnt candidates whose ids are in
// L.sort.id[0, cnt), sorted in LDS by falling p then id: by rank (one
// candidate per thread, a 64-bit key of p's bits above the complement of
// the id, so a larger key comes first; p >= 0) up to kRankMax of them,
// bitonic above. False if the nucleus reaches past the list; with `head`,
// also if it reaches the list's group of its smallest p: the list then
// holds every token of p above that one but maybe not every token of that
// p. have_p: L.sort.p[0, cnt) already holds their p.
constexpr int kRankMax = 128;
__device__ bool pick_sorted(const Probs &P, int cnt, int V, float topp, float u, SelLds &L, int32_t *out,
                            bool head, bool have_p = false) {
    __shared__ int s_n, s_pick, s_m;
    const int t = threadIdx.x;
    if (t == 0) {
        s_n = INT32_MAX;
        s_m = 0;
    }
    if (cnt <= kRankMax) {
        uint64_t *key = (uint64_t *)(L.sort.pre + kCap - kRankMax);   // (clear of pre[0, cnt))
        uint64_t k = 0;
        float p = 0.f;
        int id = 0;
        if (t < cnt) {
            id = L.sort.id[t];
            p = have_p ? L.sort.p[t] : P(id);
            k = ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(~(uint32_t)id);
            key[t] = k;
        }
        __syncthreads();
        int rank = 0;
        if (t < cnt)
            for (int j = 0; j < cnt; ++j) rank += key[j] > k ? 1 : 0;
        __syncthreads();
        if (t < cnt) {
            L.sort.p[rank] = p;
            L.sort.id[rank] = id;
        }
        __syncthreads();
    } else {
        // padded to a power of two with entries that sort last
        int N2 = 64;
        while (N2 < cnt) N2 <<= 1;
        for (int i = t; i < N2; i += kSelThreads) {
            if (i < cnt) {
                if (!have_p) L.sort.p[i] = P(L.sort.id[i]);
            } else {
                L.sort.p[i] = -1.f;
                L.sort.id[i] = INT32_MAX;
            }
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
    }
    // running f64 sums: thread t adds its run of C sorted entries in order
    const int C = (cnt + kSelThreads - 1) / kSelThreads;
    const int lo = min(t * C, cnt), hi = min(lo + C, cnt);
    double run = 0;
    int above = 0;
    const float pmin = L.sort.p[cnt - 1];
    for (int i = lo; i < hi; ++i) {
        run += (double)L.sort.p[i];
        above += L.sort.p[i] > pmin ? 1 : 0;
    }
    if (head && above) atomicAdd(&s_m, above);
    double tot, acc;
    (void)block_scan_f64(run, &acc, &tot);
    for (int i = lo; i < hi; ++i) {
        acc += (double)L.sort.p[i];
        L.sort.pre[i] = acc;
    }
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
    if (head && cnt != V && n > s_m) return false;
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

// ------------------------------------------------ the radix select on the grid
//
// When the nucleus is too wide for the one-block sort, the select launch's
// blocks run the radix select together instead of one block alone. Each
// block takes a contiguous slice of the vocabulary: it stores p of its
// slice, and per level it histograms its slice (per-wave copies added in
// wave order), adds the histogram to the level's slot with device atomics
// and arrives; once every block has arrived, every block reads the slot's
// sums and makes the same choice. Level 0 (no prefix yet) is histogrammed
// as p is stored and serves every select of the call; a later select whose
// prefix at a level equals the nucleus select's reads that select's slot.
// The id of the k-th token of a key in index order: each block counts its
// slice's matches, every block finds the slice that holds the k-th, and
// that block finds the token.
static_assert(kSelBlocks <= 64, "the id search's per-block counts: one lane each");

struct GridSel {
    SampRadix *rx;
    const float *ps;      // the stored p
    unsigned *err;        // raised when an arrival wait times out
    int lo, hi;           // this block's slice
    uint32_t pre0[4];     // the nucleus select's prefix at each level
    int lv0;              // levels whose slot the nucleus select filled
};

// This block's slice [lo, hi) of V tokens (64-token aligned).
__device__ __forceinline__ void slice_of(int V, int *lo, int *hi) {
    const int seg = ((V + (int)gridDim.x - 1) / (int)gridDim.x + 63) & ~63;
    *lo = min((int)blockIdx.x * seg, V);
    *hi = min(*lo + seg, V);
}

// Arrive at counter *cnt once this block's atomics and stores are done, and
// wait (bounded) until every block of the launch has; false in every thread
// of the block if the wait timed out, with *err raised. One thread's acquire
// serves the block, as in last_block.
__device__ bool arrive_wait(unsigned *cnt, unsigned *err) {
    __shared__ int s_ok;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 1;
        unsigned spins = 0;
        while (ld_agent(cnt) < gridDim.x) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > (1u << 20)) {   // ~1 s: the blocks were not co-resident
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                ok = 0;
                break;
            }
        }
        if (ok) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
        }
        s_ok = ok;
    }
    __syncthreads();
    return s_ok != 0;
}

__device__ __forceinline__ void hist_clear(SelLds &L) {
    for (int j = threadIdx.x; j < (kSelThreads / 64) * kRadixBins; j += kSelThreads) {
        (&L.hist.cnt[0][0])[j] = 0;
        (&L.hist.mass[0][0])[j] = 0.0;
    }
}

// The block's histogram (its waves' copies added in wave order) into the
// slot's sums, then the arrival.
__device__ bool hist_publish(GridSel &g, int slot, int nb, SelLds &L) {
    __syncthreads();
    for (int j = threadIdx.x; j < nb; j += kSelThreads) {
        double m = 0;
        unsigned c = 0;
        for (int q = 0; q < kSelThreads / 64; ++q) {
            m += L.hist.mass[q][j];
            c += L.hist.cnt[q][j];
        }
        if (c) {
            unsafeAtomicAdd(&g.rx->hm[slot][j], m);
            __hip_atomic_fetch_add(&g.rx->hc[slot][j], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    return arrive_wait(&g.rx->arrive[slot], g.err);
}

// radix_select over the stored p, by every block of the launch (s: 0 the
// nucleus select, 1 the draw's); every block returns the same Select (ok
// false: a wait timed out). Slot 0 holds level 0 already.
__device__ Select gselect(GridSel &g, int s, double X, SelLds &L, bool *ok) {
    const int t = threadIdx.x, w = t >> 6;
    Select r{false, 0u, 0, 0, 0.0, 0.0};
    uint32_t prefix = 0;
    for (int lv = 0; lv < 4; ++lv) {
        const int kw = lv < 3 ? 8 : 7, sh = lv < 3 ? 23 - 8 * lv : 0, nb = 1 << kw;
        int slot = 0;
        if (lv > 0) {
            if (s > 0 && lv < g.lv0 && prefix == g.pre0[lv]) {
                slot = lv;   // the nucleus select's histogram of the same prefix
            } else {
                slot = 3 * s + lv;
                hist_clear(L);
                __syncthreads();
                for (int i0 = g.lo + t; i0 < g.hi; i0 += 4 * kSelThreads) {
                    float v[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int i = i0 + u * kSelThreads;
                        v[u] = i < g.hi ? g.ps[i] : 0.f;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const uint32_t k = __float_as_uint(v[u]);
                        if (i0 + u * kSelThreads < g.hi && (k >> (sh + kw)) == prefix) {
                            const int b = (int)((k >> sh) & (uint32_t)(nb - 1));
                            atomicAdd(&L.hist.cnt[w][b], 1u);
                            atomicAdd(&L.hist.mass[w][b], (double)v[u]);
                        }
                    }
                }
                if (!hist_publish(g, slot, nb, L)) {
                    *ok = false;
                    return r;
                }
            }
        }
        if (s == 0) {
            g.pre0[lv] = prefix;
            g.lv0 = lv + 1;
        }
        // thread t takes bin nb-1-t of the slot
        const int bb = nb - 1 - t;
        double m = 0;
        int c = 0;
        if (bb >= 0) {
            m = ld_agent(&g.rx->hm[slot][bb]);
            c = (int)ld_agent(&g.rx->hc[slot][bb]);
        }
        if (!level_choose(m, c, bb, lv, kw, X, r, &prefix)) return r;
    }
    r.found = true;
    r.key = prefix;
    return r;
}

// *out = the id of the (rank + 1)-th token in index order whose stored p has
// the bits key, by every block (the block whose slice holds it writes it).
// False if the wait timed out.
__device__ bool gid_of(GridSel &g, uint32_t key, int rank, int32_t *out) {
    __shared__ int s_cnt[kSelThreads / 64];
    __shared__ int s_owner, s_local;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int nw = kSelThreads / 64;
    // the slice in parts of seg2 tokens, one per wave
    const int seg2 = ((g.hi - g.lo + nw - 1) / nw + 63) & ~63;
    const int plo = min(g.lo + w * seg2, g.hi), phi = min(plo + seg2, g.hi);
    int cw = 0;
    for (int i = plo; i < phi; i += 64) {
        const int j = i + lane;
        cw += __popcll(__ballot(j < phi && __float_as_uint(g.ps[j]) == key));
    }
    if (lane == 0) s_cnt[w] = cw;
    __syncthreads();
    if (t == 0) {
        int n = 0;
        for (int q = 0; q < nw; ++q) n += s_cnt[q];
        st_agent(&g.rx->gcnt[blockIdx.x], (unsigned)n);
    }
    if (!arrive_wait(&g.rx->arrive[kRSlots], g.err)) return false;
    if (w == 0) {
        // lane q holds block q's count: the block where the running count passes rank
        const int n = lane < (int)gridDim.x ? (int)ld_agent(&g.rx->gcnt[lane]) : 0;
        int incl = n;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        const unsigned long long past = __ballot(incl > rank);
        if (lane == 0) s_owner = past ? __ffsll((long long)past) - 1 : -1;
        const int owner = past ? __ffsll((long long)past) - 1 : -1;
        if (owner >= 0 && lane == owner) s_local = rank - (incl - n);
    }
    __syncthreads();
    if (s_owner < 0) {   // (never: every pass counts the same tokens)
        if (blockIdx.x == 0 && t == 0) *out = 0;
        return true;
    }
    if ((int)blockIdx.x != s_owner) return true;
    int before = 0;
    for (int q = 0; q < w; ++q) before += s_cnt[q];
    const int k0 = s_local;
    if (k0 >= before && k0 < before + cw) {
        int k = k0 - before;
        for (int i = plo; i < phi; i += 64) {
            const unsigned long long bal = __ballot(i + lane < phi && __float_as_uint(g.ps[i + lane]) == key);
            const int n = __popcll(bal);
            if (k < n) {
                unsigned long long m = bal;
                for (int j = 0; j < k; ++j) m &= m - 1;   // drop the k lowest matches
                if (lane == 0) *out = i + (__ffsll((long long)m) - 1);
                break;
            }
            k -= n;
        }
    }
    return true;
}

// pick_radix by every block of the launch: p of this block's slice stored
// with its level-0 histogram, then the selects.
__device__ void gpick_radix(const Probs &P0, int V, float topp, float u, SelLds &L, SampWs *ws, unsigned *err,
                            int32_t *out) {
    const int t = threadIdx.x, w = t >> 6;
    GridSel g;
    g.rx = &ws->rx;
    g.ps = ws->p;
    g.err = err;
    g.lv0 = 0;
    slice_of(V, &g.lo, &g.hi);
    hist_clear(L);
    __syncthreads();
    for (int i0 = g.lo + t; i0 < g.hi; i0 += 4 * kSelThreads) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = i0 + q * kSelThreads;
            v[q] = i < g.hi ? P0.lg[i] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = i0 + q * kSelThreads;
            if (i < g.hi) {
                const float p = P0.of(v[q]);
                ws->p[i] = p;
                const int b = (int)((__float_as_uint(p) >> 23) & (kRadixBins - 1));
                atomicAdd(&L.hist.cnt[w][b], 1u);
                atomicAdd(&L.hist.mass[w][b], (double)p);
            }
        }
    }
    if (!hist_publish(g, 0, kRadixBins, L)) return;
    const Probs P{P0.lg, ws->p, P0.mx, P0.temp, P0.den};
    bool ok = true;
    const Select sn = gselect(g, 0, (double)topp, L, &ok);
    if (!ok) return;
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
    if (r <= 0.f) {
        // the first token of the order: the largest p, the lowest id
        const Select s0 = gselect(g, 1, 1e-300, L, &ok);   // (a target below the largest p)
        if (ok) (void)gid_of(g, s0.key, 0, out);
        return;
    }
    const Select sp = gselect(g, 1, (double)r, L, &ok);
    if (!ok) return;
    if (sp.found) {
        const int jp = tie_place(sp.above_mass, __uint_as_float(sp.key), sp.ties, (double)r);
        if (sp.above + jp <= n) {
            (void)gid_of(g, sp.key, jp - 1, out);
            return;
        }
    }
    // past the nucleus: its last token
    if (sn.found) {
        (void)gid_of(g, sn.key, jn - 1, out);
        return;
    }
    if (blockIdx.x == 0) {   // (a total below topp by a rounding: the order's last token; block 0 alone)
        const int id = last_in_order(P, V);
        if (t == 0) *out = id >= 0 ? id : 0;
    }
}

// The fast candidates' threshold: tokens with e >= tc go on the fast list.
// Any tc gives exact picks (the fast path checks that what it orders is a
// head of the whole order and holds the nucleus); with tc = (1 - topp) / 2V
// the tokens left out carry less than (1 - topp) / 2 of den (den >= 1: the
// maximum's e is 1), so the list usually holds the nucleus.
__device__ __forceinline__ float fast_tc(float topp, int V) { return (1.f - topp) / (2.f * (float)V); }

// The fast path, in the top-p launch's last block: the cnt (<= kCapF)
// tokens of the fast list, one per thread (its id and logit lv). Every token left out of the list
// has p at most the list's smallest, pmin (its e is below every listed e).
// A histogram of the list's p over their top 10 bits (f64 masses) gives the
// highest bin edge from which the listed mass reaches topp; the tokens at
// or above that edge are ordered. If the edge is above pmin they are every
// token of p >= edge, a head of the whole order closed under equal p;
// otherwise they are the whole list, whose order is exact above pmin.
// False (nothing written) if the nucleus is not inside what was ordered.
__device__ bool pick_fast(const Probs &P, int cnt, int V, float topp, float u, int id, float lv, SelLds &L,
                          int32_t *out) {
    __shared__ double s_lm[256];
    __shared__ int s_hit, s_nf;
    __shared__ uint32_t s_pmin;
    const int t = threadIdx.x, lane = t & 63;
    if (t < 256) s_lm[t] = 0.0;
    if (t == 0) {
        s_hit = INT32_MAX;
        s_nf = 0;
        s_pmin = 0xFFFFFFFFu;
    }
    const float p = t < cnt ? P.of(lv) : 0.f;
    __syncthreads();
    const uint32_t bits = __float_as_uint(p);
    if (t < cnt) {
        atomicAdd(&s_lm[bits >> 22], (double)p);   // (p in [0, 1]: bins 0..254)
        atomicMin(&s_pmin, bits);
    }
    __syncthreads();
    // thread t takes bin 255 - t; the first bin from the top where the
    // listed mass reaches topp (a relative margin far above the f64
    // rounding of these sums)
    const int hb = 255 - t;
    double ex, tot;
    const double in = block_scan_f64(hb >= 0 ? s_lm[hb] : 0.0, &ex, &tot);
    if (hb >= 0 && in >= (double)topp * (1.0 + 1e-12)) atomicMin(&s_hit, t);
    __syncthreads();
    const uint32_t edge = s_hit == INT32_MAX ? 0u : (uint32_t)(255 - s_hit) << 22;
    const bool head = edge <= s_pmin && cnt != V;
    // the listed tokens at or above the edge, gathered in LDS
    const bool keep = t < cnt && bits >= edge;
    const unsigned long long bal = __ballot(keep);
    if (bal) {
        const int lead = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane == lead) base = atomicAdd(&s_nf, __popcll(bal));
        base = __shfl(base, lead, 64);
        if (keep) {
            const int pos = base + __popcll(bal & ((1ull << lane) - 1));
            L.sort.id[pos] = id;
            L.sort.p[pos] = p;
        }
    }
    __syncthreads();
    const int nf = s_nf;
    return pick_sorted(P, nf, V, topp, u, L, out, head, true);
}

// The fast path for a list of at most 64 tokens, in one wave (lane i holds
// entry i: id, logit lv): ranked by falling p then id with cross-lane
// reads, moved to their places, then the reference's own loops over the
// sorted p in one lane (the f64 running sum in order, the nucleus, the
// draw): no block-wide step. As pick_fast, false unless the nucleus ends
// above the list's smallest p (or the list is the vocabulary).
__device__ bool pick_fast_wave(const Probs &P, int cnt, int V, float topp, float u, int id, float lv,
                               int32_t *out) {
    const int lane = threadIdx.x & 63;
    const bool valid = lane < cnt;
    const float p = valid ? P.of(lv) : 0.f;
    // keys: p's bits above the id's complement (>= 2^31); padding lanes get
    // distinct keys below every real one, so the ranks are a permutation
    const uint64_t key = valid ? ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(~(uint32_t)id)
                               : (uint64_t)(63 - lane);
    const uint32_t klo = (uint32_t)key, khi = (uint32_t)(key >> 32);
    int rank = 0;
    for (int j = 0; j < 64; ++j) {
        const uint64_t kj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(khi, j) << 32) |
                            (uint64_t)(uint32_t)__builtin_amdgcn_readlane(klo, j);
        rank += kj > key ? 1 : 0;
    }
    // lane r receives the entry of rank r
    const float sp = __int_as_float(__builtin_amdgcn_ds_permute(rank * 4, __float_as_int(p)));
    const int sid = __builtin_amdgcn_ds_permute(rank * 4, id);
    // the reference's loops (engine/midge.c:669-676), run by every lane on
    // the same values
    double cum = 0;
    int n = 0;
    bool reached = false;
    for (; n < cnt; ++n) {
        cum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(sp), n));
        if (cum >= (double)topp) {
            ++n;
            reached = true;
            break;
        }
    }
    if (!reached && cnt != V) return false;
    if (cnt != V) {
        // the entries above the smallest p are the head of the whole order
        const float pmin = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sp), cnt - 1));
        const int m = __popcll(__ballot(lane < cnt && sp > pmin));
        if (n > m) return false;
    }
    const float r = u * (float)cum;
    double acc = 0;
    int pick = __builtin_amdgcn_readlane(sid, n - 1);
    for (int i = 0; i < n; ++i) {
        acc += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(sp), i));
        if ((double)r <= acc) {
            pick = __builtin_amdgcn_readlane(sid, i);
            break;
        }
    }
    if (lane == 0) *out = pick;
    return true;
}

// The top-p launch (temp > 0). Every block: e of its tokens (grid-stride),
// their f64 sum, its e histogram (stored for the select launch), and its
// fast candidates, gathered in LDS and appended to the fast list with one
// counter add per block. The last block: den, then the fast path.
__global__ void __launch_bounds__(kSelThreads) k_samp_topp(const float *__restrict__ lg, int V, float temp,
                                                           float topp, float u, SampWs *ws,
                                                           int32_t *__restrict__ out) {
    __shared__ SelLds L;
    __shared__ unsigned s_cnt[kHB];
    __shared__ float s_mass[kHB];
    __shared__ double sd[kSelThreads / 64];
    __shared__ float s_den;
    __shared__ int s_n, s_fb;
    __shared__ int s_fid[kCapF];
    const int t = threadIdx.x, lane = t & 63;
    for (int b = t; b < kHB; b += kSelThreads) {
        s_cnt[b] = 0;
        s_mass[b] = 0.f;
    }
    if (t == 0) s_n = 0;
    // the radix select's slots start at zero in every call
    for (int j = blockIdx.x * kSelThreads + t; j < (int)(sizeof(SampRadix) / 4); j += gridDim.x * kSelThreads)
        ((unsigned *)&ws->rx)[j] = 0u;
    const float mx = ws->mx;
    const float tc = fast_tc(topp, V);
    __syncthreads();
    const int Vr = (V + 63) & ~63;   // whole waves take part in the ballots
    double s = 0;
    for (int i = blockIdx.x * kSelThreads + t; i < Vr; i += gridDim.x * kSelThreads) {
        const float e = i < V ? samp_e(lg[i], mx, temp) : 0.f;
        s += e;
        const int hb = (int)(__float_as_uint(e) >> 20);
        if (i < V && hb >= kHLo) {   // e >= 2^-40, or NaN (the top bin)
            const int b = min(hb - kHLo, kHB - 1);
            atomicAdd(&s_cnt[b], 1u);
            atomicAdd(&s_mass[b], e);
        }
        // the block's fast candidates into LDS (the first kCapF; the count goes on)
        const bool in = i < V && e >= tc;
        const unsigned long long bal = __ballot(in);
        if (!bal) continue;
        const int lead = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane == lead) base = atomicAdd(&s_n, __popcll(bal));
        base = __shfl(base, lead, 64);
        const int pos = base + __popcll(bal & ((1ull << lane) - 1));
        if (in && pos < kCapF) s_fid[pos] = i;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) sd[t >> 6] = s;
    __syncthreads();
    // one counter add per block appends them to the fast list
    const int nb = s_n;
    if (t == 0) s_fb = nb ? (int)atomicAdd(&ws->ncand, (unsigned)nb) : 0;
    __syncthreads();
    const int fb = s_fb;
    for (int j = t; j < nb && fb + j < kCapF; j += kSelThreads) st_agent(&ws->cand[fb + j], s_fid[j]);
    for (int b = t; b < kHB; b += kSelThreads) {
        st_agent(&ws->bcnt[blockIdx.x][b], s_cnt[b]);
        st_agent(&ws->bmass[blockIdx.x][b], s_mass[b]);
    }
    if (t == 0) {
        double d = 0;
        for (int w = 0; w < kSelThreads / 64; ++w) d += sd[w];
        st_agent(&ws->dsum[blockIdx.x], d);
    }
    if (!last_block(&ws->done[1])) return;

    // one round of loads: the blocks' sums, the fast list's count and its
    // entries whatever the count (an entry past it may be an earlier call's,
    // so the index is clamped to the vocabulary; it is not used), then the
    // entries' logits
    double d = 0;
    if (t < 64)
        for (int b = t; b < (int)gridDim.x; b += 64) d += ld_agent(&ws->dsum[b]);
    const int cnt = (int)ld_agent(&ws->ncand);
    const int id = t < kCapF ? min(max(ld_agent(&ws->cand[t]), 0), V - 1) : 0;
    const float lv = lg[id];
    // den: lane l adds blocks l, l + 64, ... in order, then a butterfly
    if (t < 64) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) d += __shfl_xor(d, o, 64);
        if (t == 0) s_den = (float)d;
    }
    __syncthreads();
    const float den = s_den;
    const Probs P{lg, nullptr, mx, temp, den};
    const bool ok = den > 0.f && den <= 3.402823466e38f && cnt >= 1;
    if (ok && cnt <= 64) {
        // one wave
        if (t >= 64) return;
        const bool fast = pick_fast_wave(P, cnt, V, topp, u, id, lv, out);
        if (t == 0) {
            ws->den = den;
            ws->fast = fast ? 1 : 0;
        }
        return;
    }
    const bool fast = ok && cnt <= kCapF && pick_fast(P, cnt, V, topp, u, id, lv, L, out);
    if (t == 0) {
        ws->den = den;
        ws->fast = fast ? 1 : 0;
    }
}

// The select launch: nothing when the fast path picked. Otherwise every
// block reads the top-p launch's per-block e histograms (the same sums in
// the same order in every block) and finds the candidate threshold T: the
// highest bin whose mass from the top reaches topp * den by a margin that
// covers the histogram's f32 rounding, T = RN(lower edge / den), so p >= T
// holds every token of those bins (division is monotone). Then, over its
// share of the tokens, the ids with p >= T (gathered in LDS, one counter add
// per block; the first kCap), or, when the candidates cannot fit, p itself.
// The last block: the sort and the pick; or, when the nucleus is too wide
// for the sort, the radix select on the grid.
__global__ void __launch_bounds__(kSelThreads) k_samp_select(const float *__restrict__ lg, int V, float temp,
                                                             float topp, float u, SampWs *ws,
                                                             int32_t *__restrict__ out, unsigned *err) {
    __shared__ SelLds L;
    __shared__ int s_hit, s_n, s_fb;
    if (ws->fast) return;
    const int t = threadIdx.x, lane = t & 63;
    const float mx = ws->mx, den = ws->den;
    const Probs P{lg, nullptr, mx, temp, den};
    // the threshold: thread t takes bin kHB - 1 - t (the blocks' histograms
    // added in block order); eight rows in flight
    const int hb = kHB - 1 - t;
    double m = 0;
    unsigned c = 0;
    if (hb >= 0) {
        const int nq = kSelBlocks;
        for (int q0 = 0; q0 < nq; q0 += 8) {
            float fm[8];
            unsigned fc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                fm[j] = ws->bmass[q0 + j][hb];
                fc[j] = ws->bcnt[q0 + j][hb];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                m += (double)fm[j];
                c += fc[j];
            }
        }
    }
    const double target = (double)topp * (double)den * (1.0 + 1e-4);
    double ex, tot;
    const double in = block_scan_f64(m, &ex, &tot);
    if (t == 0) {
        s_hit = INT32_MAX;
        s_n = 0;
    }
    __syncthreads();
    if (hb >= 0 && in >= target) atomicMin(&s_hit, t);
    __syncthreads();
    const int hit = s_hit;
    int nc;
    (void)block_scan_int(t <= hit ? (int)c : 0, &nc);
    // at least the tokens of the bins from the top through the hit are
    // candidates (every token when no bin reaches the target)
    const float tp = hit == INT32_MAX ? 0.f : __uint_as_float((uint32_t)(kHLo + kHB - 1 - hit) << 20) / den;
    const bool radix = (hit == INT32_MAX ? V : nc) > kCap;
    if (radix) {
        gpick_radix(P, V, topp, u, L, ws, err, out);
        return;
    }
    const int Vr = (V + 63) & ~63;
    for (int i = blockIdx.x * kSelThreads + t; i < Vr; i += gridDim.x * kSelThreads) {
        const float p = i < V ? P(i) : 0.f;
        const bool inc = i < V && p >= tp;
        const unsigned long long bal = __ballot(inc);
        if (!bal) continue;
        const int lead = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane == lead) base = atomicAdd(&s_n, __popcll(bal));
        base = __shfl(base, lead, 64);
        const int pos = base + __popcll(bal & ((1ull << lane) - 1));
        if (inc && pos < kCap) L.sort.id[pos] = i;
    }
    __syncthreads();
    {
        const int nb = s_n;
        if (t == 0) s_fb = nb ? (int)atomicAdd(&ws->nsel, (unsigned)nb) : 0;
        __syncthreads();
        const int fb = s_fb;
        for (int j = t; j < nb && fb + j < kCap; j += kSelThreads) st_agent(&ws->cand[fb + j], L.sort.id[j]);
    }
    if (!last_block(&ws->done[2])) return;
    const int cnt = (int)ld_agent(&ws->nsel);
    if (cnt >= 1 && cnt <= kCap) {
        for (int j = t; j < cnt; j += kSelThreads) L.sort.id[j] = ld_agent(&ws->cand[j]);
        __syncthreads();
        if (pick_sorted(P, cnt, V, topp, u, L, out, false)) return;
        __syncthreads();
    }
    pick_radix(P, V, topp, u, L, out);   // (the histogram fell short: p recomputed, one block)
}

// zeroes the workspace head (counters, histogram) of a fresh workspace
__global__ void k_samp_clear(uint32_t *w, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) w[i] = 0u;
}

// The library-owned workspace, its head zeroed whenever the slot is
// (re)allocated (a fill kernel, so that a caller's graph capture records no
// memset node).
int sample_scratch(uint64_t bytes, void **ws) {
    bool fresh = false;
    MH_TRY(scratch(S_SAMPLE, bytes, ws, &fresh));
    if (fresh) {
        MH_LAUNCH("sample_clear", k_samp_clear, dim3(8), dim3(256), 0, stream(), (uint32_t *)*ws, (int)(kWsHead / 4));
        MH_TRY(hip_check(hipGetLastError(), "sample workspace clear"));
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
    unsigned *err = nullptr;   // (made at initialisation: the static entry point allocates nothing)
    MH_TRY(async_flag(F_SAMPLE, kSampleTimeout, &err));
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
    SAMP_LAUNCH("sample_topp", k_samp_topp, dim3(kSelBlocks), dim3(kSelThreads), logits, V, temp, topp, u, ws, out);
    SAMP_LAUNCH("sample_select", k_samp_select, dim3(kSelBlocks), dim3(kSelThreads), logits, V, temp, topp, u, ws,
                out, err);
#undef SAMP_LAUNCH
    return hip_check(hipGetLastError(), "sample launch");
}

// ------------------------------------------ the fixed, allocation-free workspace

// Vocabularies up to 2^18 tokens (gpt-oss: 201088) fit the fixed workspace:
// 1,273,888 bytes of device memory per GPU (the 225,312-byte head: block
// maxima, f64 sums, two 64 x 328 histograms, counters and 8192 candidates;
// then 2^18 floats of p), held until the process ends.
constexpr int64_t kStaticMaxV = 1 << 18;
static __device__ __align__(256) uint8_t samp_static_ws[kWsHead + kStaticMaxV * 4];

// The array's device address on each GPU (its host-side name is no device
// address), looked up once per device at initialisation.
constexpr int kMaxDevices = 64;
static void *g_static_ws[kMaxDevices];

int sample_static_setup(int device) {
    unsigned *err = nullptr;   // the radix select's error flag, made here so that no call allocates it
    MH_TRY(async_flag(F_SAMPLE, kSampleTimeout, &err));
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
