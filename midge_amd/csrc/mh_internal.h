// mh_internal.h — host-side state and helpers shared by libmidge_hip's
// translation units, plus the device-side primitives every kernel uses.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/midge_hip.h"

// ------------------------------------------------------------------ host

namespace mh {

// Record a failure message for mh_last_error() and return `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the last-error message (called on entry by public functions).
void clear_error();

// Returns 0, or records the HIP error and returns MH_E_HIP.
int hip_check(hipError_t e, const char *what);
#define MH_HIP(call)                                              \
    do {                                                          \
        int _rc = ::mh::hip_check((call), #call);                 \
        if (_rc) return _rc;                                      \
    } while (0)
#define MH_TRY(expr)                                              \
    do {                                                          \
        int _rc = (expr);                                         \
        if (_rc) return _rc;                                      \
    } while (0)

bool initialised();
int require_init();
hipStream_t stream();
int device_cus();   // compute units on the current device
int current_device();   // the device mh_init() opened
// Looks up the sampling path's fixed workspace on `device` (current) and
// clears its counters; mh_init() calls it (mh_sample.hip).
int sample_static_setup(int device);

// Pointer resolution. Weights: a host pointer inside a registered region
// (translated) or device memory. Activations (_dev calls): device memory
// only. Both check [p, p+bytes) lies inside one allocation/region.
int resolve_weight(const void *p, uint64_t bytes, const void **dev, const char *what);
int resolve_dev(const void *p, uint64_t bytes, const char *what);

// Device memory counted against MIDGE_HIP_MAX_BYTES (MH_E_NOMEM beyond it);
// dev_release frees it and returns the bytes to the count.
int dev_alloc(void **p, uint64_t bytes, const char *what);
void dev_release(void *p, uint64_t bytes);
// Objects that hold device memory of their own (decode plans) register a
// release callback; mh_shutdown calls it for every object still alive.
void register_owner(void *key, void (*release)(void *));
void unregister_owner(void *key);

// Library-owned device scratch that grows on demand (slot = purpose id).
// Contents are not preserved across growth; *fresh (optional) tells whether
// this call (re)allocated the slot (its contents are then undefined, also
// when the new allocation lands at an address the slot had before).
enum Scratch { S_X = 0, S_Y, S_XB, S_H, S_YE, S_RL, S_SEL, S_W, S_PLAN, S_MISC, S_LIST, S_Q, S_XQ, S_ORD, S_SAMPLE, S_ATTN,
               S_ATTN1, S_CROUTE, S_COUNT };
int scratch(Scratch slot, uint64_t bytes, void **p, bool *fresh = nullptr);

// Host-mapped error flags owned by the runtime, one per purpose: allocated
// (zeroed) and watched by mh_sync on first use after mh_init, freed by
// mh_shutdown. *dev is the device address kernels raise.
enum AsyncFlag { F_ATTN1 = 0, F_PREFILL_SCALE, F_SAMPLE, F_COUNT };
int async_flag(AsyncFlag id, const char *msg, unsigned **dev);

// Path switches for comparisons (tests, benchmarks): read once from the
// environment by mh_init (MIDGE_HIP_<name> set and not "0"), changed at run
// time by mh_set_switch. Off by default.
//   NO_MFMA     batched int8 GEMVs, the prefill and the decode step without
//               the matrix-core kernels
//   NO_FUSED    stack decode / expert apply as per-layer launches
//   ATTN_SPLIT  attention as four launches instead of k_attn1
//   COOP        the one-launch decode step as a cooperative launch
//   Q8_NO_ROWS  long batched int8 GEMVs on the register-operand kernel
//   BATCH_GEMV  decode steps of 2-16 tokens on the per-assignment GEMVs
//               instead of the expert-grouped matrix-core kernels
//   SPLIT_ROUTE a stack decode's layer boundary (combine, norm, router,
//               top-k) as three launches instead of k_combine_route
enum Switch { SW_NO_MFMA = 0, SW_NO_FUSED, SW_ATTN_SPLIT, SW_COOP, SW_Q8_NO_ROWS, SW_BATCH_GEMV, SW_SPLIT_ROUTE, SW_COUNT };
bool sw(Switch s);

// The number of successful mh_init calls so far (never reset): state that a
// function caches per initialisation (kernel attributes) keeps the value it
// was set under and redoes its set-up when it differs.
uint64_t init_epoch();

// Bytes per element class for a tensor view.
int wt_bytes(int dt, int64_t rows, int64_t cols, uint64_t *data_bytes, uint64_t *scale_bytes);

// Resolve a tensor view's data/scales to device pointers after checks.
struct DevWT {
    int dt;
    int64_t rows, cols;
    const uint8_t *data;
    const void *scales;
};
int resolve_wt(const mh_wt *t, DevWT *out, const char *what);

// Launch helpers implemented in mh_gemv.hip / mh_moe.hip.
int launch_gemv(const DevWT &w, const float *x, float *y, int batch, hipStream_t s);
int launch_rmsnorm(const float *x, const float *w, float *out, int64_t n, float eps,
                   int batch, hipStream_t s);

// Asynchronous failures: a kernel sets *flag (host-mapped pinned memory);
// mh_sync() and the entry points that return results in host memory
// (sync_checked) report and clear any raised flag.
void watch_async_error(unsigned *flag, const char *msg);
void unwatch_async_error(unsigned *flag);
// Waits for stream s, then reports (and clears) a raised error flag.
int sync_checked(hipStream_t s);

// A fully resolved MoE layer (device pointers).
struct DevLayer {
    int64_t hidden, ffn;
    int n_experts, top_k;
    float alpha, limit, norm_eps;
    int act_plain, router_norm, expert_dt;
    uint64_t expert_stride;
    uint64_t off[9];
    const uint8_t *experts;
    DevWT router;
    const float *router_b, *mlp_norm;
};
// Shape/layout checks of a layer description (no pointer access, no HIP).
int validate_layer(const mh_moe_layer *L);
int resolve_layer(const mh_moe_layer *L, DevLayer *out);

// Assignments of sel[N] (N = tokens * k) grouped by expert (mh_prefill.hip):
// offs[E + 1] into the list, the token (assignment / k) and the slot
// (assignment) of each list position; in the S_LIST scratch, E <= 4096.
struct ExpertLists {
    int *offs, *list_tok, *slot_of;
};
int launch_expert_lists(const int32_t *sel, int N, int E, int k, ExpertLists *out, hipStream_t s);

// Expert-major prefill with scaled MFMA (mh_prefill.hip): the routed
// experts of n tokens into ye[n * k][hidden] (slot order); the caller adds
// them to x with the prefill combine.
bool prefill_mfma_ok(const DevLayer &L);
int run_expert_major_mfma(const DevLayer &L, int n, const float *xb, const int32_t *sel, float *ye,
                          hipStream_t s);

// One-launch decode step for a whole stack at batch 1 (mh_decode.hip).
struct StepPlan;
int step_plan_create(const DevLayer *layers, int n_layers, StepPlan **out);
void step_plan_destroy(StepPlan *p);
bool step_plan_ok(const StepPlan *p);
// 1 if every MXFP4 scale of the plan's layers is f16-exact (the expert-
// grouped matrix-core kernels may run them).
bool step_plan_few(const StepPlan *p);
// The expert FFN of a decode step of 2-16 tokens on the f16 matrix cores,
// each routed expert's weights read once for its tokens (mh_grouped.hip): h
// from xb, then ye, from the top-k kernel's expert-sorted order.
// grouped_ok: the layer and token count fit.
bool grouped_ok(const DevLayer &L, int n);
int launch_grouped(const DevLayer &L, int n, const int32_t *order, const float *xb, float *h, float *ye,
                   hipStream_t s);
// Runs layers [first, first + n_layers) of a plan in one launch; sel, w and
// usage are indexed from layer `first`. With gxb (then one layer, gsel and
// gw [K]): expert_apply per slot with the routing given, x += w_i
// expert_{sel_i}(gxb) in ascending expert order; MH_E_UNSUPPORTED if the
// expert-group kernel cannot run it.
int step_run(StepPlan *p, const DevLayer *layers, int first, int n_layers, float *x, int32_t *sel, float *w,
             uint32_t *usage, hipStream_t s, const float *gxb = nullptr, const int32_t *gsel = nullptr,
             const float *gw = nullptr);

// Kernel timing (mh_profile_*): while enabled, every launch made through
// MH_LAUNCH is bracketed by HIP events on its stream and accounted under its
// name. Off by default; costs nothing when off.
bool profiling();
void prof_begin(const char *name, hipStream_t s);
void prof_end(hipStream_t s);
void prof_add(const char *name, double ms);   // account a duration measured elsewhere

}  // namespace mh

#define MH_LAUNCH(name, kernel, grid, block, lds, strm, ...)                  \
    do {                                                                    \
        const bool _prof = ::mh::profiling();                               \
        if (_prof) ::mh::prof_begin(name, strm);                            \
        hipLaunchKernelGGL(kernel, grid, block, lds, strm, __VA_ARGS__);    \
        if (_prof) ::mh::prof_end(strm);                                    \
    } while (0)

// ---------------------------------------------------------------- device

typedef float mh_v2f __attribute__((ext_vector_type(2)));
// 16 bytes of packed weights as four dwords (a native vector, so it can be
// loaded with the non-temporal builtin).
typedef uint32_t mh_u4 __attribute__((ext_vector_type(4)));

// Global-address-space views: loads through them are global_load (not flat),
// which the compiler cannot infer for pointers read from device tables.
typedef const uint8_t __attribute__((address_space(1))) *mh_gbytes;
__device__ __forceinline__ mh_gbytes mh_global(const void *p) { return (mh_gbytes)p; }
__device__ __forceinline__ mh_u4 mh_load16(mh_gbytes p) {
    return __builtin_nontemporal_load((const mh_u4 __attribute__((address_space(1))) *)p);
}
// The same through the caches: for lines that several load instructions
// share (a non-temporal line can be fetched again for each of them).
__device__ __forceinline__ mh_u4 mh_load16_cached(mh_gbytes p) {
    return *(const mh_u4 __attribute__((address_space(1))) *)p;
}
__device__ __forceinline__ uint32_t mh_load_u16(mh_gbytes p) {
    return *(const uint16_t __attribute__((address_space(1))) *)p;
}

// binary16 bits -> f32 (exact for every encoding; v_cvt_f32_f16).
__device__ __forceinline__ float mh_f16(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// Dot of one 16-byte MXFP4 chunk (32 E2M1 codes, low nibble = even column)
// with xr[0..31]. The codes are converted exactly by the CDNA4 FP4 converter
// (scale 1.0), accumulated in f32.
__device__ __forceinline__ float mh_dot_mxfp4(mh_u4 q, const float *xr) {
    float a = 0.f, b = 0.f;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        mh_v2f p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0);
        mh_v2f p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1);
        mh_v2f p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2);
        mh_v2f p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3);
        a = __builtin_fmaf(p0.x, xr[8 * d + 0], a);
        b = __builtin_fmaf(p0.y, xr[8 * d + 1], b);
        a = __builtin_fmaf(p1.x, xr[8 * d + 2], a);
        b = __builtin_fmaf(p1.y, xr[8 * d + 3], b);
        a = __builtin_fmaf(p2.x, xr[8 * d + 4], a);
        b = __builtin_fmaf(p2.y, xr[8 * d + 5], b);
        a = __builtin_fmaf(p3.x, xr[8 * d + 6], a);
        b = __builtin_fmaf(p3.y, xr[8 * d + 7], b);
    }
    return a + b;
}

// Dot of one 16-byte q4g32 chunk ((nibble - 8), low nibble = even column).
__device__ __forceinline__ float mh_dot_q4(mh_u4 q, const float *xr) {
    float a = 0.f, b = 0.f;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float lo = (float)((int)((w[d] >> (8 * j)) & 15u) - 8);
            float hi = (float)((int)((w[d] >> (8 * j + 4)) & 15u) - 8);
            a = __builtin_fmaf(lo, xr[8 * d + 2 * j], a);
            b = __builtin_fmaf(hi, xr[8 * d + 2 * j + 1], b);
        }
    }
    return a + b;
}

// Dot of one 16-byte int8 chunk (16 weights) with xr[0..15].
__device__ __forceinline__ float mh_dot_i8(mh_u4 q, const float *xr) {
    float a = 0.f, b = 0.f;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            a = __builtin_fmaf((float)(int8_t)(w[d] >> (8 * j)), xr[4 * d + j], a);
            b = __builtin_fmaf((float)(int8_t)(w[d] >> (8 * j + 8)), xr[4 * d + j + 1], b);
        }
    }
    return a + b;
}

// Dot of one 16-byte f32 chunk (4 weights).
__device__ __forceinline__ float mh_dot_f32(mh_u4 q, const float *xr) {
    float a = __builtin_fmaf(__uint_as_float(q.x), xr[0], __uint_as_float(q.y) * xr[1]);
    float b = __builtin_fmaf(__uint_as_float(q.z), xr[2], __uint_as_float(q.w) * xr[3]);
    return a + b;
}

// Elements per 16-byte chunk, per dtype.
template <int DT> struct mh_chunk;
template <> struct mh_chunk<MH_DT_F32> { static constexpr int E = 4; };
template <> struct mh_chunk<MH_DT_Q8R> { static constexpr int E = 16; };
template <> struct mh_chunk<MH_DT_Q4G32> { static constexpr int E = 32; };
template <> struct mh_chunk<MH_DT_MXFP4> { static constexpr int E = 32; };

template <int DT>
__device__ __forceinline__ float mh_dot_chunk(mh_u4 q, const float *xr) {
    if constexpr (DT == MH_DT_MXFP4) return mh_dot_mxfp4(q, xr);
    else if constexpr (DT == MH_DT_Q4G32) return mh_dot_q4(q, xr);
    else if constexpr (DT == MH_DT_Q8R) return mh_dot_i8(q, xr);
    else return mh_dot_f32(q, xr);
}

// Wave64 sum (all lanes get the result).
__device__ __forceinline__ float mh_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// DPP lane exchanges (no LDS). A source lane outside the row mask, or past
// the row for a shift, leaves the destination's own value (update_dpp's
// `old` operand is the value itself) unless noted.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_keep(int x) {
    return __builtin_amdgcn_update_dpp(x, x, CTRL, ROW_MASK, 0xF, false);
}
// v of lane + K within the lane's row of 16 (0 past the row's end)
template <int K>
__device__ __forceinline__ float dpp_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + K, 0xF, 0xF, false));
}
// v of lane ^ 1, lane ^ 2 (quad permutations: every lane has a source)
__device__ __forceinline__ float dpp_x1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_x2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// Maximum / minimum over the wave, returned to every lane: quad
// permutations, half-row and row mirrors, then the row broadcasts (lane 63
// ends with the wave's), then lane 63 read out.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    return fmaxf(v, __int_as_float(dpp_keep<CTRL, ROW_MASK>(__float_as_int(v))));
}
__device__ __forceinline__ float wave_max(float v) {
    v = dpp_max_step<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v);   // row_mirror
    v = dpp_max_step<0x142, 0xA>(v);   // row_bcast:15
    v = dpp_max_step<0x143, 0xC>(v);   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_min_step(int v) {
    return min(v, dpp_keep<CTRL, ROW_MASK>(v));
}
__device__ __forceinline__ int wave_min(int v) {
    v = dpp_min_step<0xB1, 0xF>(v);
    v = dpp_min_step<0x4E, 0xF>(v);
    v = dpp_min_step<0x141, 0xF>(v);
    v = dpp_min_step<0x140, 0xF>(v);
    v = dpp_min_step<0x142, 0xA>(v);
    v = dpp_min_step<0x143, 0xC>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// Sum over the wave with DPP (every lane gets lane 63's total): within rows
// of 16, then the row broadcasts; rows a step does not write add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add_step(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add_step<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_add_step<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_add_step<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_add_step<0x140, 0xF>(v);   // row_mirror
    v = dpp_add_step<0x142, 0xA>(v);   // row_bcast:15
    v = dpp_add_step<0x143, 0xC>(v);   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
