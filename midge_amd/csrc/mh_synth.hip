// mh_synth.hip — seeded synthetic inputs generated in HBM (declared in
// include/midge_hip_synth.h). Every value is a pure function of (key, index)
// using integer arithmetic and explicitly rounded f32 operations, so the CPU
// regenerates any slice bit for bit.
#include "../../include/midge_hip_synth.h"
#include "mh_internal.h"

namespace mh {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t hash64(uint64_t key, uint64_t i) {
    return mix64(key + (i + 1) * 0x9e3779b97f4a7c15ull);
}

__device__ __forceinline__ void fill_bytes(uint8_t *dst, uint64_t n, uint64_t key, uint64_t tid, uint64_t nth) {
    const uint64_t words = n / 8;
    uint64_t *d64 = (uint64_t *)dst;   // callers pass 8-byte aligned blobs
    for (uint64_t i = tid; i < words; i += nth) d64[i] = hash64(key, i);
    for (uint64_t i = words * 8 + tid; i < n; i += nth) dst[i] = (uint8_t)(hash64(key, i >> 3) >> (8 * (i & 7)));
}

__device__ __forceinline__ void fill_scales(uint16_t *dst, uint64_t n, uint64_t key, int emin, uint32_t span,
                                            uint64_t tid, uint64_t nth) {
    for (uint64_t i = tid; i < n; i += nth) {
        const int e = emin + (int)((uint32_t)(hash64(key, i) >> 32) % span);
        dst[i] = (uint16_t)((e + 15) << 10);
    }
}

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i, float c) {
    const uint64_t h = hash64(key, i);
    const int s = (int)(h & 0xffff) + (int)((h >> 16) & 0xffff) + (int)((h >> 32) & 0xffff) + (int)(h >> 48);
    return (float)(s - 131070) * c;
}

__global__ void k_bytes(uint8_t *dst, uint64_t n, uint64_t key) {
    fill_bytes(dst, n, key, (uint64_t)blockIdx.x * blockDim.x + threadIdx.x, (uint64_t)gridDim.x * blockDim.x);
}

__global__ void k_scales(uint16_t *dst, uint64_t n, uint64_t key, int emin, uint32_t span) {
    fill_scales(dst, n, key, emin, span, (uint64_t)blockIdx.x * blockDim.x + threadIdx.x,
                (uint64_t)gridDim.x * blockDim.x);
}

__global__ void k_i8(int8_t *dst, uint64_t n, uint64_t key) {
    const uint64_t nth = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += nth) {
        const uint32_t f = (uint32_t)(hash64(key, i >> 2) >> (16 * (i & 3))) & 0xffffu;
        dst[i] = (int8_t)((int)(f % 255u) - 127);
    }
}

__global__ void k_normal(float *dst, uint64_t n, uint64_t key, float c) {
    const uint64_t nth = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += nth) dst[i] = normal_at(key, i, c);
}

__global__ void k_uniform(float *dst, uint64_t n, uint64_t key, float lo, float c) {
#pragma clang fp contract(off)   // lo + h * c rounded twice, as on the CPU
    const uint64_t nth = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += nth)
        dst[i] = lo + (float)(hash64(key, i) >> 40) * c;
}

struct TableArgs {
    uint8_t *base;
    uint64_t stride;
    uint64_t off[9];
    uint64_t dbytes[3], nscales[3], nbias[3];
    int E;
    uint64_t key;
    int emin;
    uint32_t span;
    float bias_c;
};

// blockIdx.y = (l * E + e) * 3 + m; blockIdx.x strides over the blob.
__global__ void k_table(TableArgs A) {
    const uint64_t lem = blockIdx.y;
    const int m = (int)(lem % 3);
    const uint64_t le = lem / 3;   // l * E + e
    uint8_t *ex = A.base + le * A.stride;
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nth = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t kb = (le * 3 + m) * 3;
    fill_bytes(ex + A.off[3 * m], A.dbytes[m], hash64(A.key, kb + 0), tid, nth);
    if (A.nscales[m])
        fill_scales((uint16_t *)(ex + A.off[3 * m + 1]), A.nscales[m], hash64(A.key, kb + 1), A.emin, A.span, tid,
                    nth);
    float *bias = (float *)(ex + A.off[3 * m + 2]);
    const uint64_t bk = hash64(A.key, kb + 2);
    for (uint64_t i = tid; i < A.nbias[m]; i += nth) bias[i] = normal_at(bk, i, A.bias_c);
}

unsigned grid_for(uint64_t n) {
    uint64_t b = (n + 255) / 256;
    if (b > 8192) b = 8192;
    if (b < 1) b = 1;
    return (unsigned)b;
}

int check_span(int emin, int emax) {
    if (emin > emax || emin < -14 || emax > 15)
        return fail(MH_E_ARG, "synth scales: exponent range [%d, %d] must lie in the f16 normal range [-14, 15]",
                    emin, emax);
    return MH_OK;
}

}  // namespace
}  // namespace mh

using namespace mh;

extern "C" {

int mh_synth_bytes_dev(void *dst, uint64_t n, uint64_t key) {
    clear_error();
    MH_TRY(require_init());
    if (!n) return MH_OK;
    MH_TRY(resolve_dev(dst, n, "synth bytes"));
    if ((uintptr_t)dst % 8) return fail(MH_E_ARG, "synth bytes: destination must be 8-byte aligned");
    MH_LAUNCH("synth", k_bytes, dim3(grid_for(n / 8 + 1)), dim3(256), 0, stream(), (uint8_t *)dst, n, key);
    return hip_check(hipGetLastError(), "synth bytes launch");
}

int mh_synth_scales_dev(uint16_t *dst, uint64_t n, uint64_t key, int emin, int emax) {
    clear_error();
    MH_TRY(check_span(emin, emax));
    MH_TRY(require_init());
    if (!n) return MH_OK;
    MH_TRY(resolve_dev(dst, n * 2, "synth scales"));
    MH_LAUNCH("synth", k_scales, dim3(grid_for(n)), dim3(256), 0, stream(), dst, n, key, emin,
                       (uint32_t)(emax - emin + 1));
    return hip_check(hipGetLastError(), "synth scales launch");
}

int mh_synth_i8_dev(int8_t *dst, uint64_t n, uint64_t key) {
    clear_error();
    MH_TRY(require_init());
    if (!n) return MH_OK;
    MH_TRY(resolve_dev(dst, n, "synth i8"));
    MH_LAUNCH("synth", k_i8, dim3(grid_for(n)), dim3(256), 0, stream(), dst, n, key);
    return hip_check(hipGetLastError(), "synth i8 launch");
}

int mh_synth_normal_dev(float *dst, uint64_t n, uint64_t key, float c) {
    clear_error();
    MH_TRY(require_init());
    if (!n) return MH_OK;
    MH_TRY(resolve_dev(dst, n * 4, "synth normal"));
    MH_LAUNCH("synth", k_normal, dim3(grid_for(n)), dim3(256), 0, stream(), dst, n, key, c);
    return hip_check(hipGetLastError(), "synth normal launch");
}

int mh_synth_uniform_dev(float *dst, uint64_t n, uint64_t key, float lo, float c) {
    clear_error();
    MH_TRY(require_init());
    if (!n) return MH_OK;
    MH_TRY(resolve_dev(dst, n * 4, "synth uniform"));
    MH_LAUNCH("synth", k_uniform, dim3(grid_for(n)), dim3(256), 0, stream(), dst, n, key, lo, c);
    return hip_check(hipGetLastError(), "synth uniform launch");
}

int mh_synth_expert_table_dev(void *base, const mh_moe_layer *shape, int n_layers, uint64_t key, int emin,
                              int emax, float bias_c) {
    clear_error();
    if (!shape || n_layers < 1) return fail(MH_E_ARG, "synth table: NULL shape or n_layers < 1");
    if (shape->expert_dt != MH_DT_MXFP4 && shape->expert_dt != MH_DT_Q4G32)
        return fail(MH_E_DTYPE, "synth table: expert dtype %d is not a 4-bit g32 type", shape->expert_dt);
    MH_TRY(check_span(emin, emax));
    MH_TRY(require_init());
    const uint64_t nle = (uint64_t)n_layers * shape->n_experts;
    if (nle * 3 > 65535) return fail(MH_E_UNSUPPORTED, "synth table: %llu layer-experts > 21845",
                                     (unsigned long long)nle);
    MH_TRY(resolve_dev(base, nle * shape->expert_stride, "synth table base"));
    TableArgs A;
    A.base = (uint8_t *)base;
    A.stride = shape->expert_stride;
    for (int i = 0; i < 9; i++) {
        A.off[i] = shape->off[i];
        if (A.off[i] % 8) return fail(MH_E_ARG, "synth table: off[%d] not 8-byte aligned", i);
    }
    if (A.stride % 8) return fail(MH_E_ARG, "synth table: stride not 8-byte aligned");
    const int64_t rows[3] = {shape->ffn, shape->ffn, shape->hidden}, cols[3] = {shape->hidden, shape->hidden,
                                                                               shape->ffn};
    for (int m = 0; m < 3; m++) {
        uint64_t db, sb;
        MH_TRY(wt_bytes(shape->expert_dt, rows[m], cols[m], &db, &sb));
        A.dbytes[m] = db;
        A.nscales[m] = sb / 2;
        A.nbias[m] = (uint64_t)rows[m];
    }
    A.E = shape->n_experts;
    A.key = key;
    A.emin = emin;
    A.span = (uint32_t)(emax - emin + 1);
    A.bias_c = bias_c;
    MH_LAUNCH("synth_table", k_table, dim3(64, (unsigned)(nle * 3)), dim3(256), 0, stream(), A);
    return hip_check(hipGetLastError(), "synth table launch");
}

}  // extern "C"
