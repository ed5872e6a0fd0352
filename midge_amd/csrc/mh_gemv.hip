// mh_gemv.hip — dense matvec kernels for the four midge dtypes, the exact
// row dequantizer and RMSNorm, and their C entry points.
//   mh_matvec / mh_matvec_dev   wk_matvec, engine/mkern.h:180-198
//   mh_row / mh_dequant_dev     wk_row, engine/mkern.h:201-236
//   mh_rmsnorm_dev              wk_rmsnorm, engine/mkern.h:238-243
#include "mh_gemv.cuh"

namespace mh {
namespace {

// ---------------------------------------------------------------- GEMV

// Y[b][r] = W[r] . X[b] for rows [blockIdx.x*rpb, +rpb), token b = blockIdx.y.
template <int DT>
__global__ void __launch_bounds__(kGemvThreads)
k_gemv(const uint8_t *__restrict__ W, const void *__restrict__ S, const float *__restrict__ X,
       float *__restrict__ Y, int rows, int cols, int ns, int rpb) {
    constexpr int E = gemv_chunk<DT>::E;
    extern __shared__ float lds[];
    const int C = cols / E;
    float *res = lds;                  // [rpb]
    float *red = lds + rpb;            // [U][ns][C]
    const int b = blockIdx.y;
    const int r0 = blockIdx.x * rpb;
    const int nf = min(rpb, rows - r0);
    const size_t rowbytes = (size_t)C * 16 * gemv_chunk<DT>::W;
    float xr[E];
    load_x<DT>(X + (size_t)b * cols, C, ns, xr);
    const uint16_t *S16 = (const uint16_t *)S;
    block_gemv<DT>(
        [&](int f) {
            int r = r0 + f;
            return RowRef{W + (size_t)r * rowbytes, S16 + (size_t)r * C};
        },
        nf, C, ns, xr, red, res);
    for (int f = threadIdx.x; f < nf; f += blockDim.x) {
        float v = res[f];
        if constexpr (DT == MH_DT_Q8R) v *= ((const float *)S)[r0 + f];
        Y[(size_t)b * rows + r0 + f] = v;
    }
}

// General fallback: one wave per (row, token), element-wise decode. Used for
// shapes the chunked kernel does not cover (odd widths, unaligned views).
template <int DT>
__global__ void __launch_bounds__(256)
k_gemv_rowwave(const uint8_t *__restrict__ W, const void *__restrict__ S, const float *__restrict__ X,
               float *__restrict__ Y, int64_t rows, int64_t cols) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.y;
    if (r >= rows) return;
    const float *x = X + (size_t)b * cols;
    float s = 0.f;
    if constexpr (DT == MH_DT_F32) {
        const float *w = (const float *)W + r * cols;
        for (int64_t c = lane; c < cols; c += 64) s = __builtin_fmaf(w[c], x[c], s);
    } else if constexpr (DT == MH_DT_Q8R) {
        const int8_t *w = (const int8_t *)W + r * cols;
        for (int64_t c = lane; c < cols; c += 64) s = __builtin_fmaf((float)w[c], x[c], s);
    } else {
        // one 32-group per lane-iteration keeps the group scale structure
        const uint8_t *w = W + r * (cols / 2);
        const uint16_t *sc = (const uint16_t *)S + r * (cols / 32);
        for (int64_t g = lane; g < cols / 32; g += 64) {
            float a = 0.f;
            for (int j = 0; j < 16; ++j) {
                uint8_t byte = w[g * 16 + j];
                float lo, hi;
                if constexpr (DT == MH_DT_MXFP4) {
                    mh_v2f v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)byte, 1.0f, 0);
                    lo = v.x;
                    hi = v.y;
                } else {
                    lo = (float)((int)(byte & 15) - 8);
                    hi = (float)((int)(byte >> 4) - 8);
                }
                a = __builtin_fmaf(lo, x[g * 32 + 2 * j], a);
                a = __builtin_fmaf(hi, x[g * 32 + 2 * j + 1], a);
            }
            s = __builtin_fmaf(mh_f16(sc[g]), a, s);
        }
    }
    s = mh_wave_sum(s);
    if (lane == 0) {
        if constexpr (DT == MH_DT_Q8R) s *= ((const float *)S)[r];
        Y[(size_t)b * rows + r] = s;
    }
}

// ------------------------------------------------------------ dequant

// out[i][c] = W[r0+i][c] dequantized, bit-exact with wk_row.
template <int DT>
__global__ void __launch_bounds__(256)
k_dequant(const uint8_t *__restrict__ W, const void *__restrict__ S, float *__restrict__ out,
          int64_t r0, int64_t n, int64_t cols) {
    const int64_t per_row = (DT == MH_DT_MXFP4 || DT == MH_DT_Q4G32) ? cols / 2 : cols;
    const int64_t total = n * per_row;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t ri = i / per_row, k = i - ri * per_row, r = r0 + ri;
        if constexpr (DT == MH_DT_F32) {
            out[ri * cols + k] = ((const float *)W)[r * cols + k];
        } else if constexpr (DT == MH_DT_Q8R) {
            out[ri * cols + k] = (float)((const int8_t *)W)[r * cols + k] * ((const float *)S)[r];
        } else {
            const uint8_t byte = W[r * per_row + k];
            const float sc = mh_f16(((const uint16_t *)S)[r * (cols / 32) + k / 16]);
            float lo, hi;
            if constexpr (DT == MH_DT_MXFP4) {
                mh_v2f v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((uint32_t)byte, 1.0f, 0);
                lo = v.x;
                hi = v.y;
            } else {
                lo = (float)((int)(byte & 15) - 8);
                hi = (float)((int)(byte >> 4) - 8);
            }
            out[ri * cols + 2 * k] = lo * sc;
            out[ri * cols + 2 * k + 1] = hi * sc;
        }
    }
}

// ------------------------------------------------------------ rmsnorm

// out[b] = x[b] * (1 / sqrt(mean(x[b]^2) + eps)) * w, one block per token.
__global__ void __launch_bounds__(1024)
k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ out, int64_t n,
          float eps) {
    __shared__ float part[16];
    const float *xb = x + (size_t)blockIdx.x * n;
    float *ob = out + (size_t)blockIdx.x * n;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s = __builtin_fmaf(xb[i], xb[i], s);
    s = mh_wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float ss = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) ss += part[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) ob[i] = xb[i] * inv * w[i];
}

template <int DT>
int launch_gemv_t(const DevWT &w, const float *x, float *y, int batch, hipStream_t s) {
    constexpr int E = gemv_chunk<DT>::E;
    const int64_t rows = w.rows, cols = w.cols;
    const bool chunked = cols % E == 0 && cols / E <= kGemvThreads && ((uintptr_t)w.data % 16) == 0 &&
                         ((uintptr_t)x % 16) == 0 && rows <= INT32_MAX;
    if (chunked) {
        const int C = (int)(cols / E);
        int ns, nt;
        gemv_shape(C, &ns, &nt);
        // about two blocks per CU across the grid, whole row-steps per block
        int64_t target = (int64_t)device_cus() * 2;
        int64_t rpb = (rows + target - 1) / target;
        rpb = ((rpb + ns - 1) / ns) * ns;
        if (rpb < ns) rpb = ns;
        if (rpb > 4096) rpb = 4096;
        const int64_t nblk = (rows + rpb - 1) / rpb;
        const size_t lds = ((size_t)rpb + gemv_lds_floats(ns, C)) * sizeof(float);
        MH_LAUNCH("gemv", k_gemv<DT>, dim3((unsigned)nblk, (unsigned)batch), dim3(nt), lds, s, w.data,
                           w.scales, x, y, (int)rows, (int)cols, ns, (int)rpb);
    } else {
        MH_LAUNCH("gemv_rowwave", k_gemv_rowwave<DT>, dim3((unsigned)((rows + 3) / 4), (unsigned)batch), dim3(256), 0,
                           s, w.data, w.scales, x, y, rows, cols);
    }
    return hip_check(hipGetLastError(), "gemv launch");
}

template <int DT>
int launch_dequant_t(const DevWT &w, int64_t r0, int64_t n, float *out, hipStream_t s) {
    const int64_t per_row = (DT == MH_DT_MXFP4 || DT == MH_DT_Q4G32) ? w.cols / 2 : w.cols;
    int64_t total = n * per_row;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    if (blocks < 1) blocks = 1;
    MH_LAUNCH("dequant", k_dequant<DT>, dim3((unsigned)blocks), dim3(256), 0, s, w.data, w.scales, out, r0, n,
                       w.cols);
    return hip_check(hipGetLastError(), "dequant launch");
}

}  // namespace

int launch_gemv(const DevWT &w, const float *x, float *y, int batch, hipStream_t s) {
    if (batch < 1 || batch > 65535) return fail(MH_E_ARG, "batch %d out of range [1, 65535]", batch);
    switch (w.dt) {
    case MH_DT_F32: return launch_gemv_t<MH_DT_F32>(w, x, y, batch, s);
    case MH_DT_Q8R: return launch_gemv_t<MH_DT_Q8R>(w, x, y, batch, s);
    case MH_DT_Q4G32: return launch_gemv_t<MH_DT_Q4G32>(w, x, y, batch, s);
    case MH_DT_MXFP4: return launch_gemv_t<MH_DT_MXFP4>(w, x, y, batch, s);
    }
    return fail(MH_E_DTYPE, "unknown dtype %d", w.dt);
}

int launch_rmsnorm(const float *x, const float *w, float *out, int64_t n, float eps, int batch, hipStream_t s) {
    if (n < 1 || batch < 1) return fail(MH_E_ARG, "rmsnorm: n=%lld batch=%d", (long long)n, batch);
    MH_LAUNCH("rmsnorm", k_rmsnorm, dim3((unsigned)batch), dim3(1024), 0, s, x, w, out, n, eps);
    return hip_check(hipGetLastError(), "rmsnorm launch");
}

static int launch_dequant(const DevWT &w, int64_t r0, int64_t n, float *out, hipStream_t s) {
    switch (w.dt) {
    case MH_DT_F32: return launch_dequant_t<MH_DT_F32>(w, r0, n, out, s);
    case MH_DT_Q8R: return launch_dequant_t<MH_DT_Q8R>(w, r0, n, out, s);
    case MH_DT_Q4G32: return launch_dequant_t<MH_DT_Q4G32>(w, r0, n, out, s);
    case MH_DT_MXFP4: return launch_dequant_t<MH_DT_MXFP4>(w, r0, n, out, s);
    }
    return fail(MH_E_DTYPE, "unknown dtype %d", w.dt);
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_matvec(const mh_wt *t, const float *x, float *y) {
    clear_error();
    if (!t) return fail(MH_E_ARG, "mh_matvec: NULL tensor");
    uint64_t db, sb;
    MH_TRY(wt_bytes(t->dt, t->rows, t->cols, &db, &sb));
    if (!x || !y) return fail(MH_E_ARG, "mh_matvec: NULL x or y");
    MH_TRY(require_init());
    DevWT w;
    MH_TRY(resolve_wt(t, &w, "mh_matvec weights"));
    void *dx, *dy;
    MH_TRY(scratch(S_X, (uint64_t)w.cols * 4, &dx));
    MH_TRY(scratch(S_Y, (uint64_t)w.rows * 4, &dy));
    hipStream_t s = stream();
    MH_HIP(hipMemcpyAsync(dx, x, (size_t)w.cols * 4, hipMemcpyHostToDevice, s));
    MH_TRY(launch_gemv(w, (const float *)dx, (float *)dy, 1, s));
    MH_HIP(hipMemcpyAsync(y, dy, (size_t)w.rows * 4, hipMemcpyDeviceToHost, s));
    MH_HIP(hipStreamSynchronize(s));
    return MH_OK;
}

int mh_row(const mh_wt *t, int64_t r, float *out) {
    clear_error();
    if (!t) return fail(MH_E_ARG, "mh_row: NULL tensor");
    uint64_t db, sb;
    MH_TRY(wt_bytes(t->dt, t->rows, t->cols, &db, &sb));
    if (!out) return fail(MH_E_ARG, "mh_row: NULL out");
    if (r < 0 || r >= t->rows) return fail(MH_E_RANGE, "mh_row: row %lld outside [0, %lld)", (long long)r,
                                           (long long)t->rows);
    MH_TRY(require_init());
    DevWT w;
    MH_TRY(resolve_wt(t, &w, "mh_row weights"));
    void *d;
    MH_TRY(scratch(S_Y, (uint64_t)w.cols * 4, &d));
    hipStream_t s = stream();
    MH_TRY(launch_dequant(w, r, 1, (float *)d, s));
    MH_HIP(hipMemcpyAsync(out, d, (size_t)w.cols * 4, hipMemcpyDeviceToHost, s));
    MH_HIP(hipStreamSynchronize(s));
    return MH_OK;
}

int mh_matvec_dev(const mh_wt *t, const float *x, float *y, int batch) {
    clear_error();
    if (!t) return fail(MH_E_ARG, "mh_matvec_dev: NULL tensor");
    uint64_t db, sb;
    MH_TRY(wt_bytes(t->dt, t->rows, t->cols, &db, &sb));
    if (batch < 1) return fail(MH_E_ARG, "mh_matvec_dev: batch %d < 1", batch);
    MH_TRY(require_init());
    DevWT w;
    MH_TRY(resolve_wt(t, &w, "mh_matvec_dev weights"));
    MH_TRY(resolve_dev(x, (uint64_t)batch * w.cols * 4, "mh_matvec_dev x"));
    MH_TRY(resolve_dev(y, (uint64_t)batch * w.rows * 4, "mh_matvec_dev y"));
    return launch_gemv(w, x, y, batch, stream());
}

int mh_dequant_dev(const mh_wt *t, int64_t r0, int64_t n, float *out) {
    clear_error();
    if (!t) return fail(MH_E_ARG, "mh_dequant_dev: NULL tensor");
    uint64_t db, sb;
    MH_TRY(wt_bytes(t->dt, t->rows, t->cols, &db, &sb));
    if (r0 < 0 || n < 0 || r0 + n > t->rows)
        return fail(MH_E_RANGE, "mh_dequant_dev: rows [%lld, %lld) outside [0, %lld)", (long long)r0,
                    (long long)(r0 + n), (long long)t->rows);
    if (n == 0) return MH_OK;
    MH_TRY(require_init());
    DevWT w;
    MH_TRY(resolve_wt(t, &w, "mh_dequant_dev weights"));
    MH_TRY(resolve_dev(out, (uint64_t)n * w.cols * 4, "mh_dequant_dev out"));
    return launch_dequant(w, r0, n, out, stream());
}

int mh_rmsnorm_dev(const float *x, const float *w, float *out, int64_t n, float eps, int batch) {
    clear_error();
    if (n < 1 || batch < 1) return fail(MH_E_ARG, "mh_rmsnorm_dev: n=%lld batch=%d", (long long)n, batch);
    MH_TRY(require_init());
    const void *dw;
    MH_TRY(resolve_dev(x, (uint64_t)n * batch * 4, "mh_rmsnorm_dev x"));
    MH_TRY(resolve_weight(w, (uint64_t)n * 4, &dw, "mh_rmsnorm_dev w"));
    MH_TRY(resolve_dev(out, (uint64_t)n * batch * 4, "mh_rmsnorm_dev out"));
    return launch_rmsnorm(x, (const float *)dw, out, n, eps, batch, stream());
}

}  // extern "C"
