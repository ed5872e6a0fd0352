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
    const uint32_t rowbytes = (uint32_t)C * 16u * gemv_chunk<DT>::W;
    float xr[E];
    load_x<DT>(X + (size_t)b * cols, C, ns, xr);
    const mh_rsrc rd = gemv_rsrc(W + (size_t)r0 * rowbytes, (uint32_t)nf * rowbytes);
    const mh_rsrc rs = gemv_rsrc((const uint16_t *)S + (size_t)r0 * C, (uint32_t)nf * (uint32_t)C * 2u);
    block_gemv<DT>(
        rd, rs, [&](int f) { return RowOff{mul24((uint32_t)f, rowbytes), mul24((uint32_t)f, 2u * C)}; },
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

// ------------------------------------------- batched int8 on the matrix cores
//
// Y[b] = diag(S) W X[b] for a batch of columns, reading each weight byte
// once per 32 columns (the per-column GEMV above reads W once per column).
// Each column of X is written as a 22-bit fixed-point number under a
// power-of-two scale, x = 2^sh * (65536 d0 + 256 d1 + d2), with balanced
// int8 digits d0, d1, d2 (|d0| <= 65). The int8 weights then meet the digits
// on v_mfma_i32_16x16x64_i8, whose int32 sums are exact, and the three sums
// are combined in f32: y = S * 2^sh * (65536 A0 + (256 A1 + A2)). The only
// rounding of x is to 2^-22 of the column's largest magnitude (relative
// error of a dot product ~1e-7, against the f32 sequential sum of mv_q8r,
// engine/mkern.h:23-31, which rounds at every step).

constexpr int kQ8Cols = 32;            // columns per group: NT 16-column tiles
constexpr int kQ8MaxK = 65536;         // |A0| <= 127 * 65 * K stays below 2^31
constexpr int kQ8NonFinite = -100000;  // shift marking a column with inf/nan

typedef int mh_i4 __attribute__((ext_vector_type(4)));

// Digits of column c = 32 * blockIdx.x + blockIdx.y, laid out as the B
// operand of the MFMA: word (group, kc, digit, n, lane) holds, for lane
// l = 16 kg + cn, the digits of column 32 group + 16 n + cn at k = 64 kc +
// 16 kg .. +15. Columns past `batch` get zero digits.
template <int NT>
__global__ void __launch_bounds__(256)
k_xdigits(const float *__restrict__ X, int K, int batch, uint8_t *__restrict__ xq, int *__restrict__ shift) {
    __shared__ float part[4];
    const int grp = blockIdx.x, cl = blockIdx.y, c = grp * kQ8Cols + cl;
    const int n = cl >> 4, cn = cl & 15, KC = K >> 6;
    const bool live = c < batch;
    const float *x = X + (size_t)(live ? c : 0) * K;
    float m = 0.f;
    if (live)
        for (int k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(x[k]));
    bool bad = false;
    if (live)
        for (int k = threadIdx.x; k < K; k += blockDim.x) bad |= !__builtin_isfinite(x[k]);
    m = __builtin_isfinite(m) ? m : __builtin_inff();
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const bool anybad = __syncthreads_or(bad);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    int e = 0;
    if (m > 0.f && !anybad) (void)frexpf(m, &e);   // 2^(e-1) <= m < 2^e
    if (threadIdx.x == 0) shift[c] = anybad ? kQ8NonFinite : e - 22;
    for (int p = threadIdx.x; p < KC * 4; p += blockDim.x) {
        const int kc = p >> 2, kg = p & 3;
        uint32_t dw[3][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int q = 0;
                if (live && !anybad) q = (int)rintf(ldexpf(x[p * 16 + 4 * j + i], 22 - e));   // |q| <= 2^22
                const int d2 = ((q + 128) & 255) - 128;
                const int q1 = (q - d2) >> 8;
                const int d1 = ((q1 + 128) & 255) - 128;
                const int d0 = (q1 - d1) >> 8;
                b0 |= (uint32_t)(d0 & 255) << (8 * i);
                b1 |= (uint32_t)(d1 & 255) << (8 * i);
                b2 |= (uint32_t)(d2 & 255) << (8 * i);
            }
            dw[0][j] = b0;
            dw[1][j] = b1;
            dw[2][j] = b2;
        }
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            const size_t word = ((((size_t)grp * KC + kc) * 3 + d) * NT + n) * 64 + kg * 16 + cn;
            *(mh_u4 *)(xq + word * 16) = mh_u4{dw[d][0], dw[d][1], dw[d][2], dw[d][3]};
        }
    }
}

// Tile shapes of the batched kernel: a wave owns MT 16-row tiles; a block is
// RW row-waves times S waves that split K between them (chunks s, s + S, ...
// of wave s), their int32 sums added in LDS (exact in any order). Weights
// are loaded DA 64-wide chunks ahead of the matrix instructions.
template <int MT_, int RW_, int S_, int DA_>
struct Q8Tile {
    static constexpr int MT = MT_, RW = RW_, S = S_, DA = DA_;
    static constexpr int threads = 64 * RW * S;
    static constexpr int rows = 16 * MT * RW;   // rows per block
};
using Q8Long = Q8Tile<4, 4, 1, 2>;    // long matrices: all of K per wave, equal row shares
using Q8Short = Q8Tile<1, 1, 8, 3>;   // short ones: 16 rows per block, K split 8 ways

// A wave computes rows 16 MT at a time as MT 16-row tiles, the columns of
// group blockIdx.y as NT 16-column tiles, three digits each: MT * NT * 3
// int32 accumulator tiles. Weight tile m, lane l = 16 g + i holds row r0 +
// 16 m + i at k = 64 kc + 16 g .. +15, the same k as the digit word of lane l,
// so every product pairs equal k. Each step issues the digit loads (L2 hits,
// one chunk ahead) before the weight loads (DA chunks ahead): loads complete
// in issue order, so waiting for a step's digits does not wait for younger
// weights. With S = 1 the grid is sized to the machine and each wave takes an
// equal contiguous share of the rows (no tail of partly filled rounds); with
// S > 1 a block owns 16 MT RW rows. Rows past a wave's share re-read its last
// row and are not stored.
template <int NT, class T>
__global__ void __launch_bounds__(T::threads, 2)
k_gemm_q8r(const int8_t *__restrict__ W, const float *__restrict__ S, const uint8_t *__restrict__ xq,
           const int *__restrict__ shift, const float *__restrict__ X, float *__restrict__ Y, int R, int K,
           int batch) {
    constexpr int MT = T::MT, SP = T::S, DA = T::DA, NA = DA + 1;
    constexpr int NACC = MT * NT * 3;
    constexpr int UNR = NA % 2 ? 2 * NA : NA;   // a multiple of both set counts
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rw = wave / SP, sp = wave - rw * SP;
    const int grp = blockIdx.y, KC = K >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int nk = sp < KC ? (KC - sp + SP - 1) / SP : 0;   // chunks of this wave
    int rbeg, rend;
    if constexpr (SP == 1) {
        const int64_t nw = (int64_t)gridDim.x * T::RW, gw = (int64_t)blockIdx.x * T::RW + rw;
        rbeg = (int)(gw * R / nw);
        rend = (int)((gw + 1) * R / nw);
    } else {
        rbeg = (blockIdx.x * T::RW + rw) * (16 * MT);
        rend = min(rbeg + 16 * MT, R);
    }
    const int rlast = max(min(rend, R) - 1, 0);
    const int ngroups = SP > 1 ? 1 : (rend - rbeg + 16 * MT - 1) / (16 * MT);
    const mh_gbytes bp = mh_global(xq + ((size_t)grp * KC * 3 * NT * 64 + lane) * 16);
    auto chunk = [&](int it) { return min(sp + it * SP, KC - 1); };
    for (int gi = 0; gi < ngroups; ++gi) {
        const int r0 = rbeg + gi * 16 * MT;
        mh_gbytes ap[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int r = min(r0 + 16 * m + i, rlast);
            ap[m] = mh_global(W + (size_t)r * K + 16 * g);
        }
        mh_i4 acc[MT][NT][3];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int d = 0; d < 3; ++d) acc[m][n][d] = mh_i4{0, 0, 0, 0};
        mh_u4 a[NA][MT], b[2][3 * NT];
        auto load_a = [&](int set, int kc) {
#pragma unroll
            for (int m = 0; m < MT; ++m) a[set][m] = mh_load16(ap[m] + (size_t)kc * 64);
        };
        auto load_b = [&](int set, int kc) {
#pragma unroll
            for (int j = 0; j < 3 * NT; ++j)
                b[set][j] =
                    *(const mh_u4 __attribute__((address_space(1))) *)(bp + ((size_t)kc * 3 * NT + j) * 1024);
        };
        auto step = [&](int j, int it) {   // j: position in the unrolled group (register sets)
            load_b((j + 1) % 2, chunk(it + 1));
            load_a((j + DA) % NA, chunk(it + DA));
            __builtin_amdgcn_sched_barrier(0);   // keep the issue order: loads, then this step's math
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int d = 0; d < 3; ++d)
                        acc[m][n][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            (mh_i4)a[j % NA][m], (mh_i4)b[j % 2][d * NT + n], acc[m][n][d], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        };
        load_b(0, chunk(0));
#pragma unroll
        for (int d = 0; d < DA; ++d) load_a(d, chunk(d));
        int it = 0;
        for (; it + UNR <= nk; it += UNR) {
#pragma unroll
            for (int j = 0; j < UNR; ++j) step(j, it + j);
        }
#pragma unroll
        for (int j = 0; j < UNR - 1; ++j)
            if (it + j < nk) step(j, it + j);
        if constexpr (SP > 1) {
            __shared__ mh_i4 red[T::RW * (SP - 1) * NACC * 64];
            if (sp > 0) {
                mh_i4 *o = red + ((size_t)(rw * (SP - 1) + sp - 1) * NACC) * 64 + lane;
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int n = 0; n < NT; ++n)
#pragma unroll
                        for (int d = 0; d < 3; ++d) o[((m * NT + n) * 3 + d) * 64] = acc[m][n][d];
            }
            __syncthreads();
            if (sp > 0) return;
            for (int w = 0; w < SP - 1; ++w) {
                const mh_i4 *o = red + ((size_t)(rw * (SP - 1) + w) * NACC) * 64 + lane;
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int n = 0; n < NT; ++n)
#pragma unroll
                        for (int d = 0; d < 3; ++d) acc[m][n][d] += o[((m * NT + n) * 3 + d) * 64];
            }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const int col = grp * kQ8Cols + 16 * n + i;
            if (col >= batch) continue;
            const int sh = shift[col];
            float *yc = Y + (size_t)col * R;
            if (sh == kQ8NonFinite) {
                // a column holding inf or nan: the plain f32 sum, so the
                // pattern of infinities and nans is that of mv_q8r
                const float *xc = X + (size_t)col * K;
#pragma unroll 1
                for (int e = 0; e < 4 * MT; ++e) {
                    const int row = r0 + 16 * (e >> 2) + 4 * g + (e & 3);
                    if (row >= rend) continue;
                    const int8_t *wr = W + (size_t)row * K;
                    float t = 0.f;
                    for (int k = 0; k < K; ++k) t = __builtin_fmaf((float)wr[k], xc[k], t);
                    yc[row] = t * S[row];
                }
                continue;
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row = r0 + 16 * m + 4 * g + q;
                    if (row >= rend) continue;
                    const float t = (float)acc[m][n][0][q] * 65536.f +
                                    ((float)acc[m][n][1][q] * 256.f + (float)acc[m][n][2][q]);
                    yc[row] = ldexpf(t, sh) * S[row];
                }
        }
    }
}

// Long int8 matrices (the lm_head) at batch 2+: a wave owns tiles of 16 MT
// rows, an equal contiguous share of them. Per K super-step of 512 columns
// it loads two of its rows' next 512 bytes with each 64-lane instruction
// (contiguous runs of whole rows: the fastest HBM pattern; the matrix-core
// operand layout, 16 rows x 64 bytes per instruction, streams ~25% slower),
// writes them to its private LDS buffer at a row stride of 528 bytes (the
// operand lanes' 16 rows then fall in distinct banks), issues the next
// super-step's loads, and runs the step's matrix instructions from LDS.
// Digits as in k_gemm_q8r (L2 hits), DB chunks ahead. 67.6 KB of LDS and
// under 256 VGPRs: two blocks per CU. (lm_head 201088 x 2880 at batch 32:
// 252 us with the operand-layout loads; with this kernel and 1024-column
// super-steps (one block per CU) 226 us at MT = 1, 214 at MT = 2, 208 with
// the digits four chunks ahead; 200 us with 512-column super-steps.)
constexpr int kQ8SS = 512;         // bytes of a row per super-step (8 chunks of 64)
constexpr int kQ8RowLds = 528;     // LDS row stride
constexpr int kQ8RowWaves = 4;     // waves per block (each with its own buffer)

template <int NT, int MT, int DB>
__global__ void __launch_bounds__(64 * kQ8RowWaves, 2)
k_gemm_q8r_rows(const int8_t *__restrict__ W, const float *__restrict__ S, const uint8_t *__restrict__ xq,
                const int *__restrict__ shift, const float *__restrict__ X, float *__restrict__ Y, int R, int K,
                int batch) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kQ8RowWaves][16 * MT * kQ8RowLds];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = blockIdx.y, KC = K >> 6, NSS = (K + kQ8SS - 1) / kQ8SS;
    const int i = lane & 15, g = lane >> 4;
    const int64_t T = (R + 16 * MT - 1) / (16 * MT), nw = (int64_t)gridDim.x * kQ8RowWaves, gw = (int64_t)blockIdx.x * kQ8RowWaves + wave;
    const int tbeg = (int)(gw * T / nw), tend = (int)((gw + 1) * T / nw);
    uint8_t *buf = lds[wave];
    const mh_gbytes bp = mh_global(xq + ((size_t)grp * KC * 3 * NT * 64 + lane) * 16);
    mh_u4 st[8 * MT];    // one super-step of the 16 MT rows: rows 2 j, 2 j + 1 (lane halves), 16 bytes a lane
    mh_u4 b[DB][3 * NT];
    auto load_b = [&](int set, int kc) {
#pragma unroll
        for (int j = 0; j < 3 * NT; ++j)
            b[set][j] = *(const mh_u4 __attribute__((address_space(1))) *)(bp + ((size_t)kc * 3 * NT + j) * 1024);
    };
    for (int tile = tbeg; tile < tend; ++tile) {
        const int r0 = tile * 16 * MT;
        auto load_ss = [&](int ss) {
            const int o = ss * kQ8SS + 16 * (lane & 31);
#pragma unroll
            for (int j = 0; j < 8 * MT; ++j) {
                const int r = min(r0 + 2 * j + (lane >> 5), R - 1);
                st[j] = o < K ? mh_load16(mh_global(W + (size_t)r * K + o)) : mh_u4{0u, 0u, 0u, 0u};
            }
        };
        mh_i4 acc[MT][NT][3];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int d = 0; d < 3; ++d) acc[m][n][d] = mh_i4{0, 0, 0, 0};
#pragma unroll
        for (int d = 0; d + 1 < DB; ++d) load_b(d, min(d, KC - 1));
        load_ss(0);
        for (int ss = 0; ss < NSS; ++ss) {
            // this super-step's rows into LDS (the wave's own LDS accesses
            // complete in order: the last step's reads are done), then the
            // next super-step's loads
#pragma unroll
            for (int j = 0; j < 8 * MT; ++j)
                *(mh_u4 *)(buf + (2 * j + (lane >> 5)) * kQ8RowLds + 16 * (lane & 31)) = st[j];
            if (ss + 1 < NSS) load_ss(ss + 1);
            const int nc = min(kQ8SS / 64, KC - (kQ8SS / 64) * ss);
            const uint8_t *ab = buf + i * kQ8RowLds + 16 * g;
            for (int c = 0; c < nc; c += DB) {
#pragma unroll
                for (int h = 0; h < DB; ++h) {
                    if (c + h >= nc) break;
                    const int kc = (kQ8SS / 64) * ss + c + h;   // its digits are in set kc % DB = h
                    load_b((h + DB - 1) % DB, min(kc + DB - 1, KC - 1));
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const mh_u4 a = *(const mh_u4 *)(ab + 16 * m * kQ8RowLds + 64 * (c + h));
#pragma unroll
                        for (int n = 0; n < NT; ++n)
#pragma unroll
                            for (int d = 0; d < 3; ++d)
                                acc[m][n][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                    (mh_i4)a, (mh_i4)b[h][d * NT + n], acc[m][n][d], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const int col = grp * kQ8Cols + 16 * n + i;
            if (col >= batch) continue;
            const int sh = shift[col];
            float *yc = Y + (size_t)col * R;
            if (sh == kQ8NonFinite) {
                // a column holding inf or nan: the plain f32 sum, so the
                // pattern of infinities and nans is that of mv_q8r
                const float *xc = X + (size_t)col * K;
#pragma unroll 1
                for (int q = 0; q < 4 * MT; ++q) {
                    const int row = r0 + 16 * (q >> 2) + 4 * g + (q & 3);
                    if (row >= R) continue;
                    const int8_t *wr = W + (size_t)row * K;
                    float t = 0.f;
                    for (int k = 0; k < K; ++k) t = __builtin_fmaf((float)wr[k], xc[k], t);
                    yc[row] = t * S[row];
                }
                continue;
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row = r0 + 16 * m + 4 * g + q;
                    if (row >= R) continue;
                    const float t = (float)acc[m][n][0][q] * 65536.f +
                                    ((float)acc[m][n][1][q] * 256.f + (float)acc[m][n][2][q]);
                    yc[row] = ldexpf(t, sh) * S[row];
                }
        }
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

// Batched int8 GEMV on the matrix cores when the shape fits it (int8 rows of
// 64-multiple width up to kQ8MaxK, 16-byte aligned operands, 2+ columns);
// *done = false leaves the call to the per-column kernel.
int launch_gemm_q8r(const DevWT &w, const float *x, float *y, int batch, hipStream_t s, bool *done) {
    *done = false;
    const int64_t R = w.rows, K = w.cols;
    if (w.dt != MH_DT_Q8R || batch < 2 || R < 1 || K < 64 || K % 64 != 0 || K > kQ8MaxK || R > (int64_t)INT32_MAX - 4096 ||
        (uintptr_t)w.data % 16 != 0)
        return MH_OK;
    if (sw(SW_NO_MFMA)) return MH_OK;
    const int groups = (batch + kQ8Cols - 1) / kQ8Cols;
    const int NT = batch > 16 ? 2 : 1;
    const uint64_t qbytes = (uint64_t)groups * (K / 64) * 3 * NT * 1024;
    void *p;
    MH_TRY(scratch(S_XQ, qbytes + (uint64_t)groups * kQ8Cols * 4, &p));
    uint8_t *xq = (uint8_t *)p;
    int *sh = (int *)(xq + qbytes);
    if (NT == 2)
        MH_LAUNCH("xdigits", k_xdigits<2>, dim3((unsigned)groups, 32), dim3(256), 0, s, x, (int)K, batch, xq, sh);
    else
        MH_LAUNCH("xdigits", k_xdigits<1>, dim3((unsigned)groups, 16), dim3(256), 0, s, x, (int)K, batch, xq, sh);
    // the long tiling when it gives every SIMD two waves, else the K-split one
    const bool longm = (R + Q8Long::rows - 1) / Q8Long::rows * (Q8Long::threads / 64) >= 2 * 4 * device_cus();
    // long: two blocks per CU, each wave an equal share of the rows
    const int64_t nlong = std::min<int64_t>((R + Q8Long::rows - 1) / Q8Long::rows, 2 * (int64_t)device_cus());
    auto go = [&](auto kern, int rows, int threads) {
        const int64_t nb = longm ? nlong : (R + rows - 1) / rows;
        MH_LAUNCH("gemm_q8r", kern, dim3((unsigned)nb, (unsigned)groups), dim3(threads), 0, s,
                  (const int8_t *)w.data, (const float *)w.scales, xq, sh, x, y, (int)R, (int)K, batch);
    };
    if (longm && !sw(SW_Q8_NO_ROWS)) {
        // two blocks of 4 waves per CU, each wave 32-row tiles
        const int64_t nb = std::min<int64_t>((R + 31) / 32 / kQ8RowWaves + 1, 2 * (int64_t)device_cus());
        auto go2 = [&](auto kern) {
            MH_LAUNCH("gemm_q8r_rows", kern, dim3((unsigned)nb, (unsigned)groups), dim3(64 * kQ8RowWaves), 0, s,
                      (const int8_t *)w.data, (const float *)w.scales, xq, sh, x, y, (int)R, (int)K, batch);
        };
        // digit chunks in flight: as many as fit beside the staged rows at
        // two waves per SIMD (three spill at two column groups)
        if (NT == 2) go2(k_gemm_q8r_rows<2, 2, 2>);
        else go2(k_gemm_q8r_rows<1, 2, 4>);
    } else if (longm) {
        if (NT == 2) go(k_gemm_q8r<2, Q8Long>, Q8Long::rows, Q8Long::threads);
        else go(k_gemm_q8r<1, Q8Long>, Q8Long::rows, Q8Long::threads);
    } else {
        if (NT == 2) go(k_gemm_q8r<2, Q8Short>, Q8Short::rows, Q8Short::threads);
        else go(k_gemm_q8r<1, Q8Short>, Q8Short::rows, Q8Short::threads);
    }
    *done = true;
    return hip_check(hipGetLastError(), "gemm_q8r launch");
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
    return sync_checked(s);
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
    return sync_checked(s);
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
    if (batch > 65535) return fail(MH_E_ARG, "batch %d out of range [1, 65535]", batch);
    bool done;
    MH_TRY(launch_gemm_q8r(w, x, y, batch, stream(), &done));
    if (done) return MH_OK;
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
