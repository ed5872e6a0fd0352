// mh_mfma16.cuh — MXFP4 rows on the f16 matrix cores (V_MFMA_F32_16X16X32_F16;
// measured layout on gfx950: lane l holds A row l % 16 and B column l % 16,
// 8 consecutive K values 8 (l / 16) .. +7 each; output lane l holds column
// l % 16 of rows 4 (l / 16) + i). A K step of 128 = 4 lane groups x 32 takes
// one 16-byte MXFP4 chunk per lane group: lane (m, g) converts dword j of
// its chunk for the step's j-th instruction, and B lane (n, g) supplies
// elements 8 j .. 8 j + 7 of the same chunk's 32 columns.
#pragma once

#include "mh_internal.h"

namespace mh {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Eight e2m1 values (one dword) times the chunk's scale s as f16: exact when
// s is zero or a power of two in [2^-23, 2^13].
__device__ __forceinline__ v8h fp4x8_f16(uint32_t w, float s) {
    const v2h a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 0);
    const v2h b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 1);
    const v2h c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 2);
    const v2h d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, s, 3);
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ uint32_t dword_of(const mh_u4 &q, int j) {
    return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}

}  // namespace
}  // namespace mh
