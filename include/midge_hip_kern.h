/* midge_hip_kern.h — the reference engine's kernel interface on libmidge_hip.
 *
 * engine/midge.c includes engine/mkern.h, whose whole body is guarded by
 * WKERN_H (engine/mkern.h:5). Building the engine with
 *
 *     cc ... -DWKERN_H -include midge_hip_kern.h -I<midge>/engine engine/midge.c \
 *        -L<repo>/midge_amd -lmidge_hip
 *
 * replaces every kernel the forward loop calls with the definitions below,
 * with the reference's own names and signatures, and no edit to midge.c:
 *
 *   wk_matvec   engine/mkern.h:180-198   -> mh_matvec (GPU, all four dtypes)
 *   wk_row      engine/mkern.h:201-236   -> mh_row    (GPU, bit-exact)
 *   wk_rmsnorm  engine/mkern.h:238-243   host (O(hidden), feeds the host loop)
 *   wk_addbias  engine/mkern.h:245-247   host
 *   wk_dot, wk_dot_f16, wk_to_f16        host (attention's f16 KV cache)
 *
 * Weights live in the engine's read-only mmaps. The first time a tensor is
 * used its data and scales are uploaded (mh_register_region) and stay
 * resident: HBM takes the place of the page cache. A host that registers the
 * whole experts.midge data region up front (one mh_register_region call
 * after model_load) uploads it in one piece instead.
 *
 * Failures follow the engine's convention: "# <message>" on stderr and exit
 * code 3 (engine/midge.c:136, 195-227).
 */
#ifndef MIDGE_HIP_KERN_H
#define MIDGE_HIP_KERN_H
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "midge_hip.h"
#include "mten.h"

_Static_assert(sizeof(WT) == sizeof(mh_wt), "WT and mh_wt must be layout-identical");
_Static_assert(offsetof(WT, data) == offsetof(mh_wt, data), "WT.data offset");
_Static_assert(offsetof(WT, scales) == offsetof(mh_wt, scales), "WT.scales offset");

static void wk_gpu_fatal(const char *what) {
    fprintf(stderr, "# gpu %s: %s\n", what, mh_last_error());
    exit(3);
}

static void wk_gpu_ready(void) {
    static int ready = 0;
    if (ready) return;
    const char *d = getenv("MIDGE_HIP_DEVICE");
    if (mh_init(d ? atoi(d) : 0) != MH_OK) wk_gpu_fatal("init");
    ready = 1;
}

/* Upload a tensor's blobs the first time they are seen. */
static void wk_gpu_resident(const WT *t) {
    size_t db = 0, sb = 0;
    wt_sizes(t->dt, t->rows, t->cols, &db, &sb);
    void *dev;
    if (db && mh_register_region(t->data, db, &dev) != MH_OK) wk_gpu_fatal("upload");
    if (sb && t->scales && mh_register_region(t->scales, sb, &dev) != MH_OK) wk_gpu_fatal("upload");
}

static void wk_matvec(const WT *t, const float *x, float *y) {
    wk_gpu_ready();
    int rc = mh_matvec((const mh_wt *)t, x, y);
    if (rc == MH_E_UNREGISTERED) {
        wk_gpu_resident(t);
        rc = mh_matvec((const mh_wt *)t, x, y);
    }
    if (rc != MH_OK) wk_gpu_fatal("matvec");
}

static void wk_row(const WT *t, int64_t r, float *out) {
    wk_gpu_ready();
    int rc = mh_row((const mh_wt *)t, r, out);
    if (rc == MH_E_UNREGISTERED) {
        wk_gpu_resident(t);
        rc = mh_row((const mh_wt *)t, r, out);
    }
    if (rc != MH_OK) wk_gpu_fatal("row");
}

/* Host-side helpers of the attention path (out of the GPU path's scope). */

static void wk_rmsnorm(const float *x, const float *w, float *out, int64_t n, float eps) {
    float ss = 0.f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

static void wk_addbias(float *y, const float *b, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] += b[i];
}

static inline float wk_dot(const float *a, const float *b, int n) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

static inline float wk_dot_f16(const float *a, const uint16_t *b, int n) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s += a[i] * wt_f16(b[i]);
    return s;
}

/* f32 -> f16 bits as the engine's KV cache stores them: round to nearest
 * even, results below the f16 normal range flush to signed zero, overflow
 * saturates to infinity. */
static inline uint16_t wk_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int e = (int)((u >> 23) & 0xffu) - 112;         /* f16 biased exponent */
    uint32_t mant = u & 0x7fffffu;
    if (e <= 0) return sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13); /* exponent+mantissa, truncated */
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;   /* carries into the exponent */
    if (h >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | h);
}

static int wk_have_avx2(void) { return 0; }

#endif /* MIDGE_HIP_KERN_H */
