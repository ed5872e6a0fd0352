/* midge_oracle.c — CPU restatement of midge's quantized-MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity oracle: tests/, the
 * smoke() check and the CPU-baseline leg of bench.py load it as a checker.
 * No product code path may link, load or call it; the HIP library never
 * falls back to it.
 *
 * Each function restates one piece of the reference engine and names the
 * file:line it follows (paths relative to the midge source tree).
 * Arithmetic follows the reference's *scalar* kernels: f32 throughout,
 * sequential sums in the same order, and no FMA contraction (this file is
 * compiled with -ffp-contract=off, as the reference's -std=c11 build is).
 *
 * Pinning (what checks each function against something other than itself):
 *   mo_f16_to_f32        exhaustive over all 65536 encodings vs numpy float16
 *   mo_fp4_value         the OCP E2M1 table + brute force over 16 codes
 *   mo_dequant_row       closed form + the compiled reference wk_row
 *   mo_matvec            brute-force f64 dot products + compiled mv_* kernels
 *   mo_rmsnorm           closed form (f64) + compiled wk_rmsnorm
 *   mo_topk_*            stable argsort invariant + brute force + compiled
 *   mo_router_weights    closed-form softmax (f64)
 *   mo_act               closed form (f64) of the clamped SwiGLU
 *   mo_expert_layout     closed-form offsets at gpt-oss shapes + compiled
 *   mo_moe_decode        compiled moe() on identical inputs
 *   mo_moe_prefill       compiled route_topk/expert_apply in expert-major order
 *   mo_synth_*           numpy restatement of the same counter hash
 *   mo_rope_table        compiled rope_init() tables, bit for bit
 *   mo_to_f16            compiled wk_to_f16 over sampled and edge inputs
 *   mo_attention         compiled attention() (scalar kernels), bit for bit
 *   mo_rng_f, mo_sample  compiled sample() with the same generator state
 *                        (through the reference shim), plus the greedy =
 *                        first argmax, tiny-top-p = argmax and sampled
 *                        frequency = softmax checks
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/midge_hip.h"

#define MO_MAX_TOPK 16   /* engine/midge.c:44 MAX_TOPK */

/* ------------------------------------------------------------ scalars */

/* IEEE binary16 -> binary32, exact for every encoding (engine/mten.h:49-57).
 * Written from the binary16 definition: subnormals are m * 2^-24, which is
 * exactly representable in f32; inf/NaN keep their payload bits. */
float mo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    float f;
    if (e == 0) {
        f = ldexpf((float)m, -24);
        if (sign) f = -f;
        return f;                                  /* +-0 and subnormals */
    }
    if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

/* FP4 E2M1 code -> value (engine/mten.h:44-47). Bit 3 is the sign, bits 2:1
 * the exponent (bias 1), bit 0 the mantissa; exponent 0 is subnormal
 * (0 or 0.5). Code 8 is -0.0. */
float mo_fp4_value(int code) {
    int s = (code >> 3) & 1, e = (code >> 1) & 3, m = code & 1;
    float mag = (e == 0) ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1);
    return s ? -mag : mag;
}

/* ------------------------------------------------------------ kernels */

/* Dequantize row r of a [rows x cols] tensor into out[cols].
 * engine/mkern.h:201-236 (wk_row). Returns MH_E_DTYPE for an unknown dt. */
int mo_dequant_row(int dt, const void *data, const void *scales, int64_t cols,
                   int64_t r, float *out) {
    switch (dt) {
    case MH_DT_F32:
        memcpy(out, (const float *)data + r * cols, (size_t)cols * 4);
        return 0;
    case MH_DT_Q8R: {
        const int8_t *w = (const int8_t *)data + r * cols;
        float s = ((const float *)scales)[r];
        for (int64_t c = 0; c < cols; c++) out[c] = (float)w[c] * s;
        return 0;
    }
    case MH_DT_Q4G32:
    case MH_DT_MXFP4: {
        const uint8_t *w = (const uint8_t *)data + r * (cols / 2);
        const uint16_t *s = (const uint16_t *)scales + r * (cols / 32);
        for (int64_t g = 0; g < cols / 32; g++) {
            float sc = mo_f16_to_f32(s[g]);
            for (int j = 0; j < 16; j++) {
                uint8_t b = w[g * 16 + j];
                float lo, hi;
                if (dt == MH_DT_MXFP4) { lo = mo_fp4_value(b & 15); hi = mo_fp4_value(b >> 4); }
                else { lo = (float)((int)(b & 15) - 8); hi = (float)((int)(b >> 4) - 8); }
                out[g * 32 + 2 * j] = lo * sc;          /* low nibble = even column */
                out[g * 32 + 2 * j + 1] = hi * sc;
            }
        }
        return 0;
    }
    }
    return MH_E_DTYPE;
}

/* y = W x, scalar reference order. engine/mkern.h:13-62 (mv_f32, mv_q8r,
 * mv_g32): one sequential f32 sum per row; for the 4-bit types a per-group
 * partial a = sum_j (lo*x[2j] then hi*x[2j+1]) is folded as acc += s*a. */
int mo_matvec(int dt, const void *data, const void *scales, const float *x,
              float *y, int64_t rows, int64_t cols) {
    if (dt != MH_DT_F32 && dt != MH_DT_Q8R && dt != MH_DT_Q4G32 && dt != MH_DT_MXFP4)
        return MH_E_DTYPE;
    for (int64_t r = 0; r < rows; r++) {
        if (dt == MH_DT_F32) {
            const float *w = (const float *)data + r * cols;
            float a = 0.f;
            for (int64_t c = 0; c < cols; c++) a += w[c] * x[c];
            y[r] = a;
        } else if (dt == MH_DT_Q8R) {
            const int8_t *w = (const int8_t *)data + r * cols;
            float a = 0.f;
            for (int64_t c = 0; c < cols; c++) a += (float)w[c] * x[c];
            y[r] = a * ((const float *)scales)[r];
        } else {
            const uint8_t *w = (const uint8_t *)data + r * (cols / 2);
            const uint16_t *s = (const uint16_t *)scales + r * (cols / 32);
            float acc = 0.f;
            for (int64_t g = 0; g < cols / 32; g++) {
                const uint8_t *wb = w + g * 16;
                const float *xg = x + g * 32;
                float a = 0.f;
                for (int j = 0; j < 16; j++) {
                    uint8_t b = wb[j];
                    float lo, hi;
                    if (dt == MH_DT_MXFP4) { lo = mo_fp4_value(b & 15); hi = mo_fp4_value(b >> 4); }
                    else { lo = (float)((int)(b & 15) - 8); hi = (float)((int)(b >> 4) - 8); }
                    a += lo * xg[2 * j];
                    a += hi * xg[2 * j + 1];
                }
                acc += mo_f16_to_f32(s[g]) * a;
            }
            y[r] = acc;
        }
    }
    return 0;
}

/* engine/mkern.h:238-243 (wk_rmsnorm): sequential f32 sum of squares. */
void mo_rmsnorm(const float *x, const float *w, float *out, int64_t n, float eps) {
    float ss = 0.f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* engine/mkern.h:245-247 (wk_addbias). */
void mo_addbias(float *y, const float *b, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] += b[i];
}

/* Top-k as moe() does it (engine/midge.c:476-486): insertion into a
 * descending list with strict comparisons, so ties keep the lower expert
 * index; slots never filled stay (-1, -1e30). */
void mo_topk_decode(const float *rl, int n_experts, int k, int *sel, float *val) {
    for (int i = 0; i < k; i++) { sel[i] = -1; val[i] = -1e30f; }
    for (int e = 0; e < n_experts; e++) {
        float v = rl[e];
        if (v > val[k - 1]) {
            int j = k - 1;
            while (j > 0 && val[j - 1] < v) { val[j] = val[j - 1]; sel[j] = sel[j - 1]; j--; }
            val[j] = v; sel[j] = e;
        }
    }
}

/* Top-k as route_topk() does it (engine/midge.c:410-422): same order, but
 * unfilled slots stay (0, -1e30). */
void mo_topk_route(const float *rl, int n_experts, int k, int *sel, float *val) {
    for (int j = 0; j < k; j++) { val[j] = -1e30f; sel[j] = 0; }
    for (int e = 0; e < n_experts; e++) {
        float v = rl[e];
        for (int j = 0; j < k; j++) {
            if (v > val[j]) {
                for (int q = k - 1; q > j; q--) { val[q] = val[q - 1]; sel[q] = sel[q - 1]; }
                val[j] = v; sel[j] = e;
                break;
            }
        }
    }
}

/* Routing weights (engine/midge.c:502-512, 423-433). router_norm=1: softmax
 * over the selected logits; 0: full-softmax probabilities, unrenormalised. */
void mo_router_weights(const float *rl, int n_experts, const float *val, int k,
                       int router_norm, float *w) {
    float mx = val[0], den = 0.f;
    if (router_norm) {
        for (int i = 0; i < k; i++) { w[i] = expf(val[i] - mx); den += w[i]; }
        for (int i = 0; i < k; i++) w[i] /= den;
    } else {
        float fmx = rl[0];
        for (int e = 1; e < n_experts; e++) if (rl[e] > fmx) fmx = rl[e];
        float fden = 0.f;
        for (int e = 0; e < n_experts; e++) fden += expf(rl[e] - fmx);
        for (int i = 0; i < k; i++) w[i] = expf(val[i] - fmx) / fden;
    }
}

/* Expert activation, in place into g (engine/midge.c:525-538, 448-462).
 * Clamped: g = min(g, limit); u = clamp(u, -limit, limit);
 * h = g / (1 + exp(-alpha g)) * (u + 1). Plain: h = silu(g) * u. */
void mo_act(float *g, const float *u, int64_t n, float alpha, float limit, int act_plain) {
    for (int64_t j = 0; j < n; j++) {
        float gj = g[j], uj = u[j];
        if (act_plain) { g[j] = gj / (1.0f + expf(-gj)) * uj; continue; }
        if (gj > limit) gj = limit;
        if (uj > limit) uj = limit;
        if (uj < -limit) uj = -limit;
        float a = gj / (1.0f + expf(-alpha * gj));
        g[j] = a * (uj + 1.0f);
    }
}

/* ------------------------------------------------------------- layout */

static uint64_t mo_align64(uint64_t x) { return (x + 63u) & ~(uint64_t)63u; }

static int mo_sizes(int dt, int64_t rows, int64_t cols, uint64_t *db, uint64_t *sb) {
    switch (dt) {
    case MH_DT_F32: *db = (uint64_t)rows * cols * 4; *sb = 0; return 0;
    case MH_DT_Q8R: *db = (uint64_t)rows * cols; *sb = (uint64_t)rows * 4; return 0;
    case MH_DT_Q4G32:
    case MH_DT_MXFP4: *db = (uint64_t)rows * cols / 2; *sb = (uint64_t)rows * (cols / 32) * 2; return 0;
    }
    return MH_E_DTYPE;
}

/* Per-expert blob offsets (engine/mten.h:101-150; tools/midgepack.py:166-205):
 * for m in gate, up, down: data, scales, f32 bias, each 64-byte aligned.
 * off[3*m + part]; expert_stride is the 64-aligned end. */
int mo_expert_layout(int dt, int64_t hidden, int64_t ffn, int64_t n_experts,
                     uint64_t off[9], uint64_t *expert_stride, uint64_t *layer_stride) {
    int64_t rows[3] = { ffn, ffn, hidden }, cols[3] = { hidden, hidden, ffn };
    uint64_t o = 0;
    for (int m = 0; m < 3; m++) {
        uint64_t db, sb;
        if (mo_sizes(dt, rows[m], cols[m], &db, &sb)) return MH_E_DTYPE;
        off[3 * m + 0] = o; o = mo_align64(o + db);
        off[3 * m + 1] = o; o = mo_align64(o + sb);
        off[3 * m + 2] = o; o = mo_align64(o + (uint64_t)rows[m] * 4);
    }
    *expert_stride = mo_align64(o);
    *layer_stride = *expert_stride * (uint64_t)n_experts;
    return 0;
}

/* ---------------------------------------------------------------- MoE */

static const uint8_t *mo_blob(const mh_moe_layer *L, int e, int m, int part) {
    return (const uint8_t *)L->experts + (uint64_t)e * L->expert_stride + L->off[3 * m + part];
}

/* Router: xb = rmsnorm(x), rl = W_r xb + b_r (engine/midge.c:471-473, 407-409). */
static int mo_router(const mh_moe_layer *L, const float *x, float *xb, float *rl) {
    mo_rmsnorm(x, L->mlp_norm, xb, L->hidden, L->norm_eps);
    int rc = mo_matvec(L->router.dt, L->router.data, L->router.scales, xb, rl,
                       L->router.rows, L->router.cols);
    if (rc) return rc;
    mo_addbias(rl, L->router_b, L->n_experts);
    return 0;
}

/* One expert's output y = down(act(gate xb + bg, up xb + bu)) + bd
 * (engine/midge.c:520-543, 442-464). scratch: 2*ffn floats. */
static int mo_expert_out(const mh_moe_layer *L, int e, const float *xb, float *y, float *scratch) {
    float *hb = scratch, *hb2 = scratch + L->ffn;
    int dt = L->expert_dt, rc;
    rc = mo_matvec(dt, mo_blob(L, e, 0, 0), mo_blob(L, e, 0, 1), xb, hb, L->ffn, L->hidden);
    if (rc) return rc;
    mo_addbias(hb, (const float *)mo_blob(L, e, 0, 2), L->ffn);
    mo_matvec(dt, mo_blob(L, e, 1, 0), mo_blob(L, e, 1, 1), xb, hb2, L->ffn, L->hidden);
    mo_addbias(hb2, (const float *)mo_blob(L, e, 1, 2), L->ffn);
    mo_act(hb, hb2, L->ffn, L->alpha, L->limit, L->act_plain);
    mo_matvec(dt, mo_blob(L, e, 2, 0), mo_blob(L, e, 2, 1), hb, y, L->hidden, L->ffn);
    mo_addbias(y, (const float *)mo_blob(L, e, 2, 2), L->hidden);
    return 0;
}

/* One expert's FFN y[hidden] = down(act(gate xb + bg, up xb + bu)) + bd
 * (engine/midge.c:442-464 without the weighted accumulate). */
int mo_expert_ffn(const mh_moe_layer *L, int e, const float *xb, float *y) {
    if (e < 0 || e >= L->n_experts) return MH_E_RANGE;
    float *scratch = (float *)malloc(sizeof(float) * (size_t)(2 * L->ffn));
    if (!scratch) return MH_E_NOMEM;
    int rc = mo_expert_out(L, e, xb, y, scratch);
    free(scratch);
    return rc;
}

/* Decode MoE layer, in place on x[hidden] (engine/midge.c:469-549):
 * router, top-k, weights, then moe = sum_i w_i y_i in selection order and
 * x += moe. sel/w receive the routing (k entries). usage (may be NULL) is
 * the [n_experts] row of this layer's histogram (midge.c:517-518). */
int mo_moe_decode(const mh_moe_layer *L, float *x, int32_t *sel_out, float *w_out,
                  uint32_t *usage, uint64_t *loads) {
    int64_t H = L->hidden;
    int k = L->top_k, E = L->n_experts;
    if (k < 1 || k > MO_MAX_TOPK || k > E) return MH_E_ARG;
    float *buf = (float *)malloc(sizeof(float) * (size_t)(2 * H + E + 2 * L->ffn + H));
    if (!buf) return MH_E_NOMEM;
    float *xb = buf, *moe = buf + H, *rl = buf + 2 * H, *scratch = rl + E, *y = scratch + 2 * L->ffn;
    int rc = mo_router(L, x, xb, rl);
    if (rc) { free(buf); return rc; }
    int sel[MO_MAX_TOPK]; float val[MO_MAX_TOPK], w[MO_MAX_TOPK];
    mo_topk_decode(rl, E, k, sel, val);
    mo_router_weights(rl, E, val, k, L->router_norm, w);
    memset(moe, 0, sizeof(float) * (size_t)H);
    for (int i = 0; i < k; i++) {
        int e = sel[i];
        if (e < 0) { free(buf); return MH_E_RANGE; }   /* reference would index out of range */
        if (usage) usage[e]++;
        if (loads) (*loads)++;
        rc = mo_expert_out(L, e, xb, y, scratch);
        if (rc) { free(buf); return rc; }
        for (int64_t j = 0; j < H; j++) moe[j] += w[i] * y[j];
    }
    for (int64_t j = 0; j < H; j++) x[j] += moe[j];
    for (int i = 0; i < k; i++) { sel_out[i] = sel[i]; w_out[i] = w[i]; }
    free(buf);
    return 0;
}

/* Router for a batch, as route_topk (engine/midge.c:404-434): per token
 * xb (saved), sel and w with MAX_TOPK-free packing [n][k]. */
int mo_route_batch(const mh_moe_layer *L, int n, const float *x, float *xb,
                   int32_t *sel_out, float *w_out) {
    int k = L->top_k, E = L->n_experts;
    if (k < 1 || k > MO_MAX_TOPK || k > E) return MH_E_ARG;
    float *rl = (float *)malloc(sizeof(float) * (size_t)E);
    if (!rl) return MH_E_NOMEM;
    for (int t = 0; t < n; t++) {
        int rc = mo_router(L, x + (int64_t)t * L->hidden, xb + (int64_t)t * L->hidden, rl);
        if (rc) { free(rl); return rc; }
        int sel[MO_MAX_TOPK]; float val[MO_MAX_TOPK];
        mo_topk_route(rl, E, k, sel, val);
        mo_router_weights(rl, E, val, k, L->router_norm, w_out + (int64_t)t * k);
        for (int i = 0; i < k; i++) sel_out[(int64_t)t * k + i] = sel[i];
    }
    free(rl);
    return 0;
}

/* Expert-major application (engine/midge.c:595-611 with expert_apply
 * 437-467): for e ascending, for t, for i: x_t += w_ti * y_e(xb_t). */
int mo_expert_major_apply(const mh_moe_layer *L, int n, const float *xb,
                          const int32_t *sel, const float *w, float *x,
                          uint32_t *usage, uint64_t *loads) {
    int64_t H = L->hidden;
    int k = L->top_k;
    float *buf = (float *)malloc(sizeof(float) * (size_t)(2 * L->ffn + H));
    if (!buf) return MH_E_NOMEM;
    float *scratch = buf, *y = buf + 2 * L->ffn;
    for (int e = 0; e < L->n_experts; e++)
        for (int t = 0; t < n; t++)
            for (int i = 0; i < k; i++)
                if (sel[(int64_t)t * k + i] == e) {
                    if (usage) usage[e]++;
                    if (loads) (*loads)++;
                    int rc = mo_expert_out(L, e, xb + (int64_t)t * H, y, scratch);
                    if (rc) { free(buf); return rc; }
                    float wt = w[(int64_t)t * k + i];
                    float *xo = x + (int64_t)t * H;
                    for (int64_t j = 0; j < H; j++) xo[j] += wt * y[j];
                }
    free(buf);
    return 0;
}

/* Prefill MoE for n tokens in place on x[n][hidden]: the MoE half of
 * forward_batch (engine/midge.c:591-611). */
int mo_moe_prefill(const mh_moe_layer *L, int n, float *x, int32_t *sel, float *w,
                   uint32_t *usage, uint64_t *loads) {
    float *xb = (float *)malloc(sizeof(float) * (size_t)n * (size_t)L->hidden + 4);
    if (!xb) return MH_E_NOMEM;
    int rc = mo_route_batch(L, n, x, xb, sel, w);
    if (!rc) rc = mo_expert_major_apply(L, n, xb, sel, w, x, usage, loads);
    free(xb);
    return rc;
}

/* -------------------------------------------------- synthetic inputs */

/* SplitMix64 finaliser over a keyed counter. The HIP generator
 * (midge_amd/csrc/mh_synth.hip) and midge_amd/synth.py compute the same
 * function; these are data generators, not part of the reference. */
static uint64_t mo_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t mo_hash64(uint64_t key, uint64_t i) {
    return mo_mix64(key + (i + 1) * 0x9e3779b97f4a7c15ull);
}

/* n bytes, byte i = byte (i % 8) of hash(key, i / 8) (little endian). */
void mo_synth_bytes(uint64_t key, uint64_t n, uint8_t *out) {
    uint64_t w = 0;
    for (uint64_t i = 0; i < n; i++) {
        if ((i & 7) == 0) w = mo_hash64(key, i >> 3);
        out[i] = (uint8_t)(w >> (8 * (i & 7)));
    }
}

/* n f16 power-of-two scales 2^e, e uniform in [emin, emax]:
 * e = emin + (hash(key, i) >> 32) % (emax - emin + 1). Normal range only. */
void mo_synth_scales(uint64_t key, uint64_t n, int emin, int emax, uint16_t *out) {
    uint32_t span = (uint32_t)(emax - emin + 1);
    for (uint64_t i = 0; i < n; i++) {
        int e = emin + (int)((uint32_t)(mo_hash64(key, i) >> 32) % span);
        out[i] = (uint16_t)((e + 15) << 10);
    }
}

/* n int8 values uniform in [-127, 127]: value i uses the 16-bit field
 * (i % 4) of hash(key, i / 4): v = field % 255 - 127. */
void mo_synth_i8(uint64_t key, uint64_t n, int8_t *out) {
    for (uint64_t i = 0; i < n; i++) {
        uint32_t f = (uint32_t)(mo_hash64(key, i >> 2) >> (16 * (i & 3))) & 0xffffu;
        out[i] = (int8_t)((int)(f % 255u) - 127);
    }
}

/* n floats (f32)(sum of the four 16-bit fields of hash(key, i) - 131070) * c:
 * an Irwin-Hall(4) stand-in for N(0, std^2) with c = std / 37837.23. */
void mo_synth_normal(uint64_t key, uint64_t n, float c, float *out) {
    for (uint64_t i = 0; i < n; i++) {
        uint64_t h = mo_hash64(key, i);
        int s = (int)(h & 0xffff) + (int)((h >> 16) & 0xffff) + (int)((h >> 32) & 0xffff) + (int)(h >> 48);
        out[i] = (float)(s - 131070) * c;
    }
}

/* n floats lo + (f32)(hash(key, i) >> 40) * c, c = (hi - lo) / 2^24. */
void mo_synth_uniform(uint64_t key, uint64_t n, float lo, float c, float *out) {
    for (uint64_t i = 0; i < n; i++) {
        float u = (float)(mo_hash64(key, i) >> 40) * c;
        out[i] = lo + u;
    }
}

/* One expert of a synthetic table (layout as mo_expert_layout): data bytes,
 * f16 scales in [emin, emax] and normal-ish f32 biases, with the keys
 * k(l,e,m,p) = hash(key, ((l * n_experts + e) * 3 + m) * 3 + p). */
int mo_synth_expert(uint8_t *dst, int dt, int64_t hidden, int64_t ffn, int64_t n_experts,
                    int layer, int expert, uint64_t key, int emin, int emax, float bias_c) {
    uint64_t off[9], es, ls;
    if (dt != MH_DT_MXFP4 && dt != MH_DT_Q4G32) return MH_E_DTYPE;
    int rc = mo_expert_layout(dt, hidden, ffn, n_experts, off, &es, &ls);
    if (rc) return rc;
    int64_t rows[3] = { ffn, ffn, hidden }, cols[3] = { hidden, hidden, ffn };
    uint64_t le = (uint64_t)layer * (uint64_t)n_experts + (uint64_t)expert;
    for (int m = 0; m < 3; m++) {
        uint64_t kb = (le * 3 + (uint64_t)m) * 3, db, sb;
        mo_sizes(dt, rows[m], cols[m], &db, &sb);
        mo_synth_bytes(mo_hash64(key, kb + 0), db, dst + off[3 * m]);
        mo_synth_scales(mo_hash64(key, kb + 1), sb / 2, emin, emax, (uint16_t *)(dst + off[3 * m + 1]));
        mo_synth_normal(mo_hash64(key, kb + 2), (uint64_t)rows[m], bias_c, (float *)(dst + off[3 * m + 2]));
    }
    return 0;
}

/* ------------------------------------------------------------ sampling */

/* The reference's generator, one draw (engine/midge.c:641-646): xorshift64
 * on *state, the high 32 bits of the multiplied state, then 24 bits as a
 * float in [0, 1). */
float mo_rng_f(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    const uint32_t u = (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 32);
    return (float)(u >> 8) / 16777216.0f;
}

typedef struct {
    float p;
    int i;
} MoPI;

/* descending probability, then ascending index (a stable sort's order) */
static int mo_pi_cmp(const void *a, const void *b) {
    const MoPI *x = (const MoPI *)a, *y = (const MoPI *)b;
    if (x->p != y->p) return x->p < y->p ? 1 : -1;
    return x->i < y->i ? -1 : x->i > y->i;
}

/* sample() (engine/midge.c:654-679) with the uniform draw u = rng_f()
 * supplied by the caller: temp <= 0 is the first maximum; otherwise the
 * temperature softmax (f32 terms, f64 denominator), the tokens by falling
 * probability, the smallest prefix whose f64 sum reaches topp, and the
 * token where the running f64 sum first reaches u * (that sum). */
int mo_sample(const float *logits, int64_t V, float temp, float topp, float u) {
    if (temp <= 0.f) {
        int best = 0;
        float bv = logits[0];
        for (int64_t i = 1; i < V; i++)
            if (logits[i] > bv) {
                bv = logits[i];
                best = (int)i;
            }
        return best;
    }
    float mx = logits[0];
    for (int64_t i = 1; i < V; i++)
        if (logits[i] > mx) mx = logits[i];
    MoPI *pi = (MoPI *)malloc((size_t)V * sizeof(MoPI));
    if (!pi) return -1;
    double den = 0;
    for (int64_t i = 0; i < V; i++) {
        pi[i].p = expf((logits[i] - mx) / temp);
        pi[i].i = (int)i;
        den += pi[i].p;
    }
    for (int64_t i = 0; i < V; i++) pi[i].p /= (float)den;
    qsort(pi, (size_t)V, sizeof(MoPI), mo_pi_cmp);
    double cum = 0;
    int64_t n = 0;
    for (; n < V; n++) {
        cum += pi[n].p;
        if (cum >= topp) {
            n++;
            break;
        }
    }
    const float r = u * (float)cum;
    double acc = 0;
    int pick = pi[n - 1].i;
    for (int64_t i = 0; i < n; i++) {
        acc += pi[i].p;
        if (r <= acc) {
            pick = pi[i].i;
            break;
        }
    }
    free(pi);
    return pick;
}

/* ------------------------------------------------------------ attention */

/* wk_to_f16 (engine/mkern.h:261-273): round to nearest even, results below
 * the normal range flush to a signed zero, and anything at or past the top
 * (inf and NaN included) becomes a signed infinity. */
uint16_t mo_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xff) - 112;   /* rebias 127 -> 15 */
    const uint32_t man = x & 0x7fffffu;
    if (e <= 0) return (uint16_t)sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t m = man >> 13;
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) {
        if (++m == 0x400u) {
            m = 0;
            if (++e >= 31) return (uint16_t)(sign | 0x7c00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | m);
}

#define MO_PI 3.14159265358979323846   /* the value of glibc's M_PI */

/* rope_init (engine/midge.c:141-175): inverse frequencies theta^(-2i/hd) in
 * f64, with YaRN's ramp between interpolation (inv / factor) and
 * extrapolation over the band [low, high] of dimensions and its magnitude
 * scale 0.1 ln(factor) + 1; tables cos/sin(p * inv) * mscale in f32. */
void mo_rope_table(int hd, float theta, int yarn, float factor, float beta_fast, float beta_slow, int orig_ctx,
                   int truncate, int ctx, float *cosv, float *sinv) {
    const int half = hd / 2;
    double *inv = (double *)malloc((size_t)half * sizeof(double));
    double mscale = 1.0;
    for (int i = 0; i < half; i++) inv[i] = 1.0 / pow((double)theta, (double)(2 * i) / hd);
    if (yarn) {
        const double f = factor, base = theta, orig = orig_ctx;
        double low = hd * log(orig / (beta_fast * 2.0 * MO_PI)) / (2.0 * log(base));
        double high = hd * log(orig / (beta_slow * 2.0 * MO_PI)) / (2.0 * log(base));
        if (truncate) {
            low = floor(low);
            high = ceil(high);
        }
        if (low < 0) low = 0;
        if (high > hd - 1) high = hd - 1;
        if (high == low) high = low + 0.001;
        for (int i = 0; i < half; i++) {
            double ramp = ((double)i - low) / (high - low);
            if (ramp < 0) ramp = 0;
            if (ramp > 1) ramp = 1;
            const double keep = 1.0 - ramp;   /* 1 = the unscaled frequency */
            inv[i] = inv[i] / f * (1.0 - keep) + inv[i] * keep;
        }
        mscale = 0.1 * log(f) + 1.0;
    }
    for (int p = 0; p < ctx; p++)
        for (int i = 0; i < half; i++) {
            const double a = (double)p * inv[i];
            cosv[(size_t)p * half + i] = (float)(cos(a) * mscale);
            sinv[(size_t)p * half + i] = (float)(sin(a) * mscale);
        }
    free(inv);
}

static void mo_rope_rotate(float *v, int heads, int hd, const float *co, const float *si) {
    const int half = hd / 2;
    for (int h = 0; h < heads; h++) {
        float *u = v + (size_t)h * hd;
        for (int i = 0; i < half; i++) {
            const float a = u[i], b = u[i + half];
            u[i] = a * co[i] - b * si[i];
            u[i + half] = b * co[i] + a * si[i];
        }
    }
}

static int mo_wt_matvec(const mh_wt *t, const float *x, float *y) {
    return mo_matvec(t->dt, t->data, t->scales, x, y, t->rows, t->cols);
}

/* attention() (engine/midge.c:341-400) for one token at position pos, host
 * arrays: rmsnorm, q/k/v + biases, per-head q/k RMSNorm if enabled, RoPE,
 * k/v to f16 slot pos % cap, per head: scores q.k * scale over the cached
 * positions, softmax with the sink logit in the denominator, the weighted
 * sum of v; o + bias; x += o. */
int mo_attention(const mh_attn_layer *L, float *x, int pos) {
    const int hd = L->head_dim, nh = L->n_heads, nkv = L->n_kv_heads, half = hd / 2;
    const int kvd = nkv * hd, gq = nh / nkv;
    const int64_t H = L->hidden;
    const int cap = (L->window > 0 && L->window < L->ctx) ? L->window : L->ctx;
    float *xb = (float *)malloc((size_t)H * 4), *q = (float *)malloc((size_t)nh * hd * 4);
    float *k = (float *)malloc((size_t)kvd * 4), *v = (float *)malloc((size_t)kvd * 4);
    float *sc = (float *)malloc((size_t)cap * 4), *ao = (float *)malloc((size_t)nh * hd * 4);
    if (!xb || !q || !k || !v || !sc || !ao) return -1;
    mo_rmsnorm(x, L->attn_norm, xb, H, L->norm_eps);
    mo_wt_matvec(&L->wq, xb, q);
    mo_addbias(q, L->bq, (int64_t)nh * hd);
    mo_wt_matvec(&L->wk, xb, k);
    mo_addbias(k, L->bk, kvd);
    mo_wt_matvec(&L->wv, xb, v);
    mo_addbias(v, L->bv, kvd);
    if (L->qk_norm) {
        for (int h = 0; h < nh; h++) mo_rmsnorm(q + (size_t)h * hd, L->qn, q + (size_t)h * hd, hd, L->norm_eps);
        for (int h = 0; h < nkv; h++) mo_rmsnorm(k + (size_t)h * hd, L->kn, k + (size_t)h * hd, hd, L->norm_eps);
    }
    const float *co = L->rope_cos + (size_t)pos * half, *si = L->rope_sin + (size_t)pos * half;
    mo_rope_rotate(q, nh, hd, co, si);
    mo_rope_rotate(k, nkv, hd, co, si);
    const int slot = pos % cap;
    for (int i = 0; i < kvd; i++) {
        L->kc[(size_t)slot * kvd + i] = mo_to_f16(k[i]);
        L->vc[(size_t)slot * kvd + i] = mo_to_f16(v[i]);
    }
    const int nctx = pos + 1 < cap ? pos + 1 : cap;
    for (int h = 0; h < nh; h++) {
        const float *qh = q + (size_t)h * hd;
        const int kh = h / gq;
        float mx = -1e30f;
        for (int t = 0; t < nctx; t++) {
            const uint16_t *kt = L->kc + (size_t)t * kvd + (size_t)kh * hd;
            float d = 0.f;
            for (int i = 0; i < hd; i++) d += qh[i] * mo_f16_to_f32(kt[i]);
            d *= L->attn_scale;
            sc[t] = d;
            if (d > mx) mx = d;
        }
        const float sinkv = L->sinks ? L->sink[h] : -1e30f;
        if (sinkv > mx) mx = sinkv;
        float den = L->sinks ? expf(sinkv - mx) : 0.f;
        for (int t = 0; t < nctx; t++) {
            sc[t] = expf(sc[t] - mx);
            den += sc[t];
        }
        const float inv = 1.0f / den;
        float *out = ao + (size_t)h * hd;
        for (int i = 0; i < hd; i++) out[i] = 0.f;
        for (int t = 0; t < nctx; t++) {
            const float w = sc[t] * inv;
            const uint16_t *vt = L->vc + (size_t)t * kvd + (size_t)kh * hd;
            for (int i = 0; i < hd; i++) out[i] += w * mo_f16_to_f32(vt[i]);
        }
    }
    mo_wt_matvec(&L->wo, ao, xb);
    mo_addbias(xb, L->bo, H);
    for (int64_t i = 0; i < H; i++) x[i] += xb[i];
    free(xb);
    free(q);
    free(k);
    free(v);
    free(sc);
    free(ao);
    return 0;
}
