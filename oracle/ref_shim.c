/* ref_shim.c — exports midge's own engine functions for parity checks.
 *
 * TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile against the
 * reference sources where they lie (engine/midge.c with its headers, via
 * -I<reference>/engine), into oracle/_ref/. Nothing of the reference is
 * copied: this file includes engine/midge.c and wraps its static functions
 * (wk_matvec, wk_row, wk_rmsnorm, route_topk, expert_apply, moe, run_bench)
 * in exported ones. Built twice: libmidge_ref.so (the engine as shipped,
 * AVX2+FMA when the CPU has it) and, with -DREF_SCALAR, libmidge_ref_scalar.so
 * whose kernels take the scalar path (MIDGE_NO_SIMD, engine/mkern.h:169-175).
 */
#define main midged_main
#include "midge.c"
#undef main

#include "../include/midge_hip.h"

#ifdef REF_SCALAR
/* wk_have_avx2() reads MIDGE_NO_SIMD once per library; latch it here and
 * restore the environment so other libraries in the process are unaffected. */
__attribute__((constructor)) static void ref_force_scalar(void) {
    const char *prev = getenv("MIDGE_NO_SIMD");
    if (!prev) setenv("MIDGE_NO_SIMD", "1", 1);
    (void)wk_have_avx2();
    if (!prev) unsetenv("MIDGE_NO_SIMD");
}
#endif

int ref_have_avx2(void) { return wk_have_avx2(); }

void ref_matvec(int dt, const void *data, const void *scales, int64_t rows, int64_t cols,
                const float *x, float *y) {
    WT t = { dt, rows, cols, data, scales };
    wk_matvec(&t, x, y);
}

void ref_row(int dt, const void *data, const void *scales, int64_t rows, int64_t cols,
             int64_t r, float *out) {
    WT t = { dt, rows, cols, data, scales };
    wk_row(&t, r, out);
}

void ref_rmsnorm(const float *x, const float *w, float *out, int64_t n, float eps) {
    wk_rmsnorm(x, w, out, n, eps);
}

uint16_t ref_to_f16(float f) { return wk_to_f16(f); }
float ref_f16(uint16_t h) { return wt_f16(h); }

void ref_expert_layout(int dt, int64_t hidden, int64_t ffn, int64_t n_experts,
                       uint64_t off[9], uint64_t *expert_stride, uint64_t *layer_stride) {
    WExLayout L;
    wt_expert_layout(&L, dt, hidden, ffn, n_experts);
    for (int m = 0; m < 3; m++)
        for (int p = 0; p < 3; p++) off[3 * m + p] = L.off[m][p];
    *expert_stride = L.expert_stride;
    *layer_stride = L.layer_stride;
}

/* A one-layer Model whose MoE tensors are the given layer's (layer index 0). */
typedef struct {
    Model m;
    WT router_w;
    const float *router_b, *mlp_norm;
} RefModel;

static int ref_model_init(RefModel *r, const mh_moe_layer *L, int nbatch) {
    memset(r, 0, sizeof(*r));
    Model *m = &r->m;
    Spec *s = &m->s;
    s->hidden = L->hidden; s->ffn = L->ffn; s->n_experts = L->n_experts; s->top_k = L->top_k;
    s->alpha = L->alpha; s->limit = L->limit; s->act_plain = L->act_plain;
    s->router_norm = L->router_norm; s->norm_eps = L->norm_eps; s->n_layers = 1;
    wt_expert_layout(&m->exl, L->expert_dt, L->hidden, L->ffn, L->n_experts);
    m->experts.base = (uint8_t *)L->experts;
    r->router_w.dt = L->router.dt; r->router_w.rows = L->router.rows; r->router_w.cols = L->router.cols;
    r->router_w.data = L->router.data; r->router_w.scales = L->router.scales;
    r->router_b = L->router_b; r->mlp_norm = L->mlp_norm;
    m->router_w = &r->router_w;
    m->router_b = &r->router_b;
    m->mlp_norm = &r->mlp_norm;
    size_t H = (size_t)L->hidden, F = (size_t)L->ffn;
    m->x = malloc(H * 4); m->xb = malloc(H * 4); m->moe = malloc(H * 4);
    m->hb = malloc(F * 4); m->hb2 = malloc(F * 4);
    m->rl = malloc((size_t)L->n_experts * 4);
    m->usage = calloc((size_t)L->n_experts, 4);
    m->bxb = malloc((size_t)nbatch * H * 4);
    m->bw = malloc((size_t)nbatch * MAX_TOPK * 4);
    m->bsel = malloc((size_t)nbatch * MAX_TOPK * sizeof(int));
    return (m->x && m->xb && m->moe && m->hb && m->hb2 && m->rl && m->usage && m->bxb && m->bw && m->bsel) ? 0 : -1;
}

static void ref_model_free(RefModel *r) {
    Model *m = &r->m;
    free(m->x); free(m->xb); free(m->moe); free(m->hb); free(m->hb2); free(m->rl);
    free(m->usage); free(m->bxb); free(m->bw); free(m->bsel);
}

/* One expert's FFN through expert_apply() (engine/midge.c:437-467) with
 * weight 1 into a zeroed output, so y = down(act(gate, up)) + bd exactly. */
int ref_expert_ffn(const mh_moe_layer *L, int e, const float *xb, float *y) {
    RefModel r;
    if (ref_model_init(&r, L, 1)) { ref_model_free(&r); return -5; }
    memset(y, 0, (size_t)L->hidden * 4);
    expert_apply(&r.m, 0, e, xb, 1.0f, y);
    ref_model_free(&r);
    return 0;
}

/* moe() on x[hidden] in place (engine/midge.c:469-549). sel/w come from
 * route_topk() on the same input, which selects identically when every
 * slot fills; usage[n_experts] (may be NULL) receives moe()'s histogram. */
int ref_moe_decode(const mh_moe_layer *L, float *x, int32_t *sel, float *w, uint32_t *usage) {
    RefModel r;
    if (ref_model_init(&r, L, 1)) { ref_model_free(&r); return -5; }
    Model *m = &r.m;
    int isel[MAX_TOPK]; float fw[MAX_TOPK];
    route_topk(m, 0, x, m->xb, isel, fw);
    memcpy(m->x, x, (size_t)L->hidden * 4);
    moe(m, 0);
    memcpy(x, m->x, (size_t)L->hidden * 4);
    for (int i = 0; i < L->top_k; i++) { sel[i] = isel[i]; w[i] = fw[i]; }
    if (usage) memcpy(usage, m->usage, (size_t)L->n_experts * 4);
    ref_model_free(&r);
    return 0;
}

/* The MoE half of forward_batch() (engine/midge.c:591-611) for n tokens on
 * x[n][hidden] in place: route_topk per token, then expert_apply in
 * expert-major order, each into its token's residual. */
int ref_moe_prefill(const mh_moe_layer *L, int n, float *x, int32_t *sel, float *w) {
    RefModel r;
    if (ref_model_init(&r, L, n)) { ref_model_free(&r); return -5; }
    Model *m = &r.m;
    int h = (int)L->hidden, k = L->top_k;
    for (int t = 0; t < n; t++)
        route_topk(m, 0, x + (size_t)t * h, m->bxb + (size_t)t * h,
                   m->bsel + t * MAX_TOPK, m->bw + t * MAX_TOPK);
    for (int e = 0; e < L->n_experts; e++)
        for (int t = 0; t < n; t++)
            for (int i = 0; i < k; i++)
                if (m->bsel[t * MAX_TOPK + i] == e)
                    expert_apply(m, 0, e, m->bxb + (size_t)t * h, m->bw[t * MAX_TOPK + i],
                                 x + (size_t)t * h);
    for (int t = 0; t < n; t++)
        for (int i = 0; i < k; i++) {
            sel[t * k + i] = m->bsel[t * MAX_TOPK + i];
            w[t * k + i] = m->bw[t * MAX_TOPK + i];
        }
    ref_model_free(&r);
    return 0;
}

/* The reference's own kernel bench (engine/midge.c:687-720): prints
 * "BENCH q4g32_gbps=<GiB/s> threads=N". */
int ref_run_bench(void) { return run_bench(); }

/* sample() (engine/midge.c:654-679) on logits[V] with the generator state
 * *rng (updated as the reference's global would be). */
int ref_sample(const float *logits, int64_t V, float temp, float topp, uint64_t *rng) {
    Model m;
    memset(&m, 0, sizeof m);
    m.s.vocab = V;
    m.logits = (float *)logits;
    m.probs = (float *)malloc((size_t)V * sizeof(float));
    if (!m.probs) return -1;
    rng_state = *rng;
    const int tok = sample(&m, temp, topp);
    *rng = rng_state;
    free(m.probs);
    return tok;
}

/* rope_init (engine/midge.c:141-175)'s tables for the given RoPE/YaRN
 * parameters and ctx positions. */
void ref_rope_table(int hd, float theta, int yarn, float factor, float beta_fast, float beta_slow, int orig_ctx,
                    int truncate, int ctx, float *cosv, float *sinv) {
    Model m;
    memset(&m, 0, sizeof m);
    m.s.head_dim = hd;
    m.s.rope_theta = theta;
    m.s.yarn = yarn;
    m.s.yarn_factor = factor;
    m.s.yarn_beta_fast = beta_fast;
    m.s.yarn_beta_slow = beta_slow;
    m.s.yarn_orig_ctx = orig_ctx;
    m.s.yarn_truncate = truncate;
    m.ctx = ctx;
    rope_init(&m);
    memcpy(cosv, m.rope_cos, (size_t)ctx * (hd / 2) * 4);
    memcpy(sinv, m.rope_sin, (size_t)ctx * (hd / 2) * 4);
    free(m.rope_cos);
    free(m.rope_sin);
}

uint16_t ref_to_f16_attn(float f) { return wk_to_f16(f); }

/* attention(m, 0, pos) (engine/midge.c:341-400) for a one-layer Model
 * holding the given layer (host arrays, x in place). */
int ref_attention(const mh_attn_layer *L, float *x, int pos) {
    Model m;
    memset(&m, 0, sizeof m);
    const int nh = L->n_heads, hd = L->head_dim, kvd = L->n_kv_heads * L->head_dim;
    int sliding = L->window > 0;
    WT wq = { L->wq.dt, L->wq.rows, L->wq.cols, L->wq.data, L->wq.scales };
    WT wk = { L->wk.dt, L->wk.rows, L->wk.cols, L->wk.data, L->wk.scales };
    WT wv = { L->wv.dt, L->wv.rows, L->wv.cols, L->wv.data, L->wv.scales };
    WT wo = { L->wo.dt, L->wo.rows, L->wo.cols, L->wo.data, L->wo.scales };
    const float *bq = L->bq, *bk = L->bk, *bv = L->bv, *bo = L->bo;
    const float *an = L->attn_norm, *qn = L->qn, *kn = L->kn, *sk = L->sink;
    uint16_t *kc = L->kc, *vc = L->vc;
    m.s.hidden = L->hidden;
    m.s.n_heads = nh;
    m.s.n_kv_heads = L->n_kv_heads;
    m.s.head_dim = hd;
    m.s.qk_norm = L->qk_norm;
    m.s.sinks = L->sinks;
    m.s.sliding_window = L->window;
    m.s.layer_sliding = &sliding;
    m.s.norm_eps = L->norm_eps;
    m.s.attn_scale = L->attn_scale;
    m.ctx = L->ctx;
    m.wq = &wq;
    m.wk = &wk;
    m.wv = &wv;
    m.wo = &wo;
    m.bq = &bq;
    m.bk = &bk;
    m.bv = &bv;
    m.bo = &bo;
    m.attn_norm = &an;
    m.qn = &qn;
    m.kn = &kn;
    m.sink = &sk;
    m.rope_cos = (float *)L->rope_cos;
    m.rope_sin = (float *)L->rope_sin;
    m.kc = &kc;
    m.vc = &vc;
    m.x = x;
    m.xb = (float *)malloc((size_t)L->hidden * 4);
    m.q = (float *)malloc((size_t)nh * hd * 4);
    m.k = (float *)malloc((size_t)kvd * 4);
    m.v = (float *)malloc((size_t)kvd * 4);
    m.att = (float *)malloc((size_t)nh * L->ctx * 4);
    m.ao = (float *)malloc((size_t)nh * hd * 4);
    int rc = (m.xb && m.q && m.k && m.v && m.att && m.ao) ? 0 : -1;
    if (!rc) attention(&m, 0, pos);
    free(m.xb);
    free(m.q);
    free(m.k);
    free(m.v);
    free(m.att);
    free(m.ao);
    return rc;
}
