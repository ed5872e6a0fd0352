/* midge_hip.h — C ABI of libmidge_hip, the MI355X (gfx950) implementation of
 * midge's quantized mixture-of-experts hot path.
 *
 * The reference engine has no exported symbols: its kernels are static
 * functions in engine/mkern.h and its MoE layer is static in engine/midge.c.
 * Each entry point below replaces one of those functions (cited per
 * declaration); include/midge_hip_kern.h maps the reference's own names onto
 * them so engine/midge.c can call the GPU without edits to its kernel calls.
 *
 * Conventions
 *  - Every function returns 0 (MH_OK) or a negative MH_E_* code; the message
 *    of the last failure on the calling thread is mh_last_error().
 *  - Weight pointers (mh_wt.data/.scales, expert tables, router, norm and
 *    bias vectors) may be host pointers inside a range registered with
 *    mh_register_region() — they are translated to the device copy at the
 *    same offset — or device pointers from mh_alloc(). Anything else is
 *    rejected with MH_E_UNREGISTERED before a kernel is launched.
 *  - Functions without the _dev suffix take host activations and are
 *    synchronous, like the reference kernels they replace. Functions with
 *    the _dev suffix take device activations and are asynchronous on the
 *    library stream (mh_set_stream / mh_get_stream).
 *  - The library is single-caller: calls from several threads must be
 *    serialised by the caller (the reference engine is single-threaded at
 *    these call sites, engine/midge.c:762-836).
 */
#ifndef MIDGE_HIP_H
#define MIDGE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tensor dtypes, numbered as engine/mten.h:42 (DT_F32 .. DT_MXFP4). */
enum { MH_DT_F32 = 0, MH_DT_Q8R = 1, MH_DT_Q4G32 = 2, MH_DT_MXFP4 = 3 };

/* Status codes. */
enum {
    MH_OK = 0,
    MH_E_ARG = -1,          /* bad argument (NULL, negative size, k > experts ...) */
    MH_E_DTYPE = -2,        /* unknown or unsupported dtype */
    MH_E_NOINIT = -3,       /* mh_init() not called / failed */
    MH_E_HIP = -4,          /* HIP runtime error (message has the HIP error string) */
    MH_E_NOMEM = -5,        /* device or host allocation failed / over MIDGE_HIP_MAX_BYTES */
    MH_E_UNREGISTERED = -6, /* pointer neither in a registered region nor device memory */
    MH_E_RANGE = -7,        /* index or byte range out of bounds */
    MH_E_UNSUPPORTED = -8   /* valid input this build does not handle (message says which) */
};

/* Tensor view, field-for-field the reference's WT (engine/mten.h:67-72). */
typedef struct mh_wt {
    int dt;
    int64_t rows, cols;
    const void *data;
    const void *scales;     /* NULL for f32 */
} mh_wt;

/* One MoE layer: everything moe() / route_topk() / expert_apply() read from
 * the reference's Model for one layer (engine/midge.c:46-87, 404-549).
 * off[] and expert_stride are wt_expert_layout()'s (engine/mten.h:136-150):
 * off[3*m + p] for m = gate, up, down and p = data, scales, bias. */
typedef struct mh_moe_layer {
    int64_t hidden, ffn;
    int32_t n_experts, top_k;       /* top_k <= 16 (engine/midge.c:44) */
    float alpha, limit, norm_eps;   /* clamped-SwiGLU params, rmsnorm eps */
    int32_t act_plain;              /* 1: silu(g)*u; 0: gpt-oss clamp */
    int32_t router_norm;            /* 1: softmax over selected; 0: full softmax */
    int32_t expert_dt;              /* MH_DT_MXFP4 or MH_DT_Q4G32 */
    uint64_t expert_stride;
    uint64_t off[9];
    const void *experts;            /* this layer's expert 0 */
    mh_wt router;                   /* n_experts x hidden, f32 or q8r */
    const float *router_b;          /* [n_experts] */
    const float *mlp_norm;          /* [hidden] */
} mh_moe_layer;

/* ------------------------------------------------------------ runtime */

/* Select the HIP device, create the library stream. Idempotent. */
int mh_init(int device);
/* Free every region, allocation, plan and the stream. */
int mh_shutdown(void);
/* Message of the last failure on this thread ("" if none). */
const char *mh_last_error(void);
/* Use `stream` (a hipStream_t, NULL = the library's own) for all _dev work. */
int mh_set_stream(void *stream);
void *mh_get_stream(void);
/* Wait for all work on the library stream, then report (and clear) a failure
 * that asynchronous work raised (a timed-out wait of a one-launch kernel, a
 * prefill scale e8m0 cannot hold). The entry points on host buffers (mh_moe,
 * mh_moe_prefill, mh_matvec, mh_row) make the same check before they return. */
int mh_sync(void);
/* Path switches for comparisons (tests, benchmarks), all off by default.
 * mh_init reads each from the environment once (MIDGE_HIP_<name> set and not
 * "0"); this call changes one at run time: "NO_MFMA" (no matrix-core
 * kernels in the batched int8 GEMV, the prefill and the decode step),
 * "NO_FUSED" (stack decode as per-layer launches), "ATTN_SPLIT" (attention
 * as four launches), "COOP" (the one-launch decode step launched
 * cooperatively), "Q8_NO_ROWS" (long batched int8 GEMVs on the
 * register-operand kernel). MH_E_ARG for an unknown name. No counterpart in
 * the reference: its only comparable knob is MIDGE_NO_SIMD, read once at
 * start-up (engine/mkern.h:75-93). */
int mh_set_switch(const char *name, int on);

/* Kernel timing. While enabled, every kernel launch is bracketed by HIP
 * events on its stream and accounted under its kernel name ("gemv",
 * "expert_gu", "expert_down", "topk", "rmsnorm", "combine_decode",
 * "combine_prefill", ...). mh_profile_query waits for the recorded launches
 * and returns the total milliseconds and launch count for `name`.
 * The reference's only timing is run_bench (engine/midge.c:687-720). */
int mh_profile_enable(int on);
int mh_profile_reset(void);
int mh_profile_query(const char *name, double *total_ms, uint64_t *launches);

/* Upload [host_base, host_base+bytes) to one HBM allocation with identical
 * offsets; later calls translate pointers inside the range. This is how the
 * experts.midge data region (engine/mten.h:84-98, base = align64(8+hl))
 * becomes the resident expert table. *dev_base receives the device copy. */
int mh_register_region(const void *host_base, uint64_t bytes, void **dev_base);
/* Drop a registered region (by host base). */
int mh_unregister_region(const void *host_base);

/* Device memory for _dev callers. The optional cap MIDGE_HIP_MAX_BYTES
 * (environment, bytes) makes allocations beyond it fail with MH_E_NOMEM. */
int mh_alloc(uint64_t bytes, void **dev);
int mh_free(void *dev);
int mh_h2d(void *dev_dst, const void *host_src, uint64_t bytes);   /* synchronous */
int mh_d2h(void *host_dst, const void *dev_src, uint64_t bytes);   /* synchronous */

/* ------------------------------------------------------ kernel level */

/* y[rows] = W x[cols]. Replaces wk_matvec (engine/mkern.h:180-198) for all
 * four dtypes; x and y are host arrays. Unlike the reference (which leaves y
 * untouched for an unknown dtype), an unknown dtype returns MH_E_DTYPE. */
int mh_matvec(const mh_wt *t, const float *x, float *y);

/* out[cols] = row r of W, dequantized. Replaces wk_row (engine/mkern.h:201-236).
 * Bit-exact with the reference (code 8 of MXFP4 is -0.0). */
int mh_row(const mh_wt *t, int64_t r, float *out);

/* y[b][rows] = W x[b][cols] for b < batch (device arrays, row-major, one
 * token per row). batch = 1 is wk_matvec on device memory; batch > 1 is the
 * reference's per-token loop of wk_matvec calls (engine/midge.c:586-590,
 * 613-618) done in one pass. For int8 (q8r) weights with batch >= 2 and cols
 * a multiple of 64 (<= 65536), each weight byte is read once per 32 tokens
 * on the int8 matrix cores, x written as three int8 digits under a power of
 * two per token (exact int32 sums; x rounded to 2^-22 of its largest
 * element; a token holding inf/nan gets the plain f32 sum). */
int mh_matvec_dev(const mh_wt *t, const float *x, float *y, int batch);

/* out[n][cols] = rows r0 .. r0+n-1 of W dequantized (device out). */
int mh_dequant_dev(const mh_wt *t, int64_t r0, int64_t n, float *out);

/* out[b] = rmsnorm(x[b]) * w for b < batch, length n each (engine/mkern.h:238-243). */
int mh_rmsnorm_dev(const float *x, const float *w, float *out, int64_t n, float eps, int batch);

/* One attention layer of the trunk for one token, attention()
 * (engine/midge.c:341-400): rmsnorm, q/k/v GEMVs + biases, optional per-head
 * q/k RMSNorm, RoPE from the given tables, k/v into the f16 cache slot
 * pos % cap, GQA softmax attention over the cached positions (with an
 * optional per-head sink logit), the o GEMV + bias, and the residual add.
 * Device arrays. cap = window if 0 < window < ctx (a sliding layer, a ring of
 * window slots), else ctx. */
typedef struct {
    int64_t hidden;
    int32_t n_heads, n_kv_heads, head_dim;
    int32_t ctx;                        /* positions the rope tables hold */
    int32_t window;                     /* sliding window of this layer, 0 = none */
    int32_t qk_norm, sinks;             /* flags (Spec.qk_norm, Spec.sinks) */
    float norm_eps, attn_scale;
    mh_wt wq, wk, wv, wo;               /* [nh*hd][hidden], [nkv*hd][hidden] x2, [hidden][nh*hd] */
    const float *bq, *bk, *bv, *bo;     /* biases */
    const float *attn_norm;             /* [hidden] */
    const float *qn, *kn;               /* [head_dim] (qk_norm), else NULL */
    const float *sink;                  /* [n_heads] (sinks), else NULL */
    const float *rope_cos, *rope_sin;   /* [ctx][head_dim / 2] (rope_init, midge.c:141-175) */
    uint16_t *kc, *vc;                  /* [cap][n_kv_heads * head_dim] f16 as wk_to_f16 writes */
} mh_attn_layer;

/* attention(m, layer, pos) on device x[hidden], in place. */
int mh_attention_dev(const mh_attn_layer *L, float *x, int pos);

/* sample() (engine/midge.c:654-679) on device logits[V]: the next token into
 * device out[0]. temp <= 0 gives the first maximum; otherwise the
 * temperature softmax, the smallest set of most probable tokens whose
 * probability reaches topp, and the token where their running sum reaches
 * u * (their sum). u is the caller's uniform draw in [0, 1), drawn where the
 * reference draws rng_f() (engine/midge.c:641-646), i.e. only when temp > 0.
 * Equal probabilities are ordered by token id (the reference's sort order
 * for equal keys under glibc's qsort). */
int mh_sample_dev(const float *logits, int64_t V, float temp, float topp, float u, int32_t *out);

/* mh_sample_dev on a fixed workspace that the library holds on each GPU
 * from mh_init() until the process ends (1,273,888 bytes: a 225,312-byte
 * head of counters, histograms and candidates, and 2^18 floats): the call allocates
 * nothing (no hipMalloc, hipFree or event), for callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation. No counterpart in the reference. V is limited to
 * 1..262144 (MH_E_ARG beyond). Every call on a GPU shares that GPU's
 * workspace: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller. Same results as
 * mh_sample_dev. */
int mh_sample_dev_static(const float *logits, int64_t V, float temp, float topp, float u, int32_t *out);

/* ------------------------------------------------------- layer level */

/* Decode MoE layer for one token, in place on host x[hidden]: rmsnorm,
 * router, stable top-k, routing weights, the routed experts' clamped-SwiGLU
 * FFNs, weighted sum in selection order and the residual add. Replaces
 * moe() (engine/midge.c:469-549). sel[top_k] / w[top_k] (host, may be NULL)
 * receive the routing for the caller's usage bookkeeping (midge.c:517-518).
 * The layer runs as one launch of the decode-step kernel where a one-layer
 * plan fits it (made on the layer's first call and kept, keyed by its
 * tensors, until mh_shutdown), else as the per-layer launches. */
int mh_moe(const mh_moe_layer *L, float *x, int32_t *sel, float *w);

/* moe() for `batch` independent tokens on device x[batch][hidden], in place.
 * sel/w (device, [batch][top_k], may be NULL). At batch 1 the one-launch
 * kernel as for mh_moe. */
int mh_moe_dev(const mh_moe_layer *L, float *x, int batch, int32_t *sel, float *w);

/* The MoE half of forward_batch() (engine/midge.c:591-611) for n tokens on
 * host x[n][hidden], in place: route_topk() per token (midge.c:404-434), then
 * every routed expert applied expert-major, each token's contributions
 * added into its residual in ascending expert order (expert_apply,
 * midge.c:437-467). sel/w (host [n][top_k], may be NULL) get the routing. */
int mh_moe_prefill(const mh_moe_layer *L, int n, float *x, int32_t *sel, float *w);

/* mh_moe_prefill on device x[n][hidden]. */
int mh_moe_prefill_dev(const mh_moe_layer *L, int n, float *x, int32_t *sel, float *w);

/* route_topk()'s selection and weights from given logits[n][n_experts]
 * (engine/midge.c:410-433), device arrays; sel/w are [n][k]. */
int mh_topk_dev(const float *logits, int n, int n_experts, int k, int router_norm,
                int32_t *sel, float *w);

/* The expert-major block of forward_batch (engine/midge.c:595-611) with the
 * routing already made: for each token t, x[t] += w[t][i] * expert_{sel[t][i]}(xb[t])
 * in ascending expert order. Device arrays; xb is the normed input. */
int mh_expert_major_dev(const mh_moe_layer *L, int n, const float *xb,
                        const int32_t *sel, const float *w, float *x);

/* ---------------------------------------------- multi-layer decode plan */

/* A device-resident stack of MoE layers (the MoE half of forward()'s layer
 * loop, engine/midge.c:557-560): pointers are resolved and scratch sized once
 * at creation. */
typedef struct mh_stack mh_stack;
int mh_stack_create(const mh_moe_layer *layers, int n_layers, int max_batch, mh_stack **out);
/* Run every layer's moe() for `batch` tokens on device x[batch][hidden].
 * sel/w (device [n_layers][batch][top_k], may be NULL) receive the routing;
 * usage (device u32 [n_layers][n_experts], may be NULL) is incremented per
 * routed expert as the reference's usage histogram is (midge.c:517-518). */
int mh_stack_decode(mh_stack *s, float *x, int batch, int32_t *sel, float *w, uint32_t *usage);
/* expert_apply (engine/midge.c:436-467) for one token with the routing
 * given, on layer `layer` of the stack: x += w[i] * expert_{sel[i]}(xb) for
 * the top_k slots in ascending expert order (slot order among equal ids, as
 * the expert-major loop adds, midge.c:595-611); a slot whose expert is
 * outside [0, n_experts) adds nothing. Device xb[hidden] (normed input, not
 * overlapping x), sel/w[top_k], x[hidden]. mh_expert_major_dev with n = 1,
 * in one launch where the stack's decode plan holds (the down projection
 * then sums in another order: within 2e-6 relative of the per-layer
 * kernels). */
int mh_stack_apply_dev(mh_stack *s, int layer, const float *xb, const int32_t *sel, const float *w, float *x);
int mh_stack_destroy(mh_stack *s);

/* ----------------------------------------------------- decode token */

/* forward() (engine/midge.c:552-565) with every tensor and activation on the
 * device: a whole decode token. The model descriptor names the engine's
 * tensors (Model, engine/midge.c:65-87): the embedding and lm_head matrices,
 * the final norm, and per layer the attention layer (its f16 k/v cache and
 * rope tables included, as mh_attention_dev takes them) and the MoE layer.
 * Every layer's MoE must share hidden, ffn, experts and top-k. */
typedef struct {
    int64_t hidden, vocab;
    int32_t n_layers;
    float norm_eps;
    mh_wt embed;                        /* [vocab][hidden], any dtype (wk_row) */
    mh_wt lm_head;                      /* [vocab][hidden] */
    const float *final_norm;            /* [hidden] */
    const mh_attn_layer *attn;          /* [n_layers] */
    const mh_moe_layer *moe;            /* [n_layers] */
} mh_model_desc;

typedef struct mh_model mh_model;
/* Resolves and checks the descriptor (the arrays it points to are copied),
 * and plans the MoE layers' one-launch kernel. */
int mh_model_create(const mh_model_desc *d, mh_model **out);
/* One token at position pos (its k/v go to each layer's cache slot pos %
 * cap): x[hidden] (device) <- embedding row `token`, then per layer
 * attention() and moe(); if logits (device [vocab]) is not NULL, the final
 * rmsnorm and the lm_head GEMV. sel / w (device [n_layers][top_k]) get each
 * layer's routing, or NULL. Asynchronous on the library stream. */
int mh_forward_dev(mh_model *m, int32_t token, int32_t pos, float *x, float *logits, int32_t *sel, float *w);
int mh_model_destroy(mh_model *m);

#ifdef __cplusplus
}
#endif
#endif /* MIDGE_HIP_H */
