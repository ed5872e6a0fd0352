// mh_forward.hip — forward() (engine/midge.c:552-565) on the device: one
// decode token through every layer with the residual x resident in HBM.
//
//   embedding   wk_row of the token's row into x (mh_dequant_dev)
//   per layer   attention() (mh_attention_dev: rmsnorm, q/k/v, rope, the
//               f16 cache, GQA softmax with sinks, o + residual), then
//               moe() as the one-launch kernel for that layer of the MoE
//               stack (routing, the routed experts' clamped SwiGLU FFNs, the
//               weighted sum and x += moe)
//   logits      final rmsnorm and the lm_head GEMV (when asked)
//
// Every launch goes to the library stream in order; nothing comes back to
// the host.
#include <vector>

#include "mh_internal.h"

struct mh_model {
    mh_model_desc d;
    std::vector<mh_attn_layer> attn;
    std::vector<mh_moe_layer> moe;
    mh_stack *stack = nullptr;
    float *xb = nullptr;   // device [hidden]: the final rmsnorm's output
    uint64_t xb_bytes = 0;
};

namespace mh {
int stack_decode_layer(mh_stack *st, int l, float *x, int32_t *sel, float *w, uint32_t *usage);
}

using namespace mh;

extern "C" {

int mh_model_create(const mh_model_desc *d, mh_model **out) {
    clear_error();
    if (!d || !out || !d->attn || !d->moe || !d->final_norm)
        return fail(MH_E_ARG, "mh_model_create: NULL descriptor, output or layer arrays");
    if (d->n_layers < 1 || d->hidden < 1 || d->vocab < 1)
        return fail(MH_E_ARG, "mh_model_create: %d layers, hidden %lld, vocab %lld", d->n_layers,
                    (long long)d->hidden, (long long)d->vocab);
    if (d->embed.rows != d->vocab || d->embed.cols != d->hidden || d->lm_head.rows != d->vocab ||
        d->lm_head.cols != d->hidden)
        return fail(MH_E_ARG, "mh_model_create: embed / lm_head shapes do not match vocab x hidden");
    for (int l = 0; l < d->n_layers; l++)
        if (d->attn[l].hidden != d->hidden || d->moe[l].hidden != d->hidden)
            return fail(MH_E_ARG, "mh_model_create: layer %d's hidden size differs from the model's", l);
    MH_TRY(require_init());
    DevWT e, h;
    MH_TRY(resolve_wt(&d->embed, &e, "model embed"));
    MH_TRY(resolve_wt(&d->lm_head, &h, "model lm_head"));
    const void *fn;
    MH_TRY(resolve_weight(d->final_norm, (uint64_t)d->hidden * 4, &fn, "model final norm"));
    mh_model *m = new mh_model();
    m->d = *d;
    m->attn.assign(d->attn, d->attn + d->n_layers);
    m->moe.assign(d->moe, d->moe + d->n_layers);
    m->d.attn = m->attn.data();
    m->d.moe = m->moe.data();
    int rc = mh_stack_create(m->moe.data(), d->n_layers, 1, &m->stack);
    if (!rc) {
        m->xb_bytes = (uint64_t)d->hidden * 4;
        void *p = nullptr;
        rc = dev_alloc(&p, m->xb_bytes, "model xb");
        m->xb = (float *)p;
    }
    if (rc) {
        if (m->stack) mh_stack_destroy(m->stack);
        delete m;
        return rc;
    }
    *out = m;
    return MH_OK;
}

int mh_forward_dev(mh_model *m, int32_t token, int32_t pos, float *x, float *logits, int32_t *sel, float *w) {
    clear_error();
    if (!m || !x) return fail(MH_E_ARG, "mh_forward_dev: NULL model or x");
    const mh_model_desc &d = m->d;
    if (token < 0 || token >= d.vocab)
        return fail(MH_E_ARG, "mh_forward_dev: token %d out of range [0, %lld)", token, (long long)d.vocab);
    MH_TRY(require_init());
    const int k = d.moe[0].top_k;
    MH_TRY(resolve_dev(x, (uint64_t)d.hidden * 4, "mh_forward_dev x"));
    if (logits) MH_TRY(resolve_dev(logits, (uint64_t)d.vocab * 4, "mh_forward_dev logits"));
    if (sel) MH_TRY(resolve_dev(sel, (uint64_t)d.n_layers * k * 4, "mh_forward_dev sel"));
    if (w) MH_TRY(resolve_dev(w, (uint64_t)d.n_layers * k * 4, "mh_forward_dev w"));
    MH_TRY(mh_dequant_dev(&d.embed, token, 1, x));
    for (int l = 0; l < d.n_layers; l++) {
        MH_TRY(mh_attention_dev(&d.attn[l], x, pos));
        MH_TRY(stack_decode_layer(m->stack, l, x, sel ? sel + (size_t)l * k : nullptr, w ? w + (size_t)l * k : nullptr,
                                  nullptr));
    }
    if (logits) {
        MH_TRY(mh_rmsnorm_dev(x, d.final_norm, m->xb, d.hidden, d.norm_eps, 1));
        MH_TRY(mh_matvec_dev(&d.lm_head, m->xb, logits, 1));
    }
    return MH_OK;
}

int mh_model_destroy(mh_model *m) {
    clear_error();
    if (!m) return MH_OK;
    if (m->stack) mh_stack_destroy(m->stack);
    if (m->xb) {
        (void)hipStreamSynchronize(stream());
        dev_release(m->xb, m->xb_bytes);
    }
    delete m;
    return MH_OK;
}

}  // extern "C"
