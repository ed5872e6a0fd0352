"""A whole decode token on the device (mh_forward_dev: forward(),
engine/midge.c:552-565) against the oracle's forward() composed from its
restatements of wk_row, attention(), moe(), wk_rmsnorm and the lm_head
matvec, over a run of positions past a sliding window (the ring wraps), at
gpt-oss's layer shapes (3 layers: sliding, full, sliding; 32 MXFP4 experts,
top-4; 64/8 heads of 64 with sinks and YaRN).

The expected values come from the compiled reference's scalar build, which
equals the oracle bit for bit (shown here at the first position; the
oracle's scalar C takes seconds per position at these widths). The bar per
position is the reference's own divergence: the same composition on its
AVX2 build against the scalar one. Logits and the final residual are held
to max(1e-3, twice that divergence) in relative L2, and every layer's expert
selection must equal the scalar build's."""
import ctypes as C

import numpy as np
import pytest

from conftest import rel_l2, say
from midge_amd import DT_Q8R, DevBuf, _lib
from midge_amd.moe import MoELayer
from midge_amd.synth import Keys, MoEShape, host_layer_experts, host_router
from oracle import pyoracle as po
from test_oracle_kernels import GPT_OSS_ROPE, AttnHost

pytestmark = pytest.mark.gpu

H, V, NL, CTX, WIN, NPOS = 2880, 2048, 3, 48, 16, 40
SHAPE = MoEShape(hidden=H, ffn=2880, n_experts=32, top_k=4)


class HostModel:
    """The model on host arrays, as the oracle and the reference take it."""

    def __init__(self, seed: int = 21):
        rng = np.random.default_rng(seed)
        self.embed = rng.integers(-127, 128, (V, H), dtype=np.int8)
        self.embed_s = (rng.random(V) * 6e-3 + 2e-3).astype(np.float32)
        self.lm = rng.integers(-127, 128, (V, H), dtype=np.int8)
        self.lm_s = (rng.random(V) * 6e-4 + 2e-4).astype(np.float32)
        self.final_norm = (1.0 + 0.05 * rng.standard_normal(H)).astype(np.float32)
        keys = Keys(seed)
        self.moe = []
        for l in range(NL):
            ex = host_layer_experts(SHAPE, keys, l)
            w, s, b, nw = host_router(SHAPE, keys, l)
            self.moe.append((ex, w, s, b, nw))
        self.seed = seed

    def attn_hosts(self):
        # layer l: sliding (window WIN) on even layers, full on odd ones
        return [AttnHost(hidden=H, nh=64, nkv=8, hd=64, ctx=CTX, window=WIN if l % 2 == 0 else 0, qk_norm=0,
                         sinks=1, seed=self.seed * 10 + l, rope=GPT_OSS_ROPE, wscale=(1e-4, 4e-4))
                for l in range(NL)]


def host_forward(hm: HostModel, attn, tok: int, pos: int, attention_fn, moe_fn):
    """forward() on the host: the composition the device step is held to."""
    x = po.dequant_row(DT_Q8R, hm.embed, hm.embed_s, H, tok)
    sels = []
    for l in range(NL):
        x = attn[l].run(attention_fn, x, pos)
        x, sel = moe_fn(po.layer_struct(SHAPE, *hm.moe[l]), x)[:2]
        sels.append(np.array(sel))
    xb = po.rmsnorm(x, hm.final_norm, 1e-5)
    return x, po.matvec(DT_Q8R, hm.lm, hm.lm_s, xb, V, H), np.array(sels)


def test_forward_dev_vs_oracle(mh):
    if not po.have_ref():
        pytest.fail("the compiled reference (oracle/_ref) is missing: it sets this test's bar")
    hm = HostModel()
    keep = []

    def dev(a):
        d = DevBuf.from_array(np.ascontiguousarray(a))
        keep.append(d)
        return d.ptr

    # the device model: the same weights, uploaded; its own f16 caches
    dev_attn = []
    for ah in hm.attn_hosts():
        L = ah.L
        D = _lib.MhAttnLayer()
        for f, _ in po.MhAttnLayer._fields_:
            if f not in ("wq", "wk", "wv", "wo"):
                setattr(D, f, getattr(L, f))
        for f in ("wq", "wk", "wv", "wo"):
            w = getattr(L, f)
            data = np.ctypeslib.as_array(C.cast(w.data, C.POINTER(C.c_int8)), (w.rows * w.cols,))
            sc = np.ctypeslib.as_array(C.cast(w.scales, C.POINTER(C.c_float)), (w.rows,))
            setattr(D, f, _lib.MhWT(w.dt, w.rows, w.cols, dev(data), dev(sc)))
        for f, n in (("bq", 4096), ("bk", 512), ("bv", 512), ("bo", H), ("attn_norm", H), ("sink", 64)):
            setattr(D, f, dev(np.ctypeslib.as_array(C.cast(getattr(L, f), C.POINTER(C.c_float)), (n,))))
        D.rope_cos, D.rope_sin = dev(ah.co), dev(ah.si)
        D.kc, D.vc = dev(np.zeros_like(ah.kc)), dev(np.zeros_like(ah.vc))
        dev_attn.append(D)
    layers = [MoELayer.host(SHAPE, *hm.moe[l]) for l in range(NL)]
    attn_arr = (_lib.MhAttnLayer * NL)(*dev_attn)
    moe_arr = (_lib.MhMoeLayer * NL)(*[ly.c() for ly in layers])
    desc = _lib.MhModelDesc()
    desc.hidden, desc.vocab, desc.n_layers, desc.norm_eps = H, V, NL, 1e-5
    desc.embed = _lib.MhWT(DT_Q8R, V, H, dev(hm.embed), dev(hm.embed_s))
    desc.lm_head = _lib.MhWT(DT_Q8R, V, H, dev(hm.lm), dev(hm.lm_s))
    desc.final_norm = dev(hm.final_norm)
    desc.attn, desc.moe = attn_arr, moe_arr
    model = C.c_void_p()
    _lib.call("mh_model_create", C.byref(desc), C.byref(model))
    xd, lgd, seld = DevBuf(H * 4), DevBuf(V * 4), DevBuf(NL * 4 * 4)
    keep += [xd, lgd, seld]
    # the reference's scalar kernels (checked against the oracle) and its AVX2 kernels
    ora, sca, avx = hm.attn_hosts(), hm.attn_hosts(), hm.attn_hosts()
    sc_moe = lambda L, x: po.ref_moe_decode(L, x, scalar=True)   # noqa: E731
    toks = np.random.default_rng(5).integers(0, V, NPOS)
    worst = []
    try:
        for pos, tok in enumerate(toks):
            say(f"forward_dev position {pos} token {tok}")
            _lib.call("mh_forward_dev", model, int(tok), pos, xd.ptr, lgd.ptr, seld.ptr, None)
            x_g, lg_g = xd.download(np.float32, (H,)), lgd.download(np.float32, (V,))
            sel_g = seld.download(np.int32, (NL, 4))
            x_o, lg_o, sel_o = host_forward(hm, sca, int(tok), pos, po.ref(scalar=True).ref_attention, sc_moe)
            if pos == 0:
                x_c, lg_c, sel_c = host_forward(hm, ora, int(tok), pos, po.oracle().mo_attention, po.moe_decode)
                assert (lg_c.view(np.uint32) == lg_o.view(np.uint32)).all() and (sel_c == sel_o).all()
            x_r, lg_r, sel_r = host_forward(hm, avx, int(tok), pos, po.ref().ref_attention, po.ref_moe_decode)
            assert (sel_r == sel_o).all(), (pos, "the reference's own builds route differently here")
            assert (sel_g == sel_o).all(), (pos, sel_g, sel_o)
            own_l, own_x = rel_l2(lg_r, lg_o), rel_l2(x_r, x_o)
            e_l, e_x = rel_l2(lg_g, lg_o), rel_l2(x_g, x_o)
            assert e_l <= max(1e-3, 2 * own_l), (pos, e_l, own_l)
            assert e_x <= max(1e-3, 2 * own_x), (pos, e_x, own_x)
            worst.append((e_l, own_l))
    finally:
        _lib.call("mh_model_destroy", model)
        for ly in layers:
            ly.release()
        for d in keep:
            d.free()
    w = np.array(worst)
    say(f"forward_dev: logits rel L2 worst {w[:, 0].max():.3g} (reference's own AVX2 vs scalar: worst "
        f"{w[:, 1].max():.3g}), {NPOS} positions, window {WIN} wrapped")


def test_forward_dev_arguments(mh):
    # argument checks before any device work
    desc = _lib.MhModelDesc()
    model = C.c_void_p()
    assert _lib.load().mh_model_create(None, C.byref(model)) == _lib.MH_E_ARG
    desc.hidden, desc.vocab, desc.n_layers = H, V, 0
    assert _lib.load().mh_model_create(C.byref(desc), C.byref(model)) == _lib.MH_E_ARG
    assert _lib.load().mh_forward_dev(None, 0, 0, None, None, None, None) == _lib.MH_E_ARG
