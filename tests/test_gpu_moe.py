"""GPU parity of the MoE layer entry points (through the C ABI) against the
oracle and the reference's golden vectors: identical expert selection,
routing weights and outputs within 1e-4 relative L2 (the bar is 1e-3)."""
import numpy as np
import pytest

import make_golden as mg
from conftest import rel_l2, say
from midge_amd import DevBuf, _lib, set_switch, synth
from midge_amd.moe import MoELayer, Stack, expert_major_dev, moe, moe_dev, moe_prefill, moe_prefill_dev, topk_dev
from midge_amd.synth import Keys, MoEShape
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
# routing weights: softmax of logits ~N(0, 20^2) amplifies the router's f32
# reassociation (~1e-6 relative on the logits) to ~1e-4 relative on the weights
WTOL = dict(rtol=1e-3, atol=1e-9)
# The one-launch step's down projection multiplies h as two f16 terms, hi = h
# rounded and lo = h - hi rounded, i.e. h to within 2^-22 (2.4e-7) of its
# magnitude, and sums in another order than the per-layer kernels; through
# the down matrix (its rows' norms times |h| over |y| stay below ~8 for these
# shapes) one layer's output then differs from theirs by at most ~2e-6.
# Chained layers amplify it like any last-bit difference, so the chain is
# held to TOL and the tight bar applies per layer.
SPLIT_TOL = 2e-6
MG = np.load(mg.os.path.join(mg.HERE, "moe.npz"))

SHAPES = {
    "tiny": MoEShape(hidden=64, ffn=64, n_experts=8, top_k=2),
    "mid": MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4),
    "gptoss20b": MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4),
}


_LIVE: list = []


@pytest.fixture(params=["mfma", "gemv"])
def prefill_path(request, mh):
    """The expert-major prefill runs the scaled-MFMA grouped GEMM for MXFP4
    experts; the NO_MFMA switch selects the per-assignment GEMV kernels.
    Both must match the oracle."""
    set_switch("NO_MFMA", request.param == "gemv")
    yield request.param
    set_switch("NO_MFMA", False)


@pytest.fixture(autouse=True)
def _release_layers():
    """Unregister every layer a test built, pass or fail (a stale region would
    collide with a later allocation at the same host address)."""
    yield
    while _LIVE:
        _LIVE.pop().release()


def build(shape: MoEShape, seed: int, layer: int = 0):
    keys = Keys(seed)
    ex = synth.host_layer_experts(shape, keys, layer)
    w, s, b, nw = synth.host_router(shape, keys, layer)
    arrays = (ex, w, s, b, nw)
    lay = MoELayer.host(shape, *arrays)
    _LIVE.append(lay)
    return keys, arrays, lay, po.layer_struct(shape, *arrays)


@pytest.mark.parametrize("name", ["tiny", "mid", "gptoss20b"])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_moe_decode_vs_oracle(mh, name, seed):
    shape = SHAPES[name]
    say(f"moe decode {name} seed={seed}")
    keys, arrays, lay, L = build(shape, seed)
    for step in range(2):
        x = synth.host_x(shape, keys, 1, step=step)[0]
        xo, sel, w = moe(lay, x)
        xr, selr, wr = po.moe_decode(L, x)
        assert (sel == selr).all(), (sel, selr)
        assert np.allclose(w, wr, **WTOL)
        assert rel_l2(xo, xr) < TOL
    lay.release()


@pytest.mark.parametrize("name", list(mg.MOE_CASES))
def test_moe_golden(mh, name):
    hidden, ffn, E, k, seed, npre = (int(v) for v in MG[f"{name}_meta"])
    shape = MoEShape(hidden=hidden, ffn=ffn, n_experts=E, top_k=k)
    say(f"moe golden {name}")
    keys, arrays, lay, L = build(shape, seed)
    x = synth.host_x(shape, keys, 1)[0]
    xo, sel, w = moe(lay, x)
    assert (sel == MG[f"{name}_decode_sel_ref"]).all()
    assert rel_l2(xo, MG[f"{name}_decode_x_ref"]) < TOL
    assert rel_l2(xo, MG[f"{name}_decode_x_ref_scalar"]) < TOL
    X = synth.host_x(shape, keys, npre, step=1)
    xp, selp, wp = moe_prefill(lay, X)
    assert (selp == MG[f"{name}_prefill_sel_ref"]).all()
    assert rel_l2(xp, MG[f"{name}_prefill_x_ref"]) < TOL
    lay.release()


def test_single_expert_ffn_gpt_oss(mh):
    # one gpt-oss expert FFN (gate, up, clamped SwiGLU, down) at 2880: a
    # one-expert top-1 layer adds exactly 1.0 * y to the residual
    shape = MoEShape(hidden=2880, ffn=2880, n_experts=1, top_k=1)
    say("single expert FFN 2880")
    keys, arrays, lay, L = build(shape, 5)
    x = synth.host_x(shape, keys, 1)[0]
    xo, sel, w = moe(lay, x)
    assert sel[0] == 0 and w[0] == 1.0
    xb = po.rmsnorm(x, arrays[4], shape.norm_eps)
    y = po.expert_ffn(L, 0, xb)
    assert rel_l2(xo - x, y) < TOL
    lay.release()


@pytest.mark.parametrize("batch", [2, 5])
def test_moe_dev_batch(mh, batch):
    shape = SHAPES["mid"]
    say(f"moe_dev batch={batch}")
    keys, arrays, lay, L = build(shape, 9)
    X = synth.host_x(shape, keys, batch)
    xd = DevBuf.from_array(X)
    sd, wd = DevBuf(batch * shape.top_k * 4), DevBuf(batch * shape.top_k * 4)
    moe_dev(lay, xd, batch, sd, wd)
    got = xd.download(np.float32, X.shape)
    sel = sd.download(np.int32, (batch, shape.top_k))
    for b in range(batch):
        xr, selr, wr = po.moe_decode(L, X[b])
        assert (sel[b] == selr).all()
        assert rel_l2(got[b], xr) < TOL
    for d in (xd, sd, wd):
        d.free()
    lay.release()


@pytest.mark.parametrize("router_dt", [_lib.DT_Q8R, _lib.DT_F32])
def test_moe_dev_batch16_128_experts(mh, router_dt):
    # the per-layer decode path at batch 16 with 128 experts x 2880 router
    # rows (the 120b router shape), int8 and f32 routers, against the oracle
    shape = MoEShape(hidden=2880, ffn=256, n_experts=128, top_k=4, router_dt=router_dt)
    say(f"moe_dev batch 16, 128 experts, router dt={router_dt}")
    keys = Keys(21)
    ex = synth.host_layer_experts(shape, keys, 0)
    w, s, b, nw = synth.host_router(shape, keys, 0)
    if router_dt == _lib.DT_F32:
        w, s = (w.astype(np.float32) * s[:, None]).astype(np.float32), None
    lay = MoELayer.host(shape, ex, w, s, b, nw)
    _LIVE.append(lay)
    L = po.layer_struct(shape, ex, w, s, b, nw)
    X = synth.host_x(shape, keys, 16)
    xd = DevBuf.from_array(X)
    sd, wd = DevBuf(16 * shape.top_k * 4), DevBuf(16 * shape.top_k * 4)
    moe_dev(lay, xd, 16, sd, wd)
    x1, s1, w1 = (xd.download(np.float32, X.shape), sd.download(np.int32, (16, shape.top_k)),
                  wd.download(np.float32, (16, shape.top_k)))
    for d in (xd, sd, wd):
        d.free()
    for t in range(16):
        xr, selr, wr = po.moe_decode(L, X[t])
        assert (s1[t] == selr).all(), t
        assert np.allclose(w1[t], wr, **WTOL), t
        assert rel_l2(x1[t], xr) < TOL, t
    lay.release()


@pytest.mark.parametrize("expert_dt", [_lib.DT_MXFP4, _lib.DT_Q4G32, _lib.DT_Q8R])
@pytest.mark.parametrize("n_experts", [4, 32])
def test_moe_dev_expert_order_bit_exact(mh, expert_dt, n_experts):
    # Up to 16 tokens, the top-k kernel sorts the assignments by expert and
    # the expert kernels walk them in that order; at 17 tokens they walk them
    # in assignment order. The first 16 tokens of a 17-token call must equal
    # a 16-token call bit for bit, and the oracle. 4 experts x top-4: every
    # token routes to every expert.
    shape = MoEShape(hidden=512, ffn=256, n_experts=n_experts, top_k=4, expert_dt=expert_dt)
    say(f"moe_dev expert order, dt={expert_dt}, {n_experts} experts")
    keys, arrays, lay, L = build(shape, 33)
    X = synth.host_x(shape, keys, 17)
    outs = []
    for n in (16, 17):
        xd = DevBuf.from_array(X[:n])
        sd, wd = DevBuf(n * shape.top_k * 4), DevBuf(n * shape.top_k * 4)
        moe_dev(lay, xd, n, sd, wd)
        outs.append((xd.download(np.float32, (n, shape.hidden)), sd.download(np.int32, (n, shape.top_k)),
                     wd.download(np.float32, (n, shape.top_k))))
        for d in (xd, sd, wd):
            d.free()
    (x16, s16, w16), (x17, s17, w17) = outs
    assert (s16 == s17[:16]).all()
    assert (w16 == w17[:16]).all()
    assert (x16 == x17[:16]).all()
    for t in range(0, 16, 5):
        xr, selr, wr = po.moe_decode(L, X[t])
        assert (s16[t] == selr).all(), t
        assert rel_l2(x16[t], xr) < TOL, t


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_prefill_vs_oracle(mh, name, prefill_path):
    shape = SHAPES[name]
    say(f"prefill {name} 40 tokens, {prefill_path}")
    keys, arrays, lay, L = build(shape, 4)
    X = synth.host_x(shape, keys, 40, step=3)
    xp, selp, wp = moe_prefill(lay, X)
    xr, selr, wr = po.moe_prefill(L, X)
    assert (selp == selr).all()
    assert np.allclose(wp, wr, **WTOL)
    assert rel_l2(xp, xr) < TOL
    # device variant
    xd = DevBuf.from_array(X)
    moe_prefill_dev(lay, xd, 40)
    assert rel_l2(xd.download(np.float32, X.shape), xr) < TOL
    xd.free()
    lay.release()


# Experts with more tokens than one pass of the matrix-core prefill holds (4
# tiles of 32): their tokens run in several passes over the same weights.
@pytest.mark.parametrize("name,n", [("tiny", 1100), ("mid", 700)])
def test_prefill_multipass_vs_oracle(mh, name, n):
    shape = SHAPES[name]
    say(f"prefill multipass {name} {n} tokens")
    keys, arrays, lay, L = build(shape, 6)
    X = synth.host_x(shape, keys, n, step=5)
    xp, selp, wp = moe_prefill(lay, X)
    xr, selr, wr = po.moe_prefill(L, X)
    routed = selr.ravel()
    counts = np.bincount(routed[routed >= 0], minlength=shape.n_experts)
    assert counts.max() > 128, counts   # at least one expert takes two passes
    assert (selp == selr).all()
    assert np.allclose(wp, wr, **WTOL)
    assert rel_l2(xp, xr) < TOL


def test_prefill_non_pow2_scale(mh):
    """A gate scale that is not a power of two: the matrix-core prefill (e8m0
    scales) reports it from the host entry point instead of returning a wrong
    x; the GEMV path multiplies any f16 scale, as the reference does, and
    matches the oracle. The report clears the flag: the next call runs."""
    shape = SHAPES["tiny"]
    say("prefill non-power-of-two scale")
    keys = Keys(8)
    ex = synth.host_layer_experts(shape, keys, 0).copy()
    one_half = np.frombuffer(np.float16(1.5).tobytes(), np.uint8)
    for e in range(shape.n_experts):
        o = shape.layout.offset(0, e, 0, 1)   # gate scales: row 0, group 0
        ex[o:o + 2] = one_half
    w, s, b, nw = synth.host_router(shape, keys, 0)
    arrays = (ex, w, s, b, nw)
    lay = MoELayer.host(shape, *arrays)
    _LIVE.append(lay)
    L = po.layer_struct(shape, *arrays)
    X = synth.host_x(shape, keys, 64, step=1)   # 8+ assignments per expert: the matrix-core path
    with pytest.raises(_lib.MidgeHipError, match="power of two"):
        moe_prefill(lay, X)
    set_switch("NO_MFMA", True)
    try:
        xp, selp, _ = moe_prefill(lay, X)
    finally:
        set_switch("NO_MFMA", False)
    xr, selr, _ = po.moe_prefill(L, X)
    assert (selp == selr).all()
    assert rel_l2(xp, xr) < TOL
    keys2, _, lay2, L2 = build(shape, 4)
    X2 = synth.host_x(shape, keys2, 64, step=2)
    xp2, _, _ = moe_prefill(lay2, X2)
    xr2, _, _ = po.moe_prefill(L2, X2)
    assert rel_l2(xp2, xr2) < TOL


# expert counts on both sides of each ranking instantiation (2, 4 and 16
# logits per lane: E <= 128, <= 256, <= 1024) and the largest top-k (16)
@pytest.mark.parametrize("E,k,router_norm", [(8, 2, 1), (128, 4, 1), (129, 4, 0), (200, 16, 1), (256, 4, 1),
                                             (257, 4, 1), (640, 16, 0), (1024, 4, 1)])
def test_topk_dev_ties_and_edges(mh, E, k, router_norm):
    say(f"topk_dev ties E={E} k={k} norm={router_norm}")
    rng = np.random.default_rng(3 + E)
    n = 64
    logits = rng.standard_normal((n, E)).astype(np.float32)
    logits[::3] = np.round(logits[::3] * 2) / 2          # many exact ties
    logits[5, :] = 0.25                                   # all equal
    logits[6, 3:] = -np.inf                               # fewer eligible than k: unfilled slots
    logits[7, E - 1] = 9.0                                # the winner in the last lane's last slot
    ld = DevBuf.from_array(logits)
    sd, wd = DevBuf(n * k * 4), DevBuf(n * k * 4)
    topk_dev(ld, n, E, k, router_norm, sd, wd)
    sel = sd.download(np.int32, (n, k))
    w = wd.download(np.float32, (n, k))
    for t in range(n):
        s, v = po.topk(logits[t], k, decode=False)
        assert (sel[t] == s).all(), (t, sel[t], s)
        assert np.allclose(w[t], po.router_weights(logits[t], v, router_norm), rtol=1e-5, atol=1e-9)
    for d in (ld, sd, wd):
        d.free()


def test_cfg3_prefill_512_tokens_sampled(mh, prefill_path):
    # expert-major prefill at gpt-oss-20b shape: 512 tokens, 32 experts, top-4,
    # router logits ~N(0,1) given directly; every token on the GPU, a sample of
    # tokens on the oracle (tokens are independent), plus usage counts
    shape = SHAPES["gptoss20b"]
    n = 512
    say(f"cfg3 prefill 512 tokens, {prefill_path}")
    keys, arrays, lay, L = build(shape, 31)
    X = synth.host_x(shape, keys, n, step=7)
    logits = synth.synth_normal(synth.hash64_int(keys.seed, 99), n * shape.n_experts,
                                synth.normal_c(1.0)).reshape(n, shape.n_experts)
    xb = np.stack([po.rmsnorm(X[t], arrays[4], shape.norm_eps) for t in range(n)])
    bufs = [DevBuf.from_array(a) for a in (logits, xb, X)]
    sd, wd = DevBuf(n * 4 * 4), DevBuf(n * 4 * 4)
    topk_dev(bufs[0], n, shape.n_experts, 4, 1, sd, wd)
    expert_major_dev(lay, n, bufs[1], sd, wd, bufs[2])
    got = bufs[2].download(np.float32, X.shape)
    sel = sd.download(np.int32, (n, 4))
    w = wd.download(np.float32, (n, 4))
    counts = np.bincount(sel.ravel(), minlength=32)
    assert counts.sum() == 2048 and counts.min() > 0
    idx = np.random.default_rng(0).choice(n, 12, replace=False)
    for t in idx:
        s, v = po.topk(logits[t], 4, decode=False)
        assert (sel[t] == s).all()
    want = po.expert_major_apply(L, xb[idx], sel[idx], w[idx], X[idx])
    assert rel_l2(got[idx], want) < TOL
    for d in bufs + [sd, wd]:
        d.free()
    lay.release()


def test_stack_chain_vs_oracle(mh):
    shape = MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4, n_layers=5)
    say("stack 5 layers batch 3")
    keys = Keys(123)
    layers, structs, keep = [], [], []
    for l in range(shape.n_layers):
        ex = synth.host_layer_experts(shape, keys, l)
        w, s, b, nw = synth.host_router(shape, keys, l)
        arrays = (ex, w, s, b, nw)
        keep.append(arrays)
        layers.append(MoELayer.host(shape, *arrays))
        _LIVE.append(layers[-1])
        structs.append(po.layer_struct(shape, *arrays))
    st = Stack(layers, max_batch=4)
    batch = 3
    X = synth.host_x(shape, keys, batch)
    xd = DevBuf.from_array(X)
    nl, k = shape.n_layers, shape.top_k
    sd, wd = DevBuf(nl * batch * k * 4), DevBuf(nl * batch * k * 4)
    ud = DevBuf.from_array(np.zeros((nl, shape.n_experts), np.uint32))
    st.decode(xd, batch, sd, wd, ud)
    got = xd.download(np.float32, X.shape)
    sel = sd.download(np.int32, (nl, batch, k))
    usage = ud.download(np.uint32, (nl, shape.n_experts))
    for b in range(batch):
        x = X[b]
        for l in range(nl):
            x, selr, wr = po.moe_decode(structs[l], x)
            assert (sel[l, b] == selr).all(), (l, b)
        assert rel_l2(got[b], x) < TOL
    for l in range(nl):
        assert (usage[l] == np.bincount(sel[l].ravel(), minlength=shape.n_experts)).all()
    st.destroy()
    for d in (xd, sd, wd, ud):
        d.free()
    for lay in layers:
        lay.release()


@pytest.mark.parametrize("router_dt,batch,rows", [(_lib.DT_Q8R, 16, True), (_lib.DT_Q8R, 5, False),
                                                  (_lib.DT_F32, 16, True)],
                         ids=["q8r-b16-rows", "q8r-b5-scratch", "f32-b16-rows"])
def test_stack_batch_fused_layer_boundary(mh, router_dt, batch, rows):
    """Decode of 2-16 tokens through a 3-layer stack at the gpt-oss-20b
    shape: each layer boundary (the previous layer's combine, the norm, the
    router logits, the top-k, the expert order) in one launch against the
    three launches (SPLIT_ROUTE): the same x and xb arithmetic, router dots
    in another order. The logits (magnitude ~20-60 here) then differ in their
    last bits, the weights (their softmax) by up to ~1e-4 relative (7.2e-5
    measured), and x through them: identical selections and usage counts,
    weights within 5e-4 relative and x within TOL per token, with the
    selections in the caller's rows or only in the library's scratch (the
    weights rewritten in place). Against the oracle on three tokens: with
    rows, the same selections, weights within WTOL and x within TOL when the
    oracle's chain applies the kernel's weights (the router's reassociation
    and the expert arithmetic held apart); without, x within WTOL's rtol of
    the oracle's own chain and the usage counts of the oracle's selections
    over every token."""
    shape = MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4, n_layers=3, router_dt=router_dt)
    say(f"fused layer boundary router dt={router_dt} batch={batch} rows={rows}")
    keys = Keys(77)
    layers, structs = [], []
    for l in range(shape.n_layers):
        ex = synth.host_layer_experts(shape, keys, l)
        w, s_, b, nw = synth.host_router(shape, keys, l)
        if router_dt == _lib.DT_F32:
            w, s_ = (w.astype(np.float32) * s_[:, None]).astype(np.float32), None
        layers.append(MoELayer.host(shape, ex, w, s_, b, nw))
        _LIVE.append(layers[-1])
        structs.append(po.layer_struct(shape, ex, w, s_, b, nw))
    st = Stack(layers, max_batch=16)
    nl, k, E = shape.n_layers, shape.top_k, shape.n_experts
    X = synth.host_x(shape, keys, batch, step=5)
    out = {}
    for mode in ("fused", "split"):
        set_switch("SPLIT_ROUTE", mode == "split")
        try:
            xd = DevBuf.from_array(X)
            sd, wd = (DevBuf(nl * batch * k * 4), DevBuf(nl * batch * k * 4)) if rows else (None, None)
            ud = DevBuf.from_array(np.zeros((nl, E), np.uint32))
            st.decode(xd, batch, sd.ptr if sd else None, wd.ptr if wd else None, ud)
            mh.sync()
            out[mode] = (xd.download(np.float32, X.shape),
                         sd.download(np.int32, (nl, batch, k)) if sd else None,
                         wd.download(np.float32, (nl, batch, k)) if wd else None,
                         ud.download(np.uint32, (nl, E)))
            for d in (xd, sd, wd, ud):
                if d:
                    d.free()
        finally:
            set_switch("SPLIT_ROUTE", False)
    st.destroy()
    xf, sf, wf, uf = out["fused"]
    xs, ss, ws, us = out["split"]
    assert (uf == us).all()
    if rows:
        assert (sf == ss).all()
        np.testing.assert_allclose(wf, ws, rtol=5e-4, atol=1e-7)
        for l in range(nl):
            assert (uf[l] == np.bincount(sf[l].ravel(), minlength=E)).all()
    worst = max(rel_l2(xf[t], xs[t]) for t in range(batch))
    say(f"fused vs split layer boundary: worst per-token rel L2 {worst:.3g}")
    for t in range(batch):
        assert rel_l2(xf[t], xs[t]) < TOL, t
    if rows:
        for t in sorted({0, batch // 2, batch - 1}):
            x = X[t][None]
            for l in range(nl):
                xb, selr, wr = po.route_batch(structs[l], x)
                assert (sf[l, t] == selr[0]).all(), (l, t)
                np.testing.assert_allclose(wf[l, t], wr[0], **WTOL)
                x = po.expert_major_apply(structs[l], xb, sf[l, t][None], wf[l, t][None], x)
            assert rel_l2(xf[t], x[0]) < TOL, t
    else:
        so = np.empty((nl, batch, k), np.int32)
        for t in range(batch):
            x = X[t]
            for l in range(nl):
                x, so[l, t], _ = po.moe_decode(structs[l], x)
            assert rel_l2(xf[t], x) < WTOL["rtol"], t
        for l in range(nl):
            assert (uf[l] == np.bincount(so[l].ravel(), minlength=E)).all()


@pytest.mark.parametrize("shape,layers", [
    (MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4), 5),
    (MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 3),
])
def test_stack_fused_step_vs_per_layer_and_oracle(mh, shape, layers):
    """Batch-1 stack decode runs as one launch; it must route exactly as the
    per-layer launches and the oracle do, and agree on x: per layer
    (teacher-forced, each layer fed the oracle's input) within SPLIT_TOL of
    the per-layer kernels, and over the whole chain within TOL of both."""
    import os
    say(f"fused step {shape.hidden}x{shape.ffn} E={shape.n_experts} layers={layers}")
    keys = Keys(77)
    lays, structs = [], []
    for l in range(layers):
        ex = synth.host_layer_experts(shape, keys, l)
        w, s, b, nw = synth.host_router(shape, keys, l)
        lays.append(MoELayer.host(shape, ex, w, s, b, nw))
        _LIVE.append(lays[-1])
        structs.append((po.layer_struct(shape, ex, w, s, b, nw), (ex, w, s, b, nw)))
    st = Stack(lays, max_batch=1)
    k = shape.top_k
    for step in range(3):
        x0 = synth.host_x(shape, keys, 1, step=step)
        out = {}
        for mode in ("fused", "per_layer"):
            if mode == "per_layer":
                set_switch("NO_FUSED", True)
            try:
                xd = DevBuf.from_array(x0)
                sd = DevBuf(layers * k * 4)
                ud = DevBuf.from_array(np.zeros((layers, shape.n_experts), np.uint32))
                st.decode(xd, 1, sd, None, ud)
                mh.sync()
                out[mode] = (xd.download(np.float32, x0.shape)[0], sd.download(np.int32, (layers, k)),
                             ud.download(np.uint32, (layers, shape.n_experts)))
                for d in (xd, sd, ud):
                    d.free()
            finally:
                set_switch("NO_FUSED", False)
        xf, sf, uf = out["fused"]
        xp, sp, up = out["per_layer"]
        assert (sf == sp).all(), (sf, sp)
        assert (uf == up).all()
        assert rel_l2(xf, xp) < TOL
        x = x0[0]
        for l in range(layers):
            x, selr, _ = po.moe_decode(structs[l][0], x)
            assert (sf[l] == selr).all(), (l, sf[l], selr)
        assert rel_l2(xf, x) < TOL
    st.destroy()
    # teacher-forced: one-layer stacks on the oracle's input of each layer
    x = synth.host_x(shape, keys, 1, step=0)[0]
    for l in range(layers):
        xo, selr, _ = po.moe_decode(structs[l][0], x)
        one = Stack([lays[l]], max_batch=1)
        got = {}
        for mode in ("fused", "per_layer"):
            if mode == "per_layer":
                set_switch("NO_FUSED", True)
            try:
                xd, sd = DevBuf.from_array(x[None, :]), DevBuf(k * 4)
                one.decode(xd, 1, sd)
                mh.sync()
                got[mode] = (xd.download(np.float32, (1, shape.hidden))[0], sd.download(np.int32, (k,)))
                xd.free()
                sd.free()
            finally:
                set_switch("NO_FUSED", False)
        one.destroy()
        for mode, (xg, sg) in got.items():
            assert (sg == selr).all(), (l, mode, sg, selr)
        assert rel_l2(got["fused"][0], got["per_layer"][0]) < SPLIT_TOL, l
        assert rel_l2(got["fused"][0], xo) < TOL, l
        x = xo


@pytest.mark.parametrize("n_experts", [32, 128], ids=["gptoss20b", "gptoss120b"])
def test_stack_multilayer_launch_y_words(mh, n_experts):
    """A launch of several layers passes y between its blocks as 32-bit
    words: the f32 rounded to a multiple of 16 units in the last place
    (within 2^-20 relative) with a 4-bit tag in the low bits, both inside
    the launch and into the last layer's combine. One-layer launches, which
    the per-layer bar SPLIT_TOL holds elsewhere, pass full f32 words. Here a
    2-layer launch (device-generated experts at the gpt-oss shape) against
    the per-layer kernels (full f32 everywhere) on the same inputs: the same
    experts in both layers, and x after the two layers within twice the
    per-layer bar widened by the words' own rounding, 2 (SPLIT_TOL + 2^-20)
    (measured: up to 4.7e-6 at 128 experts)."""
    shape = MoEShape(hidden=2880, ffn=2880, n_experts=n_experts, top_k=4, n_layers=2)
    say(f"2-layer launch vs per-layer kernels, E={n_experts}")
    st, bufs, keys = Stack.synthetic(shape, 91 + n_experts, 1)
    k = shape.top_k
    worst = 0.0
    for step in range(8):
        x0 = synth.host_x(shape, keys, 1, step=step)
        out = {}
        for mode in ("fused", "per_layer"):
            set_switch("NO_FUSED", mode == "per_layer")
            try:
                xd, sd = DevBuf.from_array(x0), DevBuf(2 * k * 4)
                st.decode(xd, 1, sd)
                mh.sync()
                out[mode] = (xd.download(np.float32, x0.shape)[0], sd.download(np.int32, (2, k)))
                xd.free()
                sd.free()
            finally:
                set_switch("NO_FUSED", False)
        assert (out["fused"][1] == out["per_layer"][1]).all(), (step, out["fused"][1], out["per_layer"][1])
        err = rel_l2(out["fused"][0], out["per_layer"][0])
        worst = max(worst, err)
        assert err < 2 * (SPLIT_TOL + 2.0 ** -20), (step, err)
    say(f"2-layer launch E={n_experts}: worst rel L2 {worst:.3g} against the per-layer kernels")
    st.destroy()
    for d in bufs:
        d.free()


@pytest.mark.parametrize("shape", [
    MoEShape(hidden=2880, ffn=2880, n_experts=1, top_k=1),
    MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4),
    MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4),
], ids=["one_expert", "mid", "gptoss20b"])
def test_stack_apply_vs_expert_major_and_oracle(mh, shape):
    """expert_apply with the routing given (mh_stack_apply_dev, engine/
    midge.c:436-467 per slot in the expert-major loop's order, 595-611): the
    one-launch kernel against the per-layer expert-major kernels (SPLIT_TOL)
    and the oracle's expert-major loop (TOL), over slot orders that are not
    ascending, a repeated expert and unfilled slots, three calls in a row on
    one stack."""
    import os
    say(f"stack apply {shape.hidden}x{shape.ffn} E={shape.n_experts} k={shape.top_k}")
    keys = Keys(91)
    ex = synth.host_layer_experts(shape, keys, 0)
    w, s, b, nw = synth.host_router(shape, keys, 0)
    lay = MoELayer.host(shape, ex, w, s, b, nw)
    _LIVE.append(lay)
    L = po.layer_struct(shape, ex, w, s, b, nw)
    st = Stack([lay], max_batch=1)
    k, E = shape.top_k, shape.n_experts
    rng = np.random.default_rng(5)
    sels = [[0], [0], [-1]] if k == 1 else [[E - 1, 2, 7, 0], [3, 3, 1, -1], [5, -1, -1, 5]]
    for sel in sels:
        sel = np.array(sel, np.int32)
        wv = rng.uniform(0.05, 1.0, k).astype(np.float32)
        xb = rng.standard_normal(shape.hidden).astype(np.float32)
        x0 = rng.standard_normal(shape.hidden).astype(np.float32)
        out = {}
        for mode in ("fused", "per_layer"):
            if mode == "per_layer":
                set_switch("NO_FUSED", True)
            try:
                bufs = [DevBuf.from_array(a) for a in (xb, sel, wv, x0)]
                st.apply(0, *bufs)
                mh.sync()
                out[mode] = bufs[3].download(np.float32, (shape.hidden,))
                for d in bufs:
                    d.free()
            finally:
                set_switch("NO_FUSED", False)
        want = po.expert_major_apply(L, xb[None], sel[None], wv[None], x0[None])[0]
        if (sel < 0).all():
            assert np.array_equal(out["fused"], x0) and np.array_equal(out["per_layer"], x0)
            continue
        # the one-launch kernel's down sums in another order: its result is
        # not bit-identical to the per-layer kernels' (so it did run)
        assert not np.array_equal(out["fused"], out["per_layer"])
        assert rel_l2(out["fused"], out["per_layer"]) < SPLIT_TOL, sel
        assert rel_l2(out["fused"], want) < TOL, sel
        assert rel_l2(out["per_layer"], want) < TOL, sel
    # xb aliasing x: the one-launch kernel would read xb while other blocks
    # write x, so the call falls back to the per-layer kernels (x += w
    # expert(x)); against the oracle with the same aliasing
    sel = np.array(sels[0], np.int32)
    wv = np.full(k, 0.5, np.float32)
    x0 = rng.standard_normal(shape.hidden).astype(np.float32)
    bufs = [DevBuf.from_array(a) for a in (x0, sel, wv)]
    st.apply(0, bufs[0], bufs[1], bufs[2], bufs[0])
    mh.sync()
    got = bufs[0].download(np.float32, (shape.hidden,))
    for d in bufs:
        d.free()
    want = po.expert_major_apply(L, x0[None], sel[None], wv[None], x0[None])[0]
    assert rel_l2(got, want) < TOL
    st.destroy()


def _composed_decode(shape, arrays, L, x):
    """moe() for one token composed from the oracle's pieces (router, stable
    top-k, weights, each filled slot's expert FFN, the combine in selection
    order), which also covers unfilled slots (expert -1, skipped)."""
    ex, w, s, b, nw = arrays
    xb = po.rmsnorm(x, nw, shape.norm_eps)
    rl = po.matvec(shape.router_dt, w, s, xb, shape.n_experts, shape.hidden) + b
    sel, val = po.topk(rl, shape.top_k, decode=True)
    wr = po.router_weights(rl, val, 1)
    moe = np.zeros(shape.hidden, np.float32)
    for i, e in enumerate(np.asarray(sel)):
        if e >= 0:
            moe = moe + np.float32(wr[i]) * po.expert_ffn(L, int(e), xb)
    return x + moe, np.asarray(sel)


@pytest.mark.parametrize("shape,batch,case", [
    (MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 2, "random"),
    (MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 7, "random"),
    (MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 16, "random"),
    (MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 16, "same"),
    (MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4), 16, "random"),
    (MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4), 9, "unfilled"),
], ids=["20b-b2", "20b-b7", "20b-b16", "20b-b16-one-run", "mid-b16", "mid-b9-unfilled"])
def test_stack_batch_grouped_kernels(mh, shape, batch, case):
    """Decode of 2-16 tokens through a stack: the expert-grouped matrix-core
    kernels (the default; assignments grouped by expert, groups of up to 4,
    each routed expert's weights read once per group) against the
    per-assignment GEMVs (the BATCH_GEMV switch) within SPLIT_TOL and the
    oracle within TOL per token, with identical selections. "same": every
    token equal, so each routed expert has a run of `batch` assignments
    (groups of 4 and a remainder); "unfilled": only two experts can be
    routed, so two slots per token are unfilled (their y is 0)."""
    say(f"grouped {shape.hidden}x{shape.ffn} E={shape.n_experts} batch={batch} {case}")
    keys = Keys(64)
    ex = synth.host_layer_experts(shape, keys, 0)
    w, s, b, nw = synth.host_router(shape, keys, 0)
    if case == "unfilled":
        b = np.full_like(b, -1e31)
        b[[2, 11]] = 0.0
    lay = MoELayer.host(shape, ex, w, s, b, nw)
    _LIVE.append(lay)
    L = po.layer_struct(shape, ex, w, s, b, nw)
    st = Stack([lay], max_batch=16)
    k = shape.top_k
    x0 = synth.host_x(shape, keys, batch, step=3)
    if case == "same":
        x0 = np.ascontiguousarray(np.repeat(x0[:1], batch, axis=0))
    out = {}
    for mode in ("grouped", "gemv"):
        if mode == "gemv":
            set_switch("BATCH_GEMV", True)
        try:
            xd, sd = DevBuf.from_array(x0), DevBuf(batch * k * 4)
            st.decode(xd, batch, sd)
            mh.sync()
            out[mode] = (xd.download(np.float32, x0.shape), sd.download(np.int32, (batch, k)))
            xd.free()
            sd.free()
        finally:
            set_switch("BATCH_GEMV", False)
    st.destroy()
    xf, sf = out["grouped"]
    xg, sg = out["gemv"]
    assert (sf == sg).all()
    # the two paths sum in different orders: not bit-identical (so the
    # matrix-core path ran), within SPLIT_TOL per token
    assert not np.array_equal(xf, xg)
    worst = max(rel_l2(xf[t], xg[t]) for t in range(batch))
    say(f"grouped vs GEMV: worst per-token rel L2 {worst:.3g}")
    for t in range(batch):
        assert rel_l2(xf[t], xg[t]) < SPLIT_TOL, t
    for t in sorted({0, batch // 2, batch - 1}):
        want, selr = _composed_decode(shape, (ex, w, s, b, nw), L, x0[t])
        assert (sf[t] == selr).all(), (t, sf[t], selr)
        assert rel_l2(xf[t], want) < TOL, t
    if case == "unfilled":
        assert (sf[:, 2:] == -1).all()


FUSED_VARIANTS = {
    "softmax_all_logits": dict(router_norm=0),
    "plain_silu": dict(act_plain=1),
    "q4g32_experts": dict(expert_dt=_lib.DT_Q4G32),
    "f32_router": dict(router_dt=_lib.DT_F32),
}


@pytest.mark.parametrize("path", ["mfma", "valu"])
@pytest.mark.parametrize("variant", list(FUSED_VARIANTS))
def test_stack_fused_step_variants(mh, variant, path):
    """The one-launch step for the layer variants the reference supports
    beside gpt-oss's (softmax over all logits, plain SiLU, q4 g32 experts, an
    f32 router), on the matrix-core and the vector-ALU down path where the
    variant allows the former: exact selection and x against the oracle."""
    import dataclasses
    import os
    shape = dataclasses.replace(MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4), **FUSED_VARIANTS[variant])
    layers = 3
    say(f"fused step variant {variant} path {path}")
    keys = Keys(314)
    lays, structs, keep = [], [], []
    for l in range(layers):
        ex = synth.host_layer_experts(shape, keys, l)
        w, s, b, nw = synth.host_router(shape, keys, l)
        if shape.router_dt == _lib.DT_F32:
            w, s = (w.astype(np.float32) * s[:, None]).astype(np.float32), None
        keep.append((ex, w, s, b, nw))
        lays.append(MoELayer.host(shape, ex, w, s, b, nw))
        _LIVE.append(lays[-1])
        structs.append(po.layer_struct(shape, ex, w, s, b, nw))
    if path == "valu":
        set_switch("NO_MFMA", True)
    try:
        st = Stack(lays, max_batch=1)
        k = shape.top_k
        for step in range(3):
            x0 = synth.host_x(shape, keys, 1, step=step)
            xd = DevBuf.from_array(x0)
            sd = DevBuf(layers * k * 4)
            st.decode(xd, 1, sd, None, None)
            mh.sync()
            xf = xd.download(np.float32, x0.shape)[0]
            sf = sd.download(np.int32, (layers, k))
            for d in (xd, sd):
                d.free()
            x = x0[0]
            for l in range(layers):
                x, selr, _ = po.moe_decode(structs[l], x)
                assert (sf[l] == selr).all(), (step, l, sf[l], selr)
            assert rel_l2(xf, x) < TOL, (step, rel_l2(xf, x))
        st.destroy()
    finally:
        set_switch("NO_MFMA", False)


def test_stack_fused_step_ties_and_unfilled_slots(mh):
    """Routing edge cases through the one-launch step, against the per-layer
    launches and the oracle: 128 experts whose router rows repeat every 8
    (exact ties in groups of 16: the top 4 are the lowest indices of the best
    group, with equal weights), and a layer where only two experts' logits
    exceed -1e30 (slots 2 and 3 unfilled: expert -1, weight 0)."""
    import os
    shape = MoEShape(hidden=256, ffn=192, n_experts=128, top_k=4)
    keys = Keys(91)
    lays, structs, host = [], [], []
    for l in range(3):
        ex = synth.host_layer_experts(shape, keys, l)
        w, s, b, nw = synth.host_router(shape, keys, l)
        if l == 1:
            w = np.ascontiguousarray(w.reshape(shape.n_experts, -1)[np.arange(shape.n_experts) % 8]).reshape(w.shape)
            s, b = s[np.arange(shape.n_experts) % 8].copy(), b[np.arange(shape.n_experts) % 8].copy()
        if l == 2:
            b = np.full_like(b, -1e31)
            b[[3, 77]] = 0.0
        lays.append(MoELayer.host(shape, ex, w, s, b, nw))
        _LIVE.append(lays[-1])
        structs.append(po.layer_struct(shape, ex, w, s, b, nw))
        host.append((ex, w, s, b, nw))
    st = Stack(lays, max_batch=1)
    k = shape.top_k
    x0 = synth.host_x(shape, keys, 1, step=5)
    out = {}
    for mode in ("fused", "per_layer"):
        if mode == "per_layer":
            set_switch("NO_FUSED", True)
        try:
            xd = DevBuf.from_array(x0)
            sd, wd = DevBuf(3 * k * 4), DevBuf(3 * k * 4)
            st.decode(xd, 1, sd, wd)
            mh.sync()
            out[mode] = (xd.download(np.float32, x0.shape)[0], sd.download(np.int32, (3, k)),
                         wd.download(np.float32, (3, k)))
            for d in (xd, sd, wd):
                d.free()
        finally:
            set_switch("NO_FUSED", False)
    st.destroy()
    xf, sf, wf = out["fused"]
    xp, sp, wp = out["per_layer"]
    x = x0[0]
    for l in range(2):
        x, selr, wr = po.moe_decode(structs[l], x)
        say(f"layer {l}: fused {sf[l].tolist()} oracle {np.asarray(selr).tolist()}")
        assert (sf[l] == selr).all() and (sp[l] == selr).all(), (l, sf[l], sp[l], selr)
        np.testing.assert_allclose(wf[l], wr, rtol=1e-5, atol=1e-7)
    # layer 2: the reference would index expert -1 for an unfilled slot
    # (engine/midge.c:515-517), so its moe() is undefined here and the oracle
    # refuses; this library skips unfilled slots. Composed from the oracle's
    # pieces: router, stable top-k, weights, and the filled experts' FFNs.
    ex, w, s, b, nw = host[2]
    xb = po.rmsnorm(x, nw, shape.norm_eps)
    rl = po.matvec(shape.router_dt, w, s, xb, shape.n_experts, shape.hidden) + b
    selr, val = po.topk(rl, k, decode=True)
    wr = po.router_weights(rl, val, 1)
    assert (sf[2] == selr).all() and (sp[2] == selr).all(), (sf[2], sp[2], selr)
    np.testing.assert_allclose(wf[2], wr, rtol=1e-5, atol=1e-7)
    moe = np.zeros_like(x)
    for i in range(k):
        if selr[i] >= 0:
            moe = (moe + np.float32(wr[i]) * po.expert_ffn(structs[2], int(selr[i]), xb)).astype(np.float32)
    x = (x + moe).astype(np.float32)
    g = sf[1][0] % 8
    assert sf[1].tolist() == [g, g + 8, g + 16, g + 24]      # ties go to the lower index
    assert np.allclose(wf[1], 0.25)
    assert sf[2][2:].tolist() == [-1, -1] and (wf[2][2:] == 0).all()
    assert sorted(sf[2][:2].tolist()) == [3, 77]
    assert rel_l2(xf, xp) < 1e-5 and rel_l2(xf, x) < TOL
