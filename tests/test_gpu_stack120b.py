"""The gpt-oss-120b expert stack at full size on the GPU (36 layers x 128
MXFP4 experts, ~60 GiB generated in HBM) against the oracle. Teacher-forced
(each layer fed the oracle's input): identical experts and 1e-4 relative L2
at every layer, for the per-layer kernels and for the one-launch decode
step. Chained (36 layers end to end, batch 1 and batch 16): identical experts
up to a near-tie, and the final hidden state as close to the oracle as the
reference's own AVX2 build gets (see the note at TIE). The oracle
regenerates only the experts each layer routes to (the generator is a pure
function of its key), so the CPU never holds the whole table."""
import ctypes as C
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import rel_l2, say
from midge_amd import DevBuf, synth
from midge_amd.moe import Stack
from midge_amd.synth import MoEShape
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
SHAPE = MoEShape(hidden=2880, ffn=2880, n_experts=128, top_k=4, n_layers=36)
SEED = 120


@pytest.fixture(scope="module")
def stack(mh):
    say("120b stack: generating 36 x 128 experts on the device")
    st, bufs, keys = Stack.synthetic(SHAPE, SEED, max_batch=16)
    mh.sync()
    yield st, keys, bufs
    st.destroy()
    for b in bufs:
        b.free()


# Router logits here are ~N(0, 20^2) sums of 2880 int8 x f32 products with a
# condition number of ~40, and the routing weights are a softmax of them, so a
# 1e-5 relative change of the residual moves a layer's output by up to ~1e-2
# relative: 36 chained layers are chaotic at f32 resolution. The reference is
# no exception: its own AVX2 build ends 1.3e-2 (token step 1035) and 2.4e-2
# (step 1001) away from its scalar build after 36 layers, with different
# experts from layer 32 / 12 on, and 5.7e-4 on well-conditioned tokens
# (steps 1018, 4242). So the chained comparison is held to what the
# reference's AVX2 build achieves on the same token (twice its distance to
# the scalar oracle, and never looser than needed below 1e-3), and two
# experts whose oracle logits are closer than TIE (relative) are a near-tie
# where either order is faithful. The teacher-forced tests below remove the
# chaining and hold every layer to 1e-4 with identical experts.
TIE = 1e-3


def oracle_chain(keys, x: np.ndarray, routed: np.ndarray, with_ref: bool):
    """Run token x through the layers on the oracle (the scalar restatement)
    and, if with_ref, on the reference's AVX2 build in lockstep; routed[l] is
    the GPU's selection for this token. Returns (oracle x, ref x or None,
    tie info or None); tie info is set when the GPU's experts differ from the
    oracle's at some layer (then the oracle x is that layer's input)."""
    L = SHAPE.layout
    table = np.zeros(L.layer_stride, np.uint8)          # lazily zeroed pages
    lib = po.oracle()
    bias_c = float(synth.normal_c(synth.EXPERT_BIAS_STD))
    xa = x.copy() if with_ref else None
    for l in range(SHAPE.n_layers):
        w, s, b, nw = synth.host_router(SHAPE, keys, l)
        Ls = po.layer_struct(SHAPE, table, w, s, b, nw)
        xb, sel, _ = po.route_batch(Ls, x[None, :])
        if not (sel[0] == routed[l]).all():
            rl = po.matvec(SHAPE.router_dt, w, s, xb[0], SHAPE.n_experts, SHAPE.hidden) + b
            a = np.setdiff1d(np.union1d(sel[0], routed[l]), np.intersect1d(sel[0], routed[l]))
            pos = [i for i in range(SHAPE.top_k) if sel[0][i] != routed[l][i]]
            involved = sorted(set(a.tolist()) | {int(sel[0][i]) for i in pos} | {int(routed[l][i]) for i in pos})
            vals = np.sort(rl[involved])
            gap = float(np.min(np.diff(vals))) / float(np.max(np.abs(vals))) if len(vals) > 1 else 0.0
            return x, None, {"layer": l, "oracle": sel[0].tolist(), "gpu": routed[l].tolist(),
                             "logits": {int(e): float(rl[e]) for e in involved}, "gap": gap}
        need = set(sel[0].tolist())
        if with_ref:
            _, asel, _ = po.route_batch(Ls, xa[None, :])
            need |= set(asel[0].tolist())

        def gen(e):
            dst = table[e * L.expert_stride:(e + 1) * L.expert_stride]
            return lib.mo_synth_expert(dst.ctypes.data, SHAPE.expert_dt, SHAPE.hidden, SHAPE.ffn,
                                       SHAPE.n_experts, l, e, keys.table, synth.EXPERT_EMIN,
                                       synth.EXPERT_EMAX, bias_c)
        with ThreadPoolExecutor(8) as pool:
            assert all(rc == 0 for rc in pool.map(gen, sorted(need)))
        x, _, _ = po.moe_decode(Ls, x)
        if with_ref:
            xa = po.ref_moe_decode(Ls, xa)[0]
    return x, xa, None


def test_device_table_matches_host_generator(stack):
    st, keys, bufs = stack
    L = SHAPE.layout
    table = bufs[0]
    for (l, e) in ((0, 0), (17, 93), (35, 127)):
        say(f"table expert l={l} e={e}")
        got = table.download(np.uint8, L.expert_stride, offset=(l * SHAPE.n_experts + e) * L.expert_stride)
        want = po.synth_expert(SHAPE.expert_dt, SHAPE.hidden, SHAPE.ffn, SHAPE.n_experts, l, e, keys.table,
                               synth.EXPERT_EMIN, synth.EXPERT_EMAX, float(synth.normal_c(synth.EXPERT_BIAS_STD)))
        assert (got == want).all()


@pytest.mark.parametrize("batch,check,calls", [(1, [0], 3), (16, [0, 5, 9], 1)])
def test_stack_decode_vs_oracle(stack, batch, check, calls):
    st, keys, bufs = stack
    nl, k = SHAPE.n_layers, SHAPE.top_k
    with_ref = po.have_ref()
    full = 0
    for call in range(calls):
        say(f"120b stack decode batch={batch} call={call}")
        X = synth.host_x(SHAPE, keys, batch, step=1000 + 17 * call + batch)
        xd = DevBuf.from_array(X)
        sd = DevBuf(nl * batch * k * 4)
        ud = DevBuf.from_array(np.zeros((nl, SHAPE.n_experts), np.uint32))
        st.decode(xd, batch, sd, None, ud)
        got = xd.download(np.float32, X.shape)
        sel = sd.download(np.int32, (nl, batch, k))
        usage = ud.download(np.uint32, (nl, SHAPE.n_experts))
        for d in (xd, sd, ud):
            d.free()
        for l in range(nl):
            assert (usage[l] == np.bincount(sel[l].ravel(), minlength=SHAPE.n_experts)).all()
        for t in check:
            say(f"oracle chain token {t} of batch {batch} call {call}")
            xr, xa, tie = oracle_chain(keys, X[t].copy(), sel[:, t], with_ref)
            if tie is None:
                err = rel_l2(got[t], xr)
                bar = 1e-3
                if xa is not None:
                    bar = max(bar, 2.0 * rel_l2(xa, xr))
                print(f"[chain] token {t}: gpu {err:.2e}, reference AVX2 build "
                      f"{rel_l2(xa, xr) if xa is not None else float('nan'):.2e}, bar {bar:.2e}", flush=True)
                assert err < bar
                full += 1
            else:
                print(f"[near-tie] token {t}: {tie}", flush=True)
                assert tie["gap"] < TIE, f"routing differs beyond a near-tie: {tie}"
    assert full >= 1, "every checked token hit a near-tie; no full 36-layer comparison was made"


def test_teacher_forced_every_layer(stack):
    """Layer by layer at full size: the GPU's moe() on the oracle's own input
    for that layer must pick the same experts (same order) and produce the
    same residual within 1e-4 relative L2."""
    from midge_amd.moe import moe_dev
    st, keys, bufs = stack
    L = SHAPE.layout
    table = np.zeros(L.layer_stride, np.uint8)
    lib = po.oracle()
    bias_c = float(synth.normal_c(synth.EXPERT_BIAS_STD))
    x = synth.host_x(SHAPE, keys, 1, step=4242)[0]
    xd = DevBuf(SHAPE.hidden * 4)
    sd, wd = DevBuf(SHAPE.top_k * 4), DevBuf(SHAPE.top_k * 4)
    worst = 0.0
    for l in range(SHAPE.n_layers):
        say(f"teacher-forced layer {l}")
        w, s, b, nw = synth.host_router(SHAPE, keys, l)
        Ls = po.layer_struct(SHAPE, table, w, s, b, nw)
        _, sel, _ = po.route_batch(Ls, x[None, :])

        def gen(e):
            dst = table[e * L.expert_stride:(e + 1) * L.expert_stride]
            return lib.mo_synth_expert(dst.ctypes.data, SHAPE.expert_dt, SHAPE.hidden, SHAPE.ffn,
                                       SHAPE.n_experts, l, e, keys.table, synth.EXPERT_EMIN,
                                       synth.EXPERT_EMAX, bias_c)
        with ThreadPoolExecutor(8) as pool:
            assert all(rc == 0 for rc in pool.map(gen, sorted(set(sel[0].tolist()))))
        xd.upload(x)
        moe_dev(st.layers[l], xd, 1, sd, wd)
        got = xd.download(np.float32, SHAPE.hidden)
        gsel = sd.download(np.int32, SHAPE.top_k)
        # the one-launch decode step on a one-layer stack of the same layer
        one = Stack([st.layers[l]], 1)
        xd.upload(x)
        one.decode(xd, 1, sd)
        got1 = xd.download(np.float32, SHAPE.hidden)
        fsel = sd.download(np.int32, SHAPE.top_k)
        one.destroy()
        x, osel, _ = po.moe_decode(Ls, x)
        assert (gsel == osel).all(), (l, gsel, osel)
        assert (fsel == osel).all(), (l, fsel, osel)
        err, err1 = rel_l2(got, x), rel_l2(got1, x)
        worst = max(worst, err, err1)
        assert err < 1e-4 and err1 < 1e-4, (l, err, err1)
    print(f"teacher-forced worst rel L2 {worst:.2e}", flush=True)
    for d in (xd, sd, wd):
        d.free()
