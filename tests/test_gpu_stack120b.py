"""The gpt-oss-120b expert stack at full size on the GPU (36 layers x 128
MXFP4 experts, ~60 GiB generated in HBM) against the oracle: for sampled
tokens of a batch-1 and a batch-16 decode step, every layer's experts must be
identical and the final hidden state within 1e-4 relative L2. The oracle
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
# condition number of ~40, so the ~1e-5 relative drift that f32
# reassociation leaves in the residual after a dozen chained layers moves
# them by ~4e-4 relative. Two experts whose oracle logits are closer than
# TIE (relative) are a near-tie: either order is faithful, and the chained
# trajectories differ from there on. The teacher-forced test below removes
# the chaining and requires identical experts at every layer.
TIE = 1e-3


def oracle_chain(keys, x: np.ndarray, routed: np.ndarray):
    """Run token x through the layers on the oracle; routed[l] is the GPU's
    selection for this token (it only decides which experts to generate; the
    oracle routes by itself). Returns (x, layers matched, tie info or None)."""
    L = SHAPE.layout
    table = np.zeros(L.layer_stride, np.uint8)          # lazily zeroed pages
    lib = po.oracle()
    bias_c = float(synth.normal_c(synth.EXPERT_BIAS_STD))
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
            return x, l, {"layer": l, "oracle": sel[0].tolist(), "gpu": routed[l].tolist(),
                          "logits": {int(e): float(rl[e]) for e in involved}, "gap": gap}
        need = sorted(set(sel[0].tolist()))

        def gen(e):
            dst = table[e * L.expert_stride:(e + 1) * L.expert_stride]
            return lib.mo_synth_expert(dst.ctypes.data, SHAPE.expert_dt, SHAPE.hidden, SHAPE.ffn,
                                       SHAPE.n_experts, l, e, keys.table, synth.EXPERT_EMIN,
                                       synth.EXPERT_EMAX, bias_c)
        with ThreadPoolExecutor(8) as pool:
            assert all(rc == 0 for rc in pool.map(gen, need))
        x, _, _ = po.moe_decode(Ls, x)
    return x, SHAPE.n_layers, None


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
            xr, matched, tie = oracle_chain(keys, X[t].copy(), sel[:, t])
            if tie is None:
                assert rel_l2(got[t], xr) < 1e-3   # 36 chained layers; the bar is 1e-3
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
        x, osel, _ = po.moe_decode(Ls, x)
        assert (gsel == osel).all(), (l, gsel, osel)
        err = rel_l2(got, x)
        worst = max(worst, err)
        assert err < 1e-4, (l, err)
    print(f"teacher-forced worst rel L2 {worst:.2e}", flush=True)
    for d in (xd, sd, wd):
        d.free()
