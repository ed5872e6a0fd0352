"""The oracle against the golden vectors the reference engine wrote
(tests/golden/make_golden.py): bit-exact with the reference's scalar path,
within f32 reassociation of its AVX2+FMA path, identical expert selection."""
import numpy as np
import pytest

import make_golden as mg
from conftest import rel_l2
from midge_amd import synth
from oracle import pyoracle as po

KG = np.load(mg.os.path.join(mg.HERE, "kernels.npz"))
MG = np.load(mg.os.path.join(mg.HERE, "moe.npz"))


@pytest.mark.parametrize("i", range(len(mg.KERNEL_CASES)))
def test_kernels_golden(i):
    dt, rows, cols, seed = (int(v) for v in KG[f"k{i}_meta"])
    data, sc, x = mg.kernel_inputs(dt, rows, cols, seed)
    y = po.matvec(dt, data, sc, x, rows, cols)
    assert (y.view(np.uint32) == KG[f"k{i}_y_ref_scalar"].view(np.uint32)).all()
    assert rel_l2(y, KG[f"k{i}_y_ref"]) < 1e-5
    for j, r in enumerate((0, rows // 2, rows - 1)):
        d = po.dequant_row(dt, data, sc, cols, r)
        assert (d.view(np.uint32) == KG[f"k{i}_rows"][j].view(np.uint32)).all()


def moe_case(name):
    hidden, ffn, E, k, seed, npre = (int(v) for v in MG[f"{name}_meta"])
    shape = synth.MoEShape(hidden=hidden, ffn=ffn, n_experts=E, top_k=k)
    keys = synth.Keys(seed)
    ex = synth.host_layer_experts(shape, keys, 0)
    w, s, b, nw = synth.host_router(shape, keys, 0)
    arrays = (ex, w, s, b, nw)
    return shape, keys, arrays, po.layer_struct(shape, *arrays), npre


@pytest.mark.parametrize("name", list(mg.MOE_CASES))
def test_moe_golden(name):
    shape, keys, arrays, L, npre = moe_case(name)
    x = synth.host_x(shape, keys, 1)[0]
    xo, sel, w = po.moe_decode(L, x)
    assert (sel == MG[f"{name}_decode_sel_ref_scalar"]).all()
    assert (sel == MG[f"{name}_decode_sel_ref"]).all()
    assert (xo.view(np.uint32) == MG[f"{name}_decode_x_ref_scalar"].view(np.uint32)).all()
    assert (w.view(np.uint32) == MG[f"{name}_decode_w_ref_scalar"].view(np.uint32)).all()
    assert rel_l2(xo, MG[f"{name}_decode_x_ref"]) < 1e-4
    xb = po.rmsnorm(x, arrays[4], shape.norm_eps)
    y = po.expert_ffn(L, 0, xb)
    assert (y.view(np.uint32) == MG[f"{name}_ffn0_y_ref_scalar"].view(np.uint32)).all()
    X = synth.host_x(shape, keys, npre, step=1)
    xo, sel, w = po.moe_prefill(L, X)
    assert (sel == MG[f"{name}_prefill_sel_ref_scalar"]).all()
    assert (sel == MG[f"{name}_prefill_sel_ref"]).all()
    assert (xo.view(np.uint32) == MG[f"{name}_prefill_x_ref_scalar"].view(np.uint32)).all()
    assert rel_l2(xo, MG[f"{name}_prefill_x_ref"]) < 1e-4


def test_prefill_equals_per_token_decode_up_to_order():
    # expert-major prefill computes per token what decode computes (midge.c:568-574),
    # only the summation order of the routed contributions differs
    shape, keys, arrays, L, npre = moe_case("mid")
    X = synth.host_x(shape, keys, npre, step=1)
    xp, selp, wp = po.moe_prefill(L, X)
    for t in range(npre):
        xd, seld, wd = po.moe_decode(L, X[t])
        assert (seld == selp[t]).all()
        assert rel_l2(xd, xp[t]) < 1e-6


def test_planted_mistake_is_caught():
    # a plausible oracle mistake (hi/lo nibble swap) must break the golden match
    name = "tiny"
    shape, keys, arrays, L, npre = moe_case(name)
    ex = arrays[0].copy()
    lay = shape.layout
    for e in range(shape.n_experts):
        for m in range(3):
            o = e * lay.expert_stride + lay.off[3 * m]
            n = lay.rows[m] * lay.cols[m] // 2
            blob = ex[o:o + n]
            ex[o:o + n] = (blob >> 4) | (blob << 4)
    L2 = po.layer_struct(shape, ex, *arrays[1:])
    x = synth.host_x(shape, keys, 1)[0]
    xo, _, _ = po.moe_decode(L2, x)
    assert rel_l2(xo, MG[f"{name}_decode_x_ref_scalar"]) > 1e-3
