"""Write the golden vectors in tests/golden/*.npz from the reference engine.

The reference engine is compiled from its own sources by `make -C oracle ref`
(oracle/_ref/, built only where the reference checkout exists). Inputs come
from the seeded generators in midge_amd.synth, so a fixture stores the
seeds, the shapes and the reference's outputs, not the weights. Outputs are
recorded from both of the reference's kernel paths: AVX2+FMA ("ref") and
its scalar fallback ("ref_scalar", MIDGE_NO_SIMD).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from midge_amd import DT_F32, DT_MXFP4, DT_Q4G32, DT_Q8R, synth  # noqa: E402
from oracle import pyoracle as po  # noqa: E402

KERNEL_SEED = 1001


def kernel_inputs(dt: int, rows: int, cols: int, seed: int):
    """Seeded tensor + x for one dtype (shared with the tests)."""
    k = synth.Keys(seed)
    x = synth.synth_normal(k.x, cols, synth.normal_c(1.0))
    if dt == DT_F32:
        return synth.synth_normal(k.table, rows * cols, synth.normal_c(0.05)), None, x
    if dt == DT_Q8R:
        return (synth.synth_i8(k.table, rows * cols),
                synth.synth_uniform(k.router_s, rows, 1e-3, synth.uniform_c(1e-3, 1e-2)), x)
    data = synth.synth_bytes(k.table, rows * cols // 2)
    if dt == DT_MXFP4:
        sc = synth.synth_scales(k.router_s, rows * cols // 32, -8, -4)
    else:   # q4g32: f16 scales in [2^-8, 2^-4) with random mantissas
        u = synth.synth_uniform(k.router_s, rows * cols // 32, 2.0 ** -8, synth.uniform_c(2.0 ** -8, 2.0 ** -4))
        sc = u.astype(np.float16).view(np.uint16)
    return data, sc, x


KERNEL_CASES = [(DT_F32, 13, 2880), (DT_Q8R, 37, 2880), (DT_Q4G32, 37, 2880), (DT_MXFP4, 37, 2880),
                (DT_Q8R, 11, 4096), (DT_MXFP4, 5, 64)]


def gen_kernels(out: dict) -> None:
    for i, (dt, rows, cols) in enumerate(KERNEL_CASES):
        data, sc, x = kernel_inputs(dt, rows, cols, KERNEL_SEED + i)
        out[f"k{i}_meta"] = np.array([dt, rows, cols, KERNEL_SEED + i], np.int64)
        out[f"k{i}_y_ref"] = po.ref_matvec(dt, data, sc, x, rows, cols, scalar=False)
        out[f"k{i}_y_ref_scalar"] = po.ref_matvec(dt, data, sc, x, rows, cols, scalar=True)
        out[f"k{i}_rows"] = np.stack([po.ref_row(dt, data, sc, rows, cols, r) for r in (0, rows // 2, rows - 1)])


MOE_CASES = {
    # name: (shape, seed, n_prefill)
    "tiny": (synth.MoEShape(hidden=64, ffn=64, n_experts=8, top_k=2), 7, 6),
    "mid": (synth.MoEShape(hidden=256, ffn=192, n_experts=16, top_k=4), 11, 9),
    "gptoss20b": (synth.MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4), 2026, 8),
}


def gen_moe(out: dict) -> None:
    for name, (shape, seed, npre) in MOE_CASES.items():
        keys = synth.Keys(seed)
        ex = synth.host_layer_experts(shape, keys, 0)
        w, s, b, nw = synth.host_router(shape, keys, 0)
        L = po.layer_struct(shape, ex, w, s, b, nw)
        x = synth.host_x(shape, keys, 1)[0]
        for tag, scalar in (("ref", False), ("ref_scalar", True)):
            xo, sel, wt, usage = po.ref_moe_decode(L, x, scalar=scalar)
            out[f"{name}_decode_x_{tag}"] = xo
            out[f"{name}_decode_sel_{tag}"] = sel
            out[f"{name}_decode_w_{tag}"] = wt
        # one expert FFN on the normed input (the single-expert configuration)
        xb = po.ref_rmsnorm(x, nw, shape.norm_eps)
        out[f"{name}_ffn0_y_ref"] = po.ref_expert_ffn(L, 0, xb)
        out[f"{name}_ffn0_y_ref_scalar"] = po.ref_expert_ffn(L, 0, xb, scalar=True)
        X = synth.host_x(shape, keys, npre, step=1)
        for tag, scalar in (("ref", False), ("ref_scalar", True)):
            xo, sel, wt = po.ref_moe_prefill(L, X, scalar=scalar)
            out[f"{name}_prefill_x_{tag}"] = xo
            out[f"{name}_prefill_sel_{tag}"] = sel
            out[f"{name}_prefill_w_{tag}"] = wt
        out[f"{name}_meta"] = np.array([shape.hidden, shape.ffn, shape.n_experts, shape.top_k, seed, npre], np.int64)


def main() -> int:
    if not po.have_ref():
        print("reference engine not built (make -C oracle ref)", file=sys.stderr)
        return 1
    out: dict = {}
    gen_kernels(out)
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **out)
    out = {}
    gen_moe(out)
    np.savez_compressed(os.path.join(HERE, "moe.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
