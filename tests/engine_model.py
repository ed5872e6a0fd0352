"""A small gpt-oss-shaped model in midge's container format, for running the
reference engine's own host (its stdin/stdout protocol, engine/midge.c:
15-24) on the CPU kernels and on libmidge_hip.

The per-layer shapes are gpt-oss's (hidden 2880, 64 query / 8 kv heads of
64, 32 MXFP4 experts of ffn 2880, top-4, clamped SwiGLU, sliding window 128
on alternate layers, attention sinks, YaRN rope); the depth and the
vocabulary are cut down so the CPU engine finishes in seconds. Weights are
seeded random numbers in the converter's formats (tools/convert.py: q8r
dense matrices, f32 router, norms, biases and sinks, MXFP4 experts with f16
power-of-two scales), written through midge_amd.container:

    dense.midge    embed, lm_head, final_norm, L{i}.attn.{q,k,v,o}[_b],
                   L{i}.attn.{norm,sinks}, L{i}.mlp.norm, L{i}.router.{w,b},
                   with the spec in its header
    experts.midge  every layer's experts at wt_expert_layout() offsets
"""
from __future__ import annotations

import os

import numpy as np

from midge_amd import DT_F32, DT_MXFP4, DT_Q8R
from midge_amd.container import DenseFile, write_experts
from midge_amd.layout import ExpertLayout


def spec(n_layers: int = 4, vocab: int = 8192, hidden: int = 2880, n_experts: int = 32) -> dict:
    """gpt-oss's layer shapes at a cut-down depth and vocabulary."""
    return {
        "arch": "gpt-oss", "hidden": hidden, "n_layers": n_layers, "n_heads": 64, "n_kv_heads": 8,
        "head_dim": 64, "vocab": vocab, "norm_eps": 1e-05,
        "moe": {"experts": n_experts, "top_k": 4, "ffn": 2880, "act": "swiglu_clamp", "alpha": 1.702,
                "limit": 7.0},
        "attn": {"layer_types": ["sliding_attention" if i % 2 == 0 else "full_attention" for i in range(n_layers)],
                 "sliding_window": 128, "sinks": True, "scale": 0.125},
        "rope": {"theta": 150000.0,
                 "yarn": {"factor": 32.0, "beta_fast": 32.0, "beta_slow": 1.0, "orig_ctx": 4096, "truncate": False}},
    }


def tiny_spec() -> dict:
    """The shapes of the reference's own end-to-end validation model
    (tools/make_tiny.py:23-50): hidden 64, 2 layers, 4 query / 2 kv heads of
    16, 4 experts of ffn 64, top-2, sliding window 8, vocabulary 128."""
    return {
        "arch": "gpt-oss", "hidden": 64, "n_layers": 2, "n_heads": 4, "n_kv_heads": 2, "head_dim": 16,
        "vocab": 128, "norm_eps": 1e-05,
        "moe": {"experts": 4, "top_k": 2, "ffn": 64, "act": "swiglu_clamp", "alpha": 1.702, "limit": 7.0},
        "attn": {"layer_types": ["sliding_attention", "full_attention"], "sliding_window": 8, "sinks": True,
                 "scale": 0.25},
        "rope": {"theta": 150000.0,
                 "yarn": {"factor": 4.0, "beta_fast": 32.0, "beta_slow": 1.0, "orig_ctx": 64, "truncate": False}},
    }


# The reference's validation prompt (tools/validate.py:39) for the tiny model.
TINY_IDS = [1, 17, 42, 5, 99, 3, 77, 12, 63, 8, 120, 31]


def _q8r(rng, rows: int, cols: int, smin: float, smax: float) -> tuple[bytes, bytes]:
    w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    s = (smin + (smax - smin) * rng.random(rows)).astype(np.float32)
    return w.tobytes(), s.tobytes()


def _vec(rng, n: int, mean: float = 0.0, std: float = 0.02) -> np.ndarray:
    return (mean + std * rng.standard_normal(n)).astype(np.float32)


def write_model(out_dir: str, seed: int = 7, tiny: bool = False, **shape) -> dict:
    """Writes dense.midge and experts.midge into out_dir; returns the spec.
    tiny: the reference's validation shapes, with its weight magnitudes
    (N(0, 0.5) matrices, tools/make_tiny.py:53-54) in the container's
    formats."""
    sp = tiny_spec() if tiny else spec(**shape)
    H, V, L = sp["hidden"], sp["vocab"], sp["n_layers"]
    nh, nkv, hd = sp["n_heads"], sp["n_kv_heads"], sp["head_dim"]
    E, F = sp["moe"]["experts"], sp["moe"]["ffn"]
    rng = np.random.default_rng(seed)
    os.makedirs(out_dir, exist_ok=True)
    d = DenseFile(sp)
    # q8r scales: uniform int8 of standard deviation 0.5 for the tiny model;
    # otherwise chosen so every projection's output stays of order one
    u = 0.5 * 3 ** 0.5 / 127
    sc = dict(embed=(u, u), lm=(u, u), attn=(u, u)) if tiny else dict(embed=(2e-3, 8e-3), lm=(2e-4, 8e-4),
                                                                       attn=(1e-4, 4e-4))
    vs = 0.1 if tiny else 0.02          # bias spread
    d.add_matrix("embed", DT_Q8R, V, H, *_q8r(rng, V, H, *sc["embed"]))
    d.add_matrix("lm_head", DT_Q8R, V, H, *_q8r(rng, V, H, *sc["lm"]))
    d.add_vector("final_norm", _vec(rng, H, 1.0, 0.1 if tiny else 0.05))
    for i in range(L):
        d.add_matrix(f"L{i}.attn.q", DT_Q8R, nh * hd, H, *_q8r(rng, nh * hd, H, *sc["attn"]))
        d.add_matrix(f"L{i}.attn.k", DT_Q8R, nkv * hd, H, *_q8r(rng, nkv * hd, H, *sc["attn"]))
        d.add_matrix(f"L{i}.attn.v", DT_Q8R, nkv * hd, H, *_q8r(rng, nkv * hd, H, *sc["attn"]))
        d.add_matrix(f"L{i}.attn.o", DT_Q8R, H, nh * hd, *_q8r(rng, H, nh * hd, *sc["attn"]))
        for nm, n in (("q_b", nh * hd), ("k_b", nkv * hd), ("v_b", nkv * hd), ("o_b", H)):
            d.add_vector(f"L{i}.attn.{nm}", _vec(rng, n, 0.0, vs))
        d.add_vector(f"L{i}.attn.norm", _vec(rng, H, 1.0, 0.1 if tiny else 0.05))
        d.add_vector(f"L{i}.attn.sinks", _vec(rng, nh, 0.0, 1.0))
        d.add_vector(f"L{i}.mlp.norm", _vec(rng, H, 1.0, 0.1 if tiny else 0.05))
        d.add_matrix(f"L{i}.router.w", DT_F32, E, H, _vec(rng, E * H, 0.0, 0.5 if tiny else 0.02).tobytes())
        d.add_vector(f"L{i}.router.b", _vec(rng, E, 0.0, 0.2 if tiny else 0.1))
    d.write(os.path.join(out_dir, "dense.midge"))
    # experts: uniform nibbles, scales 2^e as f16 with e uniform in [-8, -4]
    # ([-4, -2] for the tiny model), biases N(0, 0.02) (0.1), at the
    # deterministic layout's offsets
    lay = ExpertLayout(DT_MXFP4, H, F, E)
    elo, ehi = (-4, -2) if tiny else (-8, -4)

    def layer_table(li: int) -> np.ndarray:
        t = np.zeros(lay.layer_stride, np.uint8)
        for e in range(E):
            for m in range(3):
                rows, cols = lay.rows[m], lay.cols[m]
                o = lay.offset(0, e, m, 0)
                t[o:o + rows * cols // 2] = np.frombuffer(rng.bytes(rows * cols // 2), np.uint8)
                sc = ((rng.integers(elo, ehi + 1, rows * cols // 32) + 15) << 10).astype(np.uint16)
                o = lay.offset(0, e, m, 1)
                t[o:o + sc.nbytes] = sc.view(np.uint8)
                o = lay.offset(0, e, m, 2)
                t[o:o + rows * 4] = _vec(rng, rows, 0.0, vs).view(np.uint8)
        return t

    write_experts(os.path.join(out_dir, "experts.midge"), DT_MXFP4, (layer_table(li) for li in range(L)))
    return sp


def prompt(n: int, vocab: int, seed: int = 3) -> list[int]:
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def run_engine(exe: str, model_dir: str, script: str, ctx: int = 512, timeout: float = 600.0,
               env: dict | None = None) -> tuple[list[np.ndarray], list[int], list[list[float]], str]:
    """Runs one engine over a protocol script (its stdin); returns the logits
    rows ("L ..." lines), the generated tokens ("T ..." lines), the fields of
    each "DONE <prompt> <generated> <seconds> <expert loads>" line, and
    stderr."""
    import subprocess
    r = subprocess.run([exe, model_dir, "--ctx", str(ctx), "--no-stats"], input=script, capture_output=True,
                       text=True, timeout=timeout, env=env)
    if r.returncode != 0:
        raise RuntimeError(f"{os.path.basename(exe)} exited {r.returncode}: {r.stderr[-2000:]}")
    logits, toks, done = [], [], []
    for ln in r.stdout.splitlines():
        if ln.startswith("L "):
            logits.append(np.array(ln[2:].split(), np.float32))
        elif ln.startswith("T "):
            toks.append(int(ln[2:]))
        elif ln.startswith("DONE "):
            done.append([float(v) for v in ln[5:].split()])
    return logits, toks, done, r.stderr
