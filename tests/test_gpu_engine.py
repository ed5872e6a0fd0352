"""The reference engine's own host on the GPU: the engine built from its
sources against libmidge_hip, at the kernel level (every wk_matvec / wk_row
on the GPU, oracle/_ref/midged_hip) and at the layer level (containers
uploaded whole at load, one mh_moe per MoE layer, one mh_moe_prefill per
prefill chunk and layer, oracle/_ref/midged_hip_layer), against the same
engine on its CPU kernels (oracle/_ref/midged), over the reference's
protocol (engine/midge.c:15-24): teacher-forced logits at every position,
then greedy generation, batched prefill and token by token
(MIDGE_NO_BATCH=1).

  tiny    the reference's own end-to-end validation model and prompt
          (tools/make_tiny.py shapes, tools/validate.py:39), held to its
          acceptance bar (tools/validate.py:125-141): logits within
          rtol = atol = 2e-3 at every position, identical greedy tokens.
  gptoss  gpt-oss's layer shapes, 4 layers, 160 prompt tokens (past the
          128-token sliding window). At these widths the reference's own
          AVX2 and scalar builds differ by up to ~4e-3 in a logit, and
          outside the validation bar at some positions. The kernel level
          (the reference's attention on the host) holds each position to
          that bar or to twice the reference's own build-to-build difference
          there. The layer level runs attention on the device, whose f16
          k/v cache takes last-bit rounding flips at other positions than
          the AVX2 build's (as in the long attention shapes of
          test_gpu_kernels), so its errors peak elsewhere: the worst over the
          run is held to twice the reference's worst, the mean to twice its
          mean (measured: worst 3.7e-3 against 3.8e-3, mean 1.4e-3 against
          1.1e-3). Greedy tokens must be identical. (Random routers put
          near-ties in the top-k at some positions for some prompts, where
          any two f32 summation orders may pick different experts; the
          prompt is one on which the reference's two builds agree on every
          pick. test_engine_host_random_prompts covers prompts drawn at
          random.)"""
import os

import numpy as np
import pytest

import engine_model as em
from conftest import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
CPU, KERN, LAYER = (os.path.join(REF, n) for n in ("midged", "midged_hip", "midged_hip_layer"))


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    for exe in (CPU, KERN, LAYER):
        if not os.path.exists(exe):
            pytest.fail(f"{exe} is not built (python -m midge_amd.build where the reference checkout exists)")
    tiny = str(tmp_path_factory.mktemp("tiny"))
    big = str(tmp_path_factory.mktemp("gptoss4"))
    return {"tiny": (tiny, em.write_model(tiny, tiny=True)), "gptoss": (big, em.write_model(big, n_layers=4))}


def _close(a, b) -> bool:
    return bool(np.allclose(b, a, rtol=2e-3, atol=2e-3))


@pytest.mark.parametrize("batched", [True, False], ids=["batched_prefill", "token_by_token"])
@pytest.mark.parametrize("which", ["tiny", "gptoss"])
def test_engine_host_on_gpu(models, which, batched):
    d, sp = models[which]
    env = dict(os.environ)
    if not batched:
        env["MIDGE_NO_BATCH"] = "1"      # forward() per prompt token (engine/midge.c:774-778)
    if which == "tiny":
        ids, n_gen, ctx = em.TINY_IDS, 24, 64
    else:
        ids, n_gen, ctx = em.prompt(160 if batched else 48, sp["vocab"], seed=9), 16, 256
    script = f"tfall: {' '.join(map(str, ids))}\ngen: {n_gen}\nquit\n"
    tag = f"engine host {which} {'batched' if batched else 'token-by-token'}"
    say(f"{tag}: cpu")
    ref = em.run_engine(CPU, d, script, ctx=ctx, env=env)
    assert len(ref[0]) == len(ids) and len(ref[1]) == n_gen
    own = None
    if which == "gptoss":   # the reference's own build-to-build difference per position
        sc = em.run_engine(CPU, d, script, ctx=ctx, env=dict(env, MIDGE_NO_SIMD="1"))
        assert sc[1] == ref[1]
        own = [float(np.max(np.abs(a - b))) for a, b in zip(ref[0], sc[0])]
    rates = {"cpu": n_gen / ref[2][1][2]}
    for name, exe in (("kernel_level", KERN), ("layer_level", LAYER)):
        say(f"{tag}: {name}")
        lg, toks, done, _ = em.run_engine(exe, d, script, ctx=ctx, env=env)
        assert len(lg) == len(ids)
        diffs = [float(np.max(np.abs(a - b))) for a, b in zip(ref[0], lg)]
        worst = max(diffs)
        over = [i for i, (a, b) in enumerate(zip(ref[0], lg))
                if not (_close(a, b) or (own is not None and diffs[i] <= 2.0 * own[i]))]
        if own is not None and name == "layer_level":
            # device attention: the run's worst and mean against the reference's own
            say(f"{tag}: {name} positions past the per-position bar: {over}")
            assert worst <= 2.0 * max(own), (name, worst, max(own))
            assert np.mean(diffs) <= 2.0 * np.mean(own), (name, np.mean(diffs), np.mean(own))
        else:
            assert not over, (name, over[0], diffs[over[0]], own[over[0]] if own else None)
        assert toks == ref[1], (name, ref[1], toks)
        # the bookkeeping: the same expert loads in every DONE line
        assert [d[3] for d in done] == [d[3] for d in ref[2]], (name, done, ref[2])
        rates[name] = n_gen / done[1][2]
        say(f"{tag}: {name} worst logit diff {worst:.2e} over {len(ids)} positions"
            + (f" (reference's own builds: {max(own):.2e})" if own else "") + f"; {n_gen} greedy tokens equal")
    say(f"{tag}: greedy decode tok/s " + ", ".join(f"{k} {v:.1f}" for k, v in rates.items()))


def test_engine_host_random_prompts(models):
    """The layer-level host over six prompts drawn at random (seeds 11-16,
    fixed before any was run, 48 tokens, then 16 greedy tokens) at gpt-oss's
    layer shapes, against the CPU engine's AVX2 build, with the reference's
    own scalar build as the yardstick: greedy tokens and the expert loads of
    every DONE line identical, and the mean logit distance over all positions
    within twice the scalar build's. (Measured: tokens and loads identical on
    all six, as for the scalar build; mean 1.35e-3 against 1.17e-3; the worst
    position 7.6e-3 against the scalar build's worst of 3.2e-3, where the
    device attention's f16 k/v cache takes its rounding flips.)"""
    d, sp = models["gptoss"]
    gpu_d, own_d = [], []
    for seed in range(11, 17):
        ids = em.prompt(48, sp["vocab"], seed=seed)
        script = f"tfall: {' '.join(map(str, ids))}\ngen: 16\nquit\n"
        say(f"engine host random prompt seed {seed}")
        ref = em.run_engine(CPU, d, script, ctx=256)
        sc = em.run_engine(CPU, d, script, ctx=256, env=dict(os.environ, MIDGE_NO_SIMD="1"))
        lg, toks, done, _ = em.run_engine(LAYER, d, script, ctx=256)
        assert len(lg) == len(ids) and len(toks) == 16
        assert toks == ref[1], (seed, ref[1], toks)
        assert [x[3] for x in done] == [x[3] for x in ref[2]], (seed, done, ref[2])
        gpu_d += [float(np.max(np.abs(a - b))) for a, b in zip(ref[0], lg)]
        own_d += [float(np.max(np.abs(a - b))) for a, b in zip(ref[0], sc[0])]
    say(f"random prompts: mean {np.mean(gpu_d):.3g} (reference's builds {np.mean(own_d):.3g}), "
        f"worst {max(gpu_d):.3g} ({max(own_d):.3g})")
    assert np.mean(gpu_d) <= 2.0 * np.mean(own_d), (np.mean(gpu_d), np.mean(own_d))


@pytest.mark.parametrize("which", ["tiny", "gptoss"])
def test_engine_host_sampling_on_gpu(models, which):
    # gen: at temperature > 0 (set: <temp> <topp> <seed>, engine/midge.c:
    # 763-771): both GPU hosts draw the engine's generator where the
    # reference does (one rng_f() per sampled token), the layer level
    # samples on the device logits (mh_sample_dev); the tokens equal the CPU
    # engine's
    d, sp = models[which]
    ids = em.TINY_IDS if which == "tiny" else em.prompt(48, sp["vocab"], seed=9)
    ctx = 64 if which == "tiny" else 256
    n_gen = 16
    script = f"set: 0.8 0.9 5\nids: {' '.join(map(str, ids))}\ngen: {n_gen}\nquit\n"
    say(f"engine host {which} sampling: cpu")
    ref = em.run_engine(CPU, d, script, ctx=ctx)
    assert len(ref[1]) == n_gen
    for name, exe in (("kernel_level", KERN), ("layer_level", LAYER)):
        say(f"engine host {which} sampling: {name}")
        _, toks, _, _ = em.run_engine(exe, d, script, ctx=ctx)
        assert toks == ref[1], (name, ref[1], toks)

