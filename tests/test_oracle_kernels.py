"""Pin the oracle's kernels (engine/mkern.h restated in oracle/midge_oracle.c).

Each check uses something other than the oracle's own formula: numpy closed
forms written from the format definitions, float64 brute-force dot products,
a stable argsort, float64 softmax / SwiGLU, the closed-form layout at gpt-oss
shapes, and the reference engine compiled from its sources (bit-exact on its
scalar path, within f32 rounding on its AVX2+FMA path).
"""
import ctypes as C

import os

import numpy as np
import pytest

from midge_amd import DT_F32, DT_MXFP4, DT_Q4G32, DT_Q8R
from oracle import pyoracle as po

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)
RNG = np.random.default_rng(20261201)


def fp4_values(codes: np.ndarray) -> np.ndarray:
    mag = E2M1[codes & 7]
    return np.where(codes & 8, -mag, mag).astype(np.float32)


def pow2_f16(e: np.ndarray) -> np.ndarray:
    """f16 bits of 2^e, e in [-24, 15] (normal and subnormal powers of two)."""
    e = np.asarray(e, np.int64)
    return np.where(e >= -14, (e + 15) << 10, 1 << np.clip(e + 24, 0, 30)).astype(np.uint16)


def make_tensor(dt: int, rows: int, cols: int, rng=RNG, sub=False):
    if dt == DT_F32:
        return rng.standard_normal((rows, cols)).astype(np.float32), None
    if dt == DT_Q8R:
        return (rng.integers(-127, 128, (rows, cols)).astype(np.int8),
                rng.uniform(1e-3, 1e-2, rows).astype(np.float32))
    data = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    if dt == DT_MXFP4:
        lo, hi = (-24, 15) if sub else (-8, -4)
        sc = pow2_f16(rng.integers(lo, hi + 1, (rows, cols // 32)))
    else:
        sc = rng.uniform(0.01, 2.0, (rows, cols // 32)).astype(np.float16).view(np.uint16)
    return data, sc


def closed_form_dequant(dt, data, scales, rows, cols):
    if dt == DT_F32:
        return data.astype(np.float32)
    if dt == DT_Q8R:
        return data.astype(np.float32) * scales[:, None]
    codes = np.empty((rows, cols), np.uint8)
    codes[:, 0::2] = data & 15        # low nibble = even column (engine/mten.h:26-30)
    codes[:, 1::2] = data >> 4
    vals = fp4_values(codes) if dt == DT_MXFP4 else (codes.astype(np.int32) - 8).astype(np.float32)
    s = scales.view(np.float16).astype(np.float32)
    return (vals.reshape(rows, cols // 32, 32) * s[:, :, None]).reshape(rows, cols)


@pytest.mark.parametrize("dt", [DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4])
def test_dequant_closed_form(dt):
    rows, cols = 7, 96
    data, sc = make_tensor(dt, rows, cols, sub=True)
    want = closed_form_dequant(dt, data, sc, rows, cols)
    for r in range(rows):
        got = po.dequant_row(dt, data, sc, cols, r)
        assert (got.view(np.uint32) == want[r].view(np.uint32)).all(), r


def test_dequant_all_codes_all_exponents():
    # every FP4 code under every f16-exact power-of-two scale, bit for bit (incl. -0.0)
    exps = np.arange(-24, 16)
    codes = np.arange(16, dtype=np.uint8)
    data = np.tile((codes[0::2] | (codes[1::2] << 4)), 4).reshape(1, 32)   # 64 columns = 2 groups
    data = np.repeat(data, len(exps), axis=0)
    sc = np.repeat(pow2_f16(exps)[:, None], 2, axis=1)
    want = closed_form_dequant(DT_MXFP4, data, sc, len(exps), 64)
    for r in range(len(exps)):
        got = po.dequant_row(DT_MXFP4, data, sc, 64, r)
        assert (got.view(np.uint32) == want[r].view(np.uint32)).all()
    assert np.signbit(want[:, 8]).all() and (want[:, 8] == 0).all()   # code 8 -> -0.0


@pytest.mark.skipif(not po.have_ref(), reason="reference engine not built here")
@pytest.mark.parametrize("dt", [DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4])
def test_dequant_vs_reference(dt):
    rows, cols = 5, 128
    data, sc = make_tensor(dt, rows, cols, sub=True)
    for r in range(rows):
        a = po.dequant_row(dt, data, sc, cols, r)
        b = po.ref_row(dt, data, sc, rows, cols, r)
        assert (a.view(np.uint32) == b.view(np.uint32)).all()


@pytest.mark.parametrize("dt", [DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4])
@pytest.mark.parametrize("shape", [(1, 32), (13, 64), (40, 2880)])
def test_matvec_brute_force(dt, shape):
    rows, cols = shape
    data, sc = make_tensor(dt, rows, cols)
    x = RNG.standard_normal(cols).astype(np.float32)
    W = closed_form_dequant(dt, data, sc, rows, cols).astype(np.float64)
    want = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    got = po.matvec(dt, data, sc, x, rows, cols)
    assert (np.abs(got - want) <= 1e-5 * mag + 1e-30).all()


@pytest.mark.skipif(not po.have_ref(), reason="reference engine not built here")
@pytest.mark.parametrize("dt", [DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4])
def test_matvec_vs_reference(dt):
    rows, cols = 33, 2880
    data, sc = make_tensor(dt, rows, cols)
    x = RNG.standard_normal(cols).astype(np.float32)
    got = po.matvec(dt, data, sc, x, rows, cols)
    scalar = po.ref_matvec(dt, data, sc, x, rows, cols, scalar=True)
    assert (got.view(np.uint32) == scalar.view(np.uint32)).all()   # same order, no FMA
    simd = po.ref_matvec(dt, data, sc, x, rows, cols, scalar=False)
    mag = np.abs(closed_form_dequant(dt, data, sc, rows, cols)) @ np.abs(x)
    assert (np.abs(got - simd) <= 1e-5 * mag).all()


def test_rmsnorm_closed_form():
    x = RNG.standard_normal(2880).astype(np.float32) * 3
    w = RNG.uniform(0.5, 1.5, 2880).astype(np.float32)
    eps = 1e-5
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean() + eps) * w
    got = po.rmsnorm(x, w, eps)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    if po.have_ref():
        r = po.ref_rmsnorm(x, w, eps)
        assert (got.view(np.uint32) == r.view(np.uint32)).all()


@pytest.mark.parametrize("decode", [True, False])
def test_topk_stable_argsort(decode):
    for trial in range(200):
        E = int(RNG.choice([4, 8, 32, 128]))
        k = int(RNG.integers(1, min(16, E) + 1))
        rl = RNG.standard_normal(E).astype(np.float32)
        if trial % 3 == 0:   # force ties
            rl = np.round(rl * 2) / 2
        sel, val = po.topk(rl, k, decode=decode)
        want = np.argsort(-rl, kind="stable")[:k]
        assert (sel == want).all(), (rl, k, sel, want)
        assert (val == rl[want]).all()


def test_topk_unfillable_slots():
    rl = np.array([-np.inf, 0.5, np.nan, -2e30], np.float32)
    sel, val = po.topk(rl, 3, decode=True)
    assert list(sel) == [1, -1, -1] and val[0] == np.float32(0.5)   # moe(): unfilled = -1
    sel, val = po.topk(rl, 3, decode=False)
    assert list(sel) == [1, 0, 0]                                    # route_topk(): unfilled = 0


def test_router_weights_softmax():
    rl = RNG.standard_normal(32).astype(np.float32) * 3
    sel, val = po.topk(rl, 4)
    w = po.router_weights(rl, val, 1)
    v = val.astype(np.float64)
    want = np.exp(v - v.max()) / np.exp(v - v.max()).sum()
    assert np.allclose(w, want, rtol=1e-6)
    w0 = po.router_weights(rl, val, 0)
    full = np.exp(rl.astype(np.float64) - rl.max())
    assert np.allclose(w0, full[sel] / full.sum(), rtol=1e-6)


def test_clamped_swiglu_closed_form():
    g = np.linspace(-12, 12, 1001).astype(np.float32)
    u = np.linspace(9, -9, 1001).astype(np.float32)
    alpha, limit = 1.702, 7.0
    got = po.act(g, u, alpha, limit)
    g64 = np.minimum(g.astype(np.float64), limit)      # upper clamp only
    u64 = np.clip(u.astype(np.float64), -limit, limit)
    want = g64 / (1 + np.exp(-alpha * g64)) * (u64 + 1)
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
    plain = po.act(g, u, alpha, limit, plain=1)
    g64 = g.astype(np.float64)
    assert np.allclose(plain, g64 / (1 + np.exp(-g64)) * u, rtol=1e-5, atol=1e-6)


# closed-form offsets of wt_expert_layout at gpt-oss hidden = ffn = 2880 (MXFP4)
GPT_OSS_OFF = [0, 4147200, 4665600, 4677120, 8824320, 9342720, 9354240, 13501440, 14019840]


def test_layout_gpt_oss():
    off, es, ls = po.expert_layout(DT_MXFP4, 2880, 2880, 128)
    assert off == GPT_OSS_OFF
    assert es == 14031360
    assert 36 * ls == 64656506880            # gpt-oss-120b expert table
    _, es20, ls20 = po.expert_layout(DT_MXFP4, 2880, 2880, 32)
    assert 24 * ls20 == 10776084480          # gpt-oss-20b expert table


@pytest.mark.skipif(not po.have_ref(), reason="reference engine not built here")
def test_layout_vs_reference():
    import ctypes as C
    r = po.ref()
    for dt in (DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4):
        for hidden, ffn, E in ((64, 64, 4), (2880, 2880, 128), (4096, 14336, 8), (96, 32, 3)):
            off = np.zeros(9, np.uint64)
            es, ls = C.c_uint64(), C.c_uint64()
            r.ref_expert_layout(dt, hidden, ffn, E, off.ctypes.data, C.addressof(es), C.addressof(ls))
            o2, es2, ls2 = po.expert_layout(dt, hidden, ffn, E)
            assert [int(v) for v in off] == o2 and es.value == es2 and ls.value == ls2


def test_layout_mirror_matches_oracle():
    from midge_amd.layout import ExpertLayout
    for dt in (DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4):
        for hidden, ffn, E in ((64, 64, 4), (2880, 2880, 128), (96, 32, 3)):
            L = ExpertLayout(dt, hidden, ffn, E)
            off, es, ls = po.expert_layout(dt, hidden, ffn, E)
            assert list(L.off) == off and L.expert_stride == es and L.layer_stride == ls


# ------------------------------------------------------------- sampling

def test_rng_matches_xorshift_closed_form():
    # engine/midge.c:641-646: xorshift64 (12, 25, 27), the high word of the
    # state times 0x2545F4914F6CDD1D, 24 bits / 2^24
    st = 0x853C49E6748FEA9B
    for _ in range(100):
        x = st
        x ^= x >> 12
        x = (x ^ (x << 25)) & (2**64 - 1)
        x ^= x >> 27
        want = ((((x * 0x2545F4914F6CDD1D) & (2**64 - 1)) >> 32) >> 8) / 16777216.0
        u, st = po.rng_f(st)
        assert st == x and u == np.float32(want)


def test_sample_greedy_is_first_argmax():
    rng = np.random.default_rng(5)
    for V in (1, 7, 1000):
        lg = np.round(rng.standard_normal(V) * 2).astype(np.float32)   # many ties
        assert po.sample(lg, 0.0, 0.9, 0.5) == int(np.argmax(lg))
    lg = np.array([np.nan, 5.0, 7.0], np.float32)   # the loop starts at a NaN: token 0
    assert po.sample(lg, 0.0, 1.0, 0.0) == 0
    lg = np.array([1.0, np.nan, 7.0, 7.0], np.float32)
    assert po.sample(lg, 0.0, 1.0, 0.0) == 2


def test_sample_nucleus_special_cases():
    rng = np.random.default_rng(6)
    lg = (rng.standard_normal(500) * 2).astype(np.float32)
    top = int(np.argmax(lg))
    for u in (0.0, 0.3, 0.999):
        assert po.sample(lg, 1.0, 1e-9, u) == top      # a nucleus of one
    assert po.sample(lg, 0.8, 1.0, 0.0) == top          # u = 0: the most probable
    # three tokens of probability 0.5, 0.3, 0.2 (temp 1): topp 0.75 keeps two
    lg = np.log(np.array([0.2, 0.5, 0.3], np.float32))
    assert po.sample(lg, 1.0, 0.75, 0.5) == 1           # r = 0.4 <= 0.5
    assert po.sample(lg, 1.0, 0.75, 0.99) == 2          # r = 0.792 > 0.5, <= 0.8
    assert po.sample(lg, 1.0, 1.0, 0.99) == 0           # the whole set: r = 0.99 > 0.8


def test_sample_frequencies_follow_the_tempered_softmax():
    lg = np.array([0.0, 1.0, 2.0, -1.0, 0.5], np.float32)
    temp = 0.7
    p = np.exp((lg - lg.max()) / temp)
    p /= p.sum()
    st, counts, N = 12345, np.zeros(5), 20000
    for _ in range(N):
        u, st = po.rng_f(st)
        counts[po.sample(lg, temp, 1.0, u)] += 1
    assert np.abs(counts / N - p).max() < 0.015


def test_sample_vs_reference():
    if not po.have_ref():
        pytest.skip("reference engine not built (oracle/_ref)")
    rng = np.random.default_rng(7)
    st = 0x853C49E6748FEA9B
    for V in (8, 1000, 20000):
        for temp in (0.0, 0.5, 1.0, 1.7):
            for topp in (0.1, 0.9, 1.0):
                lg = (rng.standard_normal(V) * 3).astype(np.float32)
                tok_ref, st2 = po.ref_sample(lg, temp, topp, st)
                u, st3 = po.rng_f(st) if temp > 0 else (0.0, st)
                assert st3 == st2
                assert po.sample(lg, temp, topp, u) == tok_ref, (V, temp, topp)
                st = st2


# ------------------------------------------------------------- attention

GPT_OSS_ROPE = dict(theta=150000.0, yarn=1, factor=32.0, beta_fast=32.0, beta_slow=1.0, orig_ctx=4096, truncate=0)


def rope_tables(hd: int, ctx: int, fn, theta=10000.0, yarn=0, factor=1.0, beta_fast=32.0, beta_slow=1.0,
                orig_ctx=4096, truncate=0):
    half = hd // 2
    co, si = np.zeros((ctx, half), np.float32), np.zeros((ctx, half), np.float32)
    fn(hd, theta, yarn, factor, beta_fast, beta_slow, orig_ctx, truncate, ctx, co.ctypes.data, si.ctypes.data)
    return co, si


class AttnHost:
    """One attention layer on host arrays (q8r projections) with its f16
    caches, as the oracle and the compiled reference take it."""

    def __init__(self, hidden, nh, nkv, hd, ctx, window, qk_norm, sinks, seed, rope=None, wscale=(5e-4, 2.5e-3)):
        rng = np.random.default_rng(seed)
        self.keep = []

        def q8(rows, cols):   # row scales uniform in wscale
            w = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
            s = (rng.random(rows) * (wscale[1] - wscale[0]) + wscale[0]).astype(np.float32)
            self.keep += [w, s]
            return po.MhWT(DT_Q8R, rows, cols, w.ctypes.data, s.ctypes.data)

        def vec(n, mean=0.0, std=0.1):
            a = (mean + std * rng.standard_normal(n)).astype(np.float32)
            self.keep.append(a)
            return a

        self.cap = window if 0 < window < ctx else ctx
        self.kvd = nkv * hd
        self.kc = np.zeros((self.cap, self.kvd), np.uint16)
        self.vc = np.zeros((self.cap, self.kvd), np.uint16)
        co, si = rope_tables(hd, ctx, po.oracle().mo_rope_table, **(rope or {}))
        self.co, self.si = co, si
        L = po.MhAttnLayer()
        L.hidden, L.n_heads, L.n_kv_heads, L.head_dim, L.ctx, L.window = hidden, nh, nkv, hd, ctx, window
        L.qk_norm, L.sinks, L.norm_eps, L.attn_scale = qk_norm, sinks, 1e-5, float(1.0 / np.sqrt(hd))
        L.wq, L.wk, L.wv, L.wo = q8(nh * hd, hidden), q8(self.kvd, hidden), q8(self.kvd, hidden), q8(hidden, nh * hd)
        L.bq, L.bk, L.bv, L.bo = (vec(nh * hd).ctypes.data, vec(self.kvd).ctypes.data, vec(self.kvd).ctypes.data,
                                  vec(hidden).ctypes.data)
        L.attn_norm = vec(hidden, 1.0).ctypes.data
        L.qn = vec(hd, 1.0).ctypes.data if qk_norm else None
        L.kn = vec(hd, 1.0).ctypes.data if qk_norm else None
        L.sink = vec(nh, 0.0, 1.0).ctypes.data if sinks else None
        L.rope_cos, L.rope_sin = co.ctypes.data, si.ctypes.data
        L.kc, L.vc = self.kc.ctypes.data, self.vc.ctypes.data
        self.L = L

    def run(self, fn, x: np.ndarray, pos: int) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        assert fn(C.byref(self.L), x.ctypes.data, pos) == 0
        return x


ATTN_SHAPES = {
    "small_sliding_sinks": dict(hidden=256, nh=8, nkv=2, hd=32, ctx=48, window=16, qk_norm=0, sinks=1),
    "small_full_qknorm": dict(hidden=256, nh=4, nkv=4, hd=32, ctx=40, window=0, qk_norm=1, sinks=0),
}


GPT_OSS_ATTN = dict(hidden=2880, nh=64, nkv=8, hd=64, ctx=160, window=128, qk_norm=0, sinks=1)
ATTN_DIV_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_divergence.npz")


def attn_divergence_gptoss() -> np.ndarray:
    """The reference's own divergence on attention() at the gpt-oss shape:
    per decode position (159 of them, past the 128-token sliding window),
    rel L2 of the attention output (x_out - x_in) of its AVX2 build against
    its scalar build, each on its own f16 cache, with the seeds the GPU test
    uses (weights 13, inputs 14). Also checks that the oracle equals the
    scalar build bit for bit at every position (outputs and caches)."""
    cfg = GPT_OSS_ATTN
    a_sc, a_rf, a_or = (AttnHost(**cfg, seed=13, rope=GPT_OSS_ROPE) for _ in range(3))
    rng = np.random.default_rng(14)
    div = np.empty(cfg["ctx"] - 1)
    for pos in range(cfg["ctx"] - 1):
        x = rng.standard_normal(cfg["hidden"]).astype(np.float32)
        xs = a_sc.run(po.ref(scalar=True).ref_attention, x, pos)
        xr = a_rf.run(po.ref().ref_attention, x, pos)
        xo = a_or.run(po.oracle().mo_attention, x, pos)
        assert (xo.view(np.uint32) == xs.view(np.uint32)).all(), pos
        assert (a_or.kc == a_sc.kc).all() and (a_or.vc == a_sc.vc).all(), pos
        d = (xs - x).astype(np.float64)
        div[pos] = np.linalg.norm((xr - x).astype(np.float64) - d) / np.linalg.norm(d)
    return div


def test_attention_divergence_fixture():
    # the per-position AVX2-vs-scalar divergence the GPU attention test's bar
    # is built from: recomputed from the compiled reference, equal to the
    # committed fixture (which the GPU test reads where the reference is absent)
    if not po.have_ref():
        pytest.skip("reference engine not built (oracle/_ref)")
    div = attn_divergence_gptoss()
    want = np.load(ATTN_DIV_FIXTURE)["div"]
    assert div.shape == want.shape
    assert np.allclose(div, want, rtol=1e-9, atol=0.0)


def test_to_f16_vs_reference():
    if not po.have_ref():
        pytest.skip("reference engine not built (oracle/_ref)")
    rng = np.random.default_rng(8)
    vals = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                           [0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1e-5, 6.0e-5, 5.96e-8, np.inf, -np.inf, np.nan,
                            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]]).astype(np.float32)
    for v in vals:
        assert po.oracle().mo_to_f16(float(v)) == po.ref().ref_to_f16_attn(float(v)), v


def test_device_f16_rule_equals_the_cache_conversion():
    # the attention kernel stores the f16 cache as: IEEE round-to-nearest-even
    # (the hardware conversion), except |f| < 2^-14 -> signed zero and NaN ->
    # signed inf; that rule equals the oracle's wk_to_f16 everywhere
    rng = np.random.default_rng(81)
    vals = np.concatenate([rng.standard_normal(40000) * 10.0 ** rng.integers(-12, 7, 40000),
                           np.frombuffer(rng.bytes(4 * 40000), np.float32),
                           [0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 2.0 ** -14, -(2.0 ** -14),
                            np.nextafter(np.float32(2.0 ** -14), np.float32(0)), 5.96e-8, np.inf, -np.inf, np.nan,
                            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]]).astype(np.float32)
    a = np.abs(vals)
    with np.errstate(over="ignore", invalid="ignore"):
        rule = vals.astype(np.float16).view(np.uint16).copy()
    sign = ((vals.view(np.uint32) >> 16) & 0x8000).astype(np.uint16)
    small = ~(a >= np.float32(2.0 ** -14))
    rule[small] = np.where(np.isnan(vals[small]), sign[small] | 0x7C00, sign[small])
    want = np.array([po.oracle().mo_to_f16(float(v)) for v in vals], np.uint16)
    assert (rule == want).all(), vals[rule != want][:8]


@pytest.mark.parametrize("rope", [dict(), GPT_OSS_ROPE, dict(GPT_OSS_ROPE, truncate=1)])
def test_rope_tables_vs_reference(rope):
    if not po.have_ref():
        pytest.skip("reference engine not built (oracle/_ref)")
    co, si = rope_tables(64, 300, po.oracle().mo_rope_table, **rope)
    cr, sr = rope_tables(64, 300, po.ref().ref_rope_table, **rope)
    assert (co.view(np.uint32) == cr.view(np.uint32)).all() and (si.view(np.uint32) == sr.view(np.uint32)).all()
    # closed form at position 1 without YaRN: cos/sin of theta^(-2i/hd)
    if not rope:
        inv = 1.0 / 10000.0 ** (np.arange(32) * 2 / 64)
        assert np.allclose(co[1], np.cos(inv), atol=1e-7) and np.allclose(si[1], np.sin(inv), atol=1e-7)


@pytest.mark.parametrize("name", list(ATTN_SHAPES))
def test_attention_vs_reference(name):
    # a sequence of positions past the sliding window (the ring wraps):
    # bit for bit against the reference's scalar kernels, and within 1e-4
    # of the reference as shipped (AVX2 matvecs)
    if not po.have_ref():
        pytest.skip("reference engine not built (oracle/_ref)")
    cfg = ATTN_SHAPES[name]
    a_or, a_sc, a_rf = (AttnHost(**cfg, seed=11) for _ in range(3))
    rng = np.random.default_rng(12)
    for pos in range(cfg["ctx"] - 2):
        x = rng.standard_normal(cfg["hidden"]).astype(np.float32)
        xo = a_or.run(po.oracle().mo_attention, x, pos)
        xs = a_sc.run(po.ref(scalar=True).ref_attention, x, pos)
        xr = a_rf.run(po.ref().ref_attention, x, pos)
        assert (xo.view(np.uint32) == xs.view(np.uint32)).all(), pos
        assert (a_or.kc == a_sc.kc).all() and (a_or.vc == a_sc.vc).all(), pos
        assert np.linalg.norm(xo - xr) / np.linalg.norm(xr - x) < 1e-4, pos
