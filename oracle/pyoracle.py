"""ctypes binding of the CPU oracle (test infrastructure only).

Loads oracle/libmidge_oracle.so (the C restatement in midge_oracle.c) and,
where it was built, oracle/_ref/libmidge_ref[_scalar].so (the reference
engine compiled from its own sources through ref_shim.c). Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg import this module;
the product package never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "libmidge_oracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libmidge_ref.so")
REF_SCALAR_LIB = os.path.join(HERE, "_ref", "libmidge_ref_scalar.so")

_P, _I, _I64, _U64, _F, _U16 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_uint16


class MhWT(C.Structure):
    _fields_ = [("dt", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("scales", C.c_void_p)]


class MhAttnLayer(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("ctx", C.c_int32), ("window", C.c_int32),
                ("qk_norm", C.c_int32), ("sinks", C.c_int32), ("norm_eps", C.c_float),
                ("attn_scale", C.c_float), ("wq", MhWT), ("wk", MhWT), ("wv", MhWT), ("wo", MhWT),
                ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("bo", C.c_void_p),
                ("attn_norm", C.c_void_p), ("qn", C.c_void_p), ("kn", C.c_void_p), ("sink", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("kc", C.c_void_p), ("vc", C.c_void_p)]


class MhMoeLayer(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("ffn", C.c_int64),
                ("n_experts", C.c_int32), ("top_k", C.c_int32),
                ("alpha", C.c_float), ("limit", C.c_float), ("norm_eps", C.c_float),
                ("act_plain", C.c_int32), ("router_norm", C.c_int32), ("expert_dt", C.c_int32),
                ("expert_stride", C.c_uint64), ("off", C.c_uint64 * 9),
                ("experts", C.c_void_p), ("router", MhWT),
                ("router_b", C.c_void_p), ("mlp_norm", C.c_void_p)]


_ORACLE_SIGS = {
    "mo_f16_to_f32": ([_U16], _F),
    "mo_fp4_value": ([_I], _F),
    "mo_dequant_row": ([_I, _P, _P, _I64, _I64, _P], _I),
    "mo_matvec": ([_I, _P, _P, _P, _P, _I64, _I64], _I),
    "mo_rmsnorm": ([_P, _P, _P, _I64, _F], None),
    "mo_addbias": ([_P, _P, _I64], None),
    "mo_topk_decode": ([_P, _I, _I, _P, _P], None),
    "mo_topk_route": ([_P, _I, _I, _P, _P], None),
    "mo_router_weights": ([_P, _I, _P, _I, _I, _P], None),
    "mo_act": ([_P, _P, _I64, _F, _F, _I], None),
    "mo_expert_layout": ([_I, _I64, _I64, _I64, _P, _P, _P], _I),
    "mo_expert_ffn": ([C.POINTER(MhMoeLayer), _I, _P, _P], _I),
    "mo_moe_decode": ([C.POINTER(MhMoeLayer), _P, _P, _P, _P, _P], _I),
    "mo_route_batch": ([C.POINTER(MhMoeLayer), _I, _P, _P, _P, _P], _I),
    "mo_expert_major_apply": ([C.POINTER(MhMoeLayer), _I, _P, _P, _P, _P, _P, _P], _I),
    "mo_moe_prefill": ([C.POINTER(MhMoeLayer), _I, _P, _P, _P, _P, _P], _I),
    "mo_hash64": ([_U64, _U64], _U64),
    "mo_synth_bytes": ([_U64, _U64, _P], None),
    "mo_synth_scales": ([_U64, _U64, _I, _I, _P], None),
    "mo_synth_i8": ([_U64, _U64, _P], None),
    "mo_synth_normal": ([_U64, _U64, _F, _P], None),
    "mo_synth_uniform": ([_U64, _U64, _F, _F, _P], None),
    "mo_synth_expert": ([_P, _I, _I64, _I64, _I64, _I, _I, _U64, _I, _I, _F], _I),
    "mo_rng_f": ([_P], _F),
    "mo_to_f16": ([_F], _U16),
    "mo_rope_table": ([_I, _F, _I, _F, _F, _F, _I, _I, _I, _P, _P], None),
    "mo_attention": ([C.POINTER(MhAttnLayer), _P, _I], _I),
    "mo_sample": ([_P, _I64, _F, _F, _F], _I),
}

_REF_SIGS = {
    "ref_have_avx2": ([], _I),
    "ref_matvec": ([_I, _P, _P, _I64, _I64, _P, _P], None),
    "ref_row": ([_I, _P, _P, _I64, _I64, _I64, _P], None),
    "ref_rmsnorm": ([_P, _P, _P, _I64, _F], None),
    "ref_to_f16": ([_F], _U16),
    "ref_f16": ([_U16], _F),
    "ref_expert_layout": ([_I, _I64, _I64, _I64, _P, _P, _P], None),
    "ref_expert_ffn": ([C.POINTER(MhMoeLayer), _I, _P, _P], _I),
    "ref_moe_decode": ([C.POINTER(MhMoeLayer), _P, _P, _P, _P], _I),
    "ref_moe_prefill": ([C.POINTER(MhMoeLayer), _I, _P, _P, _P], _I),
    "ref_run_bench": ([], _I),
    "ref_sample": ([_P, _I64, _F, _F, _P], _I),
    "ref_rope_table": ([_I, _F, _I, _F, _F, _F, _I, _I, _I, _P, _P], None),
    "ref_to_f16_attn": ([_F], _U16),
    "ref_attention": ([C.POINTER(MhAttnLayer), _P, _I], _I),
}

_cache: dict[str, C.CDLL] = {}


def _load(path: str, sigs: dict) -> C.CDLL:
    if path in _cache:
        return _cache[path]
    if not os.path.isfile(path):
        raise FileNotFoundError(f"{path} not built (run `make -C oracle` / `make -C oracle ref`)")
    lib = C.CDLL(path)
    for name, (args, res) in sigs.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    _cache[path] = lib
    return lib


def oracle() -> C.CDLL:
    return _load(ORACLE_LIB, _ORACLE_SIGS)


def have_ref() -> bool:
    return os.path.isfile(REF_LIB) and os.path.isfile(REF_SCALAR_LIB)


def ref(scalar: bool = False) -> C.CDLL:
    return _load(REF_SCALAR_LIB if scalar else REF_LIB, _REF_SIGS)


def _p(a) -> int:
    if a is None:
        return 0
    if isinstance(a, np.ndarray):
        return int(a.ctypes.data)
    return int(a)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} returned {rc}")


# -------------------------------------------------------------- oracle API

def f16_to_f32(h: int) -> float:
    return oracle().mo_f16_to_f32(h)


def fp4_value(code: int) -> float:
    return oracle().mo_fp4_value(code)


def dequant_row(dt: int, data: np.ndarray, scales, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    _check(oracle().mo_dequant_row(dt, _p(data), _p(scales), cols, r, _p(out)), "dequant_row")
    return out


def matvec(dt: int, data: np.ndarray, scales, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    _check(oracle().mo_matvec(dt, _p(data), _p(scales), _p(x), _p(y), rows, cols), "matvec")
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    oracle().mo_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), _p(out), x.size, eps)
    return out


def topk(rl: np.ndarray, k: int, decode: bool = True):
    rl = np.ascontiguousarray(rl, np.float32)
    sel = np.empty(k, np.int32)
    val = np.empty(k, np.float32)
    f = oracle().mo_topk_decode if decode else oracle().mo_topk_route
    f(_p(rl), rl.size, k, _p(sel), _p(val))
    return sel, val


def router_weights(rl: np.ndarray, val: np.ndarray, router_norm: int) -> np.ndarray:
    rl = np.ascontiguousarray(rl, np.float32)
    val = np.ascontiguousarray(val, np.float32)
    w = np.empty(val.size, np.float32)
    oracle().mo_router_weights(_p(rl), rl.size, _p(val), val.size, router_norm, _p(w))
    return w


def act(g: np.ndarray, u: np.ndarray, alpha: float, limit: float, plain: int = 0) -> np.ndarray:
    g = np.array(g, np.float32, copy=True)
    u = np.ascontiguousarray(u, np.float32)
    oracle().mo_act(_p(g), _p(u), g.size, alpha, limit, plain)
    return g


def expert_layout(dt: int, hidden: int, ffn: int, n_experts: int):
    off = np.zeros(9, np.uint64)
    es = C.c_uint64()
    ls = C.c_uint64()
    _check(oracle().mo_expert_layout(dt, hidden, ffn, n_experts, _p(off), C.addressof(es), C.addressof(ls)),
           "expert_layout")
    return [int(o) for o in off], int(es.value), int(ls.value)


def layer_struct(shape, experts: np.ndarray, router_w, router_s, router_b, mlp_norm) -> MhMoeLayer:
    """The layer description over host arrays (keep the arrays alive)."""
    off, es, _ = expert_layout(shape.expert_dt, shape.hidden, shape.ffn, shape.n_experts)
    c = MhMoeLayer()
    c.hidden, c.ffn, c.n_experts, c.top_k = shape.hidden, shape.ffn, shape.n_experts, shape.top_k
    c.alpha, c.limit, c.norm_eps = shape.alpha, shape.limit, shape.norm_eps
    c.act_plain, c.router_norm, c.expert_dt = shape.act_plain, shape.router_norm, shape.expert_dt
    c.expert_stride = es
    for i, o in enumerate(off):
        c.off[i] = o
    c.experts = _p(experts)
    c.router = MhWT(shape.router_dt, shape.n_experts, shape.hidden, _p(router_w), _p(router_s))
    c.router_b = _p(router_b)
    c.mlp_norm = _p(mlp_norm)
    return c


def expert_ffn(L: MhMoeLayer, e: int, xb: np.ndarray) -> np.ndarray:
    xb = np.ascontiguousarray(xb, np.float32)
    y = np.empty(L.hidden, np.float32)
    _check(oracle().mo_expert_ffn(C.byref(L), e, _p(xb), _p(y)), "expert_ffn")
    return y


def moe_decode(L: MhMoeLayer, x: np.ndarray, usage: np.ndarray | None = None):
    x = np.array(x, np.float32, copy=True)
    sel = np.empty(L.top_k, np.int32)
    w = np.empty(L.top_k, np.float32)
    loads = C.c_uint64(0)
    _check(oracle().mo_moe_decode(C.byref(L), _p(x), _p(sel), _p(w), _p(usage), C.addressof(loads)),
           "moe_decode")
    return x, sel, w


def moe_prefill(L: MhMoeLayer, x: np.ndarray):
    x = np.array(x, np.float32, copy=True).reshape(-1, L.hidden)
    n = x.shape[0]
    sel = np.empty((n, L.top_k), np.int32)
    w = np.empty((n, L.top_k), np.float32)
    loads = C.c_uint64(0)
    _check(oracle().mo_moe_prefill(C.byref(L), n, _p(x), _p(sel), _p(w), 0, C.addressof(loads)), "moe_prefill")
    return x, sel, w


def route_batch(L: MhMoeLayer, x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, L.hidden)
    n = x.shape[0]
    xb = np.empty_like(x)
    sel = np.empty((n, L.top_k), np.int32)
    w = np.empty((n, L.top_k), np.float32)
    _check(oracle().mo_route_batch(C.byref(L), n, _p(x), _p(xb), _p(sel), _p(w)), "route_batch")
    return xb, sel, w


def expert_major_apply(L: MhMoeLayer, xb: np.ndarray, sel: np.ndarray, w: np.ndarray, x: np.ndarray):
    x = np.array(x, np.float32, copy=True).reshape(-1, L.hidden)
    n = x.shape[0]
    loads = C.c_uint64(0)
    _check(oracle().mo_expert_major_apply(C.byref(L), n, _p(np.ascontiguousarray(xb, np.float32)),
                                          _p(np.ascontiguousarray(sel, np.int32)),
                                          _p(np.ascontiguousarray(w, np.float32)), _p(x), 0,
                                          C.addressof(loads)), "expert_major_apply")
    return x


def synth_bytes(key: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    oracle().mo_synth_bytes(key, n, _p(out))
    return out


def synth_scales(key: int, n: int, emin: int, emax: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    oracle().mo_synth_scales(key, n, emin, emax, _p(out))
    return out


def synth_i8(key: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int8)
    oracle().mo_synth_i8(key, n, _p(out))
    return out


def synth_normal(key: int, n: int, c: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().mo_synth_normal(key, n, c, _p(out))
    return out


def synth_uniform(key: int, n: int, lo: float, c: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().mo_synth_uniform(key, n, lo, c, _p(out))
    return out


def synth_expert(dt: int, hidden: int, ffn: int, n_experts: int, layer: int, expert: int, key: int,
                 emin: int, emax: int, bias_c: float) -> np.ndarray:
    _, es, _ = expert_layout(dt, hidden, ffn, n_experts)
    out = np.zeros(es, np.uint8)
    _check(oracle().mo_synth_expert(_p(out), dt, hidden, ffn, n_experts, layer, expert, key, emin, emax, bias_c),
           "synth_expert")
    return out


# ------------------------------------------------------------ reference API

def ref_matvec(dt: int, data, scales, x: np.ndarray, rows: int, cols: int, scalar: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    ref(scalar).ref_matvec(dt, _p(data), _p(scales), rows, cols, _p(x), _p(y))
    return y


def ref_row(dt: int, data, scales, rows: int, cols: int, r: int) -> np.ndarray:
    out = np.empty(cols, np.float32)
    ref().ref_row(dt, _p(data), _p(scales), rows, cols, r, _p(out))
    return out


def ref_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    ref().ref_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), _p(out), x.size, eps)
    return out


def ref_expert_ffn(L: MhMoeLayer, e: int, xb: np.ndarray, scalar: bool = False) -> np.ndarray:
    xb = np.ascontiguousarray(xb, np.float32)
    y = np.empty(L.hidden, np.float32)
    _check(ref(scalar).ref_expert_ffn(C.byref(L), e, _p(xb), _p(y)), "ref_expert_ffn")
    return y


def ref_moe_decode(L: MhMoeLayer, x: np.ndarray, scalar: bool = False):
    x = np.array(x, np.float32, copy=True)
    sel = np.empty(L.top_k, np.int32)
    w = np.empty(L.top_k, np.float32)
    usage = np.zeros(L.n_experts, np.uint32)
    _check(ref(scalar).ref_moe_decode(C.byref(L), _p(x), _p(sel), _p(w), _p(usage)), "ref_moe_decode")
    return x, sel, w, usage


def ref_moe_prefill(L: MhMoeLayer, x: np.ndarray, scalar: bool = False):
    x = np.array(x, np.float32, copy=True).reshape(-1, L.hidden)
    n = x.shape[0]
    sel = np.empty((n, L.top_k), np.int32)
    w = np.empty((n, L.top_k), np.float32)
    _check(ref(scalar).ref_moe_prefill(C.byref(L), n, _p(x), _p(sel), _p(w)), "ref_moe_prefill")
    return x, sel, w


def rng_f(state: int) -> tuple[float, int]:
    """One draw of the reference's generator: (u, next state)."""
    st = C.c_uint64(state)
    u = oracle().mo_rng_f(C.byref(st))
    return float(u), int(st.value)


def sample(logits: np.ndarray, temp: float, topp: float, u: float) -> int:
    """sample() with the uniform draw u supplied."""
    lg = np.ascontiguousarray(logits, np.float32)
    return int(oracle().mo_sample(_p(lg), lg.size, temp, topp, u))


def ref_sample(logits: np.ndarray, temp: float, topp: float, state: int) -> tuple[int, int]:
    """The compiled reference sample() from generator state `state`: (token, next state)."""
    lg = np.ascontiguousarray(logits, np.float32)
    st = C.c_uint64(state)
    tok = ref().ref_sample(_p(lg), lg.size, temp, topp, C.byref(st))
    return int(tok), int(st.value)
