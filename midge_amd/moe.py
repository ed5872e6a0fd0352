"""Layer-level interface, named after the reference's MoE functions.

    moe(layer, x)                  moe()                 engine/midge.c:469-549
    moe_prefill(layer, x)          forward_batch() MoE   engine/midge.c:591-611
    route_topk_dev / topk_dev      route_topk()          engine/midge.c:404-434
    expert_major_dev               expert-major block    engine/midge.c:595-611
    Stack.decode                   forward() layer loop, MoE half, midge.c:557-560

A `MoELayer` carries what the reference's Model holds for one layer: the
layer's slice of the expert table (experts.midge at wt_expert_layout()
offsets), the router, its bias and the mlp norm weight.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib, synth
from .device import DevBuf, Region
from .kern import WT
from .synth import Keys, MoEShape


class MoELayer:
    def __init__(self, shape: MoEShape, experts, router: WT, router_b, mlp_norm):
        self.shape = shape
        self.experts = experts
        self.router = router
        self.router_b = router_b
        self.mlp_norm = mlp_norm
        self._keep: list = []

    @staticmethod
    def _p(a) -> int:
        if isinstance(a, np.ndarray):
            return int(a.ctypes.data)
        return int(a)

    def c(self) -> _lib.MhMoeLayer:
        s, L = self.shape, self.shape.layout
        c = _lib.MhMoeLayer()
        c.hidden, c.ffn, c.n_experts, c.top_k = s.hidden, s.ffn, s.n_experts, s.top_k
        c.alpha, c.limit, c.norm_eps = s.alpha, s.limit, s.norm_eps
        c.act_plain, c.router_norm, c.expert_dt = s.act_plain, s.router_norm, s.expert_dt
        c.expert_stride = L.expert_stride
        for i, o in enumerate(L.off):
            c.off[i] = o
        c.experts = self._p(self.experts)
        c.router = self.router.c()
        c.router_b = self._p(self.router_b)
        c.mlp_norm = self._p(self.mlp_norm)
        return c

    # ------------------------------------------------------------ builders

    @classmethod
    def host(cls, shape: MoEShape, experts: np.ndarray, router_w: np.ndarray, router_s: np.ndarray | None,
             router_b: np.ndarray, mlp_norm: np.ndarray, register: bool = True) -> "MoELayer":
        """A layer over host arrays; with register=True every array is uploaded
        through mh_register_region (the drop-in path for mmap'd blobs)."""
        router = WT(shape.router_dt, shape.n_experts, shape.hidden, router_w, router_s)
        lay = cls(shape, experts, router, router_b, mlp_norm)
        if register:
            for a in (experts, router_w, router_s, router_b, mlp_norm):
                if isinstance(a, np.ndarray) and a.nbytes:
                    lay._keep.append(Region(a))
        return lay

    @classmethod
    def synthetic_host(cls, shape: MoEShape, seed: int, layer: int = 0, register: bool = True) -> "MoELayer":
        keys = Keys(seed)
        experts = synth.host_layer_experts(shape, keys, layer)
        w, s, b, nw = synth.host_router(shape, keys, layer)
        return cls.host(shape, experts, w, s, b, nw, register=register)

    def release(self) -> None:
        """Unregister / free what this layer uploaded (idempotent)."""
        for r in self._keep:
            if isinstance(r, Region):
                r.release()
            elif isinstance(r, DevBuf):
                r.free()
        self._keep.clear()


def moe(layer: MoELayer, x: np.ndarray):
    """moe() on host x[hidden]: returns (x_out, sel[k], w[k])."""
    s = layer.shape
    x = np.array(x, dtype=np.float32, copy=True).reshape(s.hidden)
    sel = np.empty(s.top_k, dtype=np.int32)
    w = np.empty(s.top_k, dtype=np.float32)
    c = layer.c()
    _lib.call("mh_moe", C.byref(c), x.ctypes.data, sel.ctypes.data, w.ctypes.data)
    return x, sel, w


def moe_dev(layer: MoELayer, x, batch: int, sel=None, w=None) -> None:
    c = layer.c()
    _lib.call("mh_moe_dev", C.byref(c), int(x), int(batch), int(sel or 0), int(w or 0))


def moe_prefill(layer: MoELayer, x: np.ndarray):
    """forward_batch()'s MoE half on host x[n][hidden]: returns (x_out, sel[n][k], w[n][k])."""
    s = layer.shape
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1, s.hidden)
    n = x.shape[0]
    sel = np.empty((n, s.top_k), dtype=np.int32)
    w = np.empty((n, s.top_k), dtype=np.float32)
    c = layer.c()
    _lib.call("mh_moe_prefill", C.byref(c), n, x.ctypes.data, sel.ctypes.data, w.ctypes.data)
    return x, sel, w


def moe_prefill_dev(layer: MoELayer, x, n: int, sel=None, w=None) -> None:
    c = layer.c()
    _lib.call("mh_moe_prefill_dev", C.byref(c), int(n), int(x), int(sel or 0), int(w or 0))


def sample_dev(logits, vocab: int, temp: float, topp: float, u: float, out) -> None:
    """sample() on device logits[vocab] into device out[0] (int32); u is the
    caller's rng_f() draw (unused when temp <= 0)."""
    _lib.call("mh_sample_dev", int(logits), int(vocab), float(temp), float(topp), float(u), int(out))


def sample_dev_static(logits, vocab: int, temp: float, topp: float, u: float, out) -> None:
    """sample_dev on the library's fixed workspace: allocates nothing
    (vocab <= 262144; overlapping calls on one GPU share the workspace and
    race)."""
    _lib.call("mh_sample_dev_static", int(logits), int(vocab), float(temp), float(topp), float(u), int(out))


def topk_dev(logits, n: int, n_experts: int, k: int, router_norm: int, sel, w) -> None:
    _lib.call("mh_topk_dev", int(logits), int(n), int(n_experts), int(k), int(router_norm), int(sel), int(w))


def expert_major_dev(layer: MoELayer, n: int, xb, sel, w, x) -> None:
    c = layer.c()
    _lib.call("mh_expert_major_dev", C.byref(c), int(n), int(xb), int(sel), int(w), int(x))


class Stack:
    """A device-resident multi-layer decode plan (mh_stack_*)."""

    @classmethod
    def synthetic(cls, shape: MoEShape, seed: int, max_batch: int):
        """A stack whose expert table (all layers, one allocation at the
        experts.midge layout), routers and norm weights are generated on the
        device from `seed` (include/midge_hip_synth.h). Returns (stack,
        buffers to free, keys); synth's host functions regenerate any slice."""
        keys = Keys(seed)
        L = shape.layout
        table = DevBuf(L.layer_stride * shape.n_layers)
        proto = MoELayer(shape, table.ptr, WT(shape.router_dt, shape.n_experts, shape.hidden, 1, 1), 1, 1).c()
        _lib.call("mh_synth_expert_table_dev", table.ptr, C.byref(proto), shape.n_layers, keys.table,
                  synth.EXPERT_EMIN, synth.EXPERT_EMAX, float(synth.normal_c(synth.EXPERT_BIAS_STD)))
        E, H = shape.n_experts, shape.hidden
        layers, bufs = [], [table]
        for l in range(shape.n_layers):
            rw, rs, rb, nw = DevBuf(E * H), DevBuf(E * 4), DevBuf(E * 4), DevBuf(H * 4)
            _lib.call("mh_synth_i8_dev", rw.ptr, E * H, keys.layer(keys.router_w, l))
            _lib.call("mh_synth_uniform_dev", rs.ptr, E, keys.layer(keys.router_s, l), synth.ROUTER_SCALE_LO,
                      float(synth.uniform_c(synth.ROUTER_SCALE_LO, synth.ROUTER_SCALE_HI)))
            _lib.call("mh_synth_normal_dev", rb.ptr, E, keys.layer(keys.router_b, l),
                      float(synth.normal_c(synth.ROUTER_BIAS_STD)))
            _lib.call("mh_synth_uniform_dev", nw.ptr, H, keys.layer(keys.norm, l), synth.NORM_LO,
                      float(synth.uniform_c(synth.NORM_LO, synth.NORM_HI)))
            bufs += [rw, rs, rb, nw]
            layers.append(MoELayer(shape, table.ptr + l * L.layer_stride,
                                   WT(shape.router_dt, E, H, rw.ptr, rs.ptr), rb.ptr, nw.ptr))
        return cls(layers, max_batch), bufs, keys

    def __init__(self, layers: list[MoELayer], max_batch: int):
        self._cl = (_lib.MhMoeLayer * len(layers))(*[l.c() for l in layers])
        p = C.c_void_p()
        _lib.call("mh_stack_create", self._cl, len(layers), int(max_batch), C.byref(p))
        self.handle = int(p.value)
        self.n_layers = len(layers)
        self.layers = layers

    def decode(self, x, batch: int, sel=None, w=None, usage=None) -> None:
        _lib.call("mh_stack_decode", self.handle, int(x), int(batch), int(sel or 0), int(w or 0),
                  int(usage or 0))

    def apply(self, layer: int, xb, sel, w, x) -> None:
        """expert_apply for one token with the routing given (device xb,
        sel, w, x): x += w_i expert_{sel_i}(xb) in ascending expert order."""
        _lib.call("mh_stack_apply_dev", self.handle, int(layer), int(xb), int(sel), int(w), int(x))

    def destroy(self) -> None:
        if self.handle:
            _lib.call("mh_stack_destroy", self.handle)
            self.handle = 0
