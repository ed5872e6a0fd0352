"""An attention layer's tensors copied to device buffers (mh_attention_dev's
argument), shared by the GPU attention tests."""
from __future__ import annotations

import ctypes

import numpy as np

from midge_amd import DevBuf, _lib
from oracle import pyoracle as po


def attn_device_layer(host, cfg: dict):
    """(mh_attn_layer over device copies of host.L's tensors with zeroed f16
    caches, the device buffers to free, the k cache, the v cache)."""
    L = host.L
    bufs = []

    def dev(ptr, nbytes):
        a = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), (nbytes,)).copy()
        d = DevBuf.from_array(a)
        bufs.append(d)
        return d.ptr

    H, nh, nkv, hd = cfg["hidden"], cfg["nh"], cfg["nkv"], cfg["hd"]
    qd, kvd = nh * hd, nkv * hd
    D = _lib.MhAttnLayer()
    for f, _ in po.MhAttnLayer._fields_:
        if f not in ("wq", "wk", "wv", "wo"):
            setattr(D, f, getattr(L, f))
    for f in ("wq", "wk", "wv", "wo"):
        w = getattr(L, f)
        setattr(D, f, _lib.MhWT(w.dt, w.rows, w.cols, dev(w.data, w.rows * w.cols), dev(w.scales, w.rows * 4)))
    for f, n in (("bq", qd), ("bk", kvd), ("bv", kvd), ("bo", H), ("attn_norm", H)):
        setattr(D, f, dev(getattr(L, f), n * 4))
    if cfg["qk_norm"]:
        D.qn, D.kn = dev(L.qn, hd * 4), dev(L.kn, hd * 4)
    if cfg["sinks"]:
        D.sink = dev(L.sink, nh * 4)
    D.rope_cos, D.rope_sin = dev(L.rope_cos, host.co.nbytes), dev(L.rope_sin, host.si.nbytes)
    kc_d = DevBuf.from_array(np.zeros_like(host.kc))
    vc_d = DevBuf.from_array(np.zeros_like(host.vc))
    bufs += [kc_d, vc_d]
    D.kc, D.vc = kc_d.ptr, vc_d.ptr
    return D, bufs, kc_d, vc_d
