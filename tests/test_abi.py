"""The C ABI without a GPU: the library loads, exports every entry point the
headers declare, and rejects bad input before touching the device."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from midge_amd import _lib
from midge_amd.synth import MoEShape

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def declared() -> set[str]:
    names = set()
    for h in HEADERS:
        txt = open(h).read()
        names |= set(re.findall(r"^\s*(?:int|void\s*\*|const char\s*\*)\s*(mh_\w+)\s*\(", txt, re.M))
    return names


def test_headers_declare_entry_points():
    names = declared()
    assert {"mh_init", "mh_matvec", "mh_row", "mh_moe", "mh_moe_prefill", "mh_stack_decode"} <= names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers every one of them
    assert declared() <= set(_lib.symbols())


def _rc(name, *args):
    return getattr(_lib.load(), name)(*args)


def _err() -> str:
    return _lib.load().mh_last_error().decode()


def test_unknown_dtype_is_an_error():
    t = _lib.MhWT(7, 4, 32, 1, 1)
    x = np.zeros(32, np.float32)
    y = np.zeros(4, np.float32)
    assert _rc("mh_matvec", C.byref(t), x.ctypes.data, y.ctypes.data) == _lib.MH_E_DTYPE
    assert "dtype" in _err()


def test_null_and_range_arguments():
    assert _rc("mh_matvec", None, None, None) == _lib.MH_E_ARG
    t = _lib.MhWT(_lib.DT_MXFP4, 4, 48, 1, 1)     # cols not a multiple of 32
    assert _rc("mh_row", C.byref(t), 0, 1) == _lib.MH_E_ARG
    t = _lib.MhWT(_lib.DT_F32, 4, 32, 1, 0)
    out = np.zeros(32, np.float32)
    assert _rc("mh_row", C.byref(t), 4, out.ctypes.data) == _lib.MH_E_RANGE
    assert _rc("mh_row", C.byref(t), -1, out.ctypes.data) == _lib.MH_E_RANGE
    # stack entry points: a NULL stack is refused before any device work
    assert _rc("mh_stack_apply_dev", None, 0, 1, 1, 1, 1) == _lib.MH_E_ARG
    assert _rc("mh_stack_decode", None, 1, 1, None, None, None) == _lib.MH_E_ARG


def _layer(**kw) -> _lib.MhMoeLayer:
    shape = MoEShape(hidden=64, ffn=64, n_experts=8, top_k=2)
    L = shape.layout
    c = _lib.MhMoeLayer()
    c.hidden, c.ffn, c.n_experts, c.top_k = 64, 64, 8, 2
    c.alpha, c.limit, c.norm_eps = 1.702, 7.0, 1e-5
    c.expert_dt = _lib.DT_MXFP4
    c.expert_stride = L.expert_stride
    for i, o in enumerate(L.off):
        c.off[i] = o
    c.router = _lib.MhWT(_lib.DT_Q8R, 8, 64, 1, 1)
    c.experts = c.router_b = c.mlp_norm = 1
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_layer_validation_before_device():
    x = np.zeros(64, np.float32)
    assert _rc("mh_moe", C.byref(_layer(top_k=0)), x.ctypes.data, None, None) == _lib.MH_E_ARG
    assert _rc("mh_moe", C.byref(_layer(top_k=17, n_experts=32)), x.ctypes.data, None, None) == _lib.MH_E_ARG
    assert _rc("mh_moe", C.byref(_layer(top_k=9)), x.ctypes.data, None, None) == _lib.MH_E_ARG
    bad = _layer()
    bad.off[4] += 64
    assert _rc("mh_moe", C.byref(bad), x.ctypes.data, None, None) == _lib.MH_E_ARG
    assert "off[4]" in _err()
    assert _rc("mh_moe", C.byref(_layer(expert_stride=1)), x.ctypes.data, None, None) == _lib.MH_E_ARG
    assert _rc("mh_moe", C.byref(_layer(expert_dt=9)), x.ctypes.data, None, None) == _lib.MH_E_DTYPE
    assert _rc("mh_moe_prefill", C.byref(_layer()), 0, x.ctypes.data, None, None) == _lib.MH_E_ARG


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_errors_cleanly():
    x = np.zeros(64, np.float32)
    assert _rc("mh_moe", C.byref(_layer()), x.ctypes.data, None, None) == _lib.MH_E_NOINIT
    assert _rc("mh_sync") == _lib.MH_E_NOINIT
    rc = _rc("mh_init", 0)
    assert rc == _lib.MH_E_HIP and "device" in _err()
    with pytest.raises(_lib.MidgeHipError):
        _lib.call("mh_init", 0)


def _attn(**kw) -> _lib.MhAttnLayer:
    a = _lib.MhAttnLayer()
    a.hidden, a.n_heads, a.n_kv_heads, a.head_dim, a.ctx, a.window = 64, 4, 2, 16, 32, 0
    a.norm_eps, a.attn_scale = 1e-5, 0.25
    a.wq = _lib.MhWT(_lib.DT_Q8R, 64, 64, 1, 1)
    a.wk = _lib.MhWT(_lib.DT_Q8R, 32, 64, 1, 1)
    a.wv = _lib.MhWT(_lib.DT_Q8R, 32, 64, 1, 1)
    a.wo = _lib.MhWT(_lib.DT_Q8R, 64, 64, 1, 1)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_attention_and_sample_validation_before_device():
    # argument checks come before any device work (no GPU needed)
    x = 1
    assert _rc("mh_attention_dev", None, x, 0) == _lib.MH_E_ARG
    assert _rc("mh_attention_dev", C.byref(_attn()), x, 32) == _lib.MH_E_ARG       # pos >= ctx
    assert "position" in _err()
    assert _rc("mh_attention_dev", C.byref(_attn()), x, -1) == _lib.MH_E_ARG
    assert _rc("mh_attention_dev", C.byref(_attn(n_kv_heads=3)), x, 0) == _lib.MH_E_ARG   # 4 % 3
    assert _rc("mh_attention_dev", C.byref(_attn(head_dim=15)), x, 0) == _lib.MH_E_ARG    # odd
    assert _rc("mh_attention_dev", C.byref(_attn(qk_norm=1)), x, 0) == _lib.MH_E_ARG      # no weights
    assert _rc("mh_attention_dev", C.byref(_attn(sinks=1)), x, 0) == _lib.MH_E_ARG        # no sinks
    bad = _attn()
    bad.wo = _lib.MhWT(_lib.DT_Q8R, 64, 32, 1, 1)
    assert _rc("mh_attention_dev", C.byref(bad), x, 0) == _lib.MH_E_ARG
    assert "projection" in _err()
    assert _rc("mh_sample_dev", None, 10, 0.0, 1.0, C.c_float(0.0), 1) == _lib.MH_E_ARG
    assert _rc("mh_sample_dev", 1, 0, 0.0, 1.0, C.c_float(0.0), 1) == _lib.MH_E_ARG
    assert "vocabulary" in _err()
    # the fixed-workspace variant: vocabularies beyond its 2^18 tokens are refused up front
    assert _rc("mh_sample_dev_static", 1, 262145, 0.0, 1.0, C.c_float(0.0), 1) == _lib.MH_E_ARG
    assert "fixed workspace" in _err()
    assert _rc("mh_sample_dev_static", None, 10, 0.0, 1.0, C.c_float(0.0), 1) == _lib.MH_E_ARG
