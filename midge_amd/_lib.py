"""ctypes binding of libmidge_hip (include/midge_hip.h, include/midge_hip_synth.h).

The shared library is loaded from this package directory only; when it is
missing the import fails loudly (there is no CPU fallback). Every binding
checks the status code and raises MidgeHipError with mh_last_error().
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libmidge_hip.so")

# engine/mten.h:42
DT_F32, DT_Q8R, DT_Q4G32, DT_MXFP4 = 0, 1, 2, 3
DT_NAMES = {"f32": DT_F32, "q8r": DT_Q8R, "q4g32": DT_Q4G32, "mxfp4": DT_MXFP4}

MH_OK, MH_E_ARG, MH_E_DTYPE, MH_E_NOINIT, MH_E_HIP, MH_E_NOMEM, MH_E_UNREGISTERED, MH_E_RANGE, \
    MH_E_UNSUPPORTED = 0, -1, -2, -3, -4, -5, -6, -7, -8
ERROR_NAMES = {
    MH_E_ARG: "MH_E_ARG", MH_E_DTYPE: "MH_E_DTYPE", MH_E_NOINIT: "MH_E_NOINIT", MH_E_HIP: "MH_E_HIP",
    MH_E_NOMEM: "MH_E_NOMEM", MH_E_UNREGISTERED: "MH_E_UNREGISTERED", MH_E_RANGE: "MH_E_RANGE",
    MH_E_UNSUPPORTED: "MH_E_UNSUPPORTED",
}


class MidgeHipError(RuntimeError):
    def __init__(self, code: int, func: str, msg: str):
        super().__init__(f"{func}: {ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code
        self.func = func


class MhWT(C.Structure):
    """mh_wt == the reference's WT (engine/mten.h:67-72)."""
    _fields_ = [("dt", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("scales", C.c_void_p)]


class MhMoeLayer(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("ffn", C.c_int64),
                ("n_experts", C.c_int32), ("top_k", C.c_int32),
                ("alpha", C.c_float), ("limit", C.c_float), ("norm_eps", C.c_float),
                ("act_plain", C.c_int32), ("router_norm", C.c_int32), ("expert_dt", C.c_int32),
                ("expert_stride", C.c_uint64), ("off", C.c_uint64 * 9),
                ("experts", C.c_void_p), ("router", MhWT),
                ("router_b", C.c_void_p), ("mlp_norm", C.c_void_p)]


class MhAttnLayer(C.Structure):
    """mh_attn_layer: one attention layer (attention(), engine/midge.c:341-400)."""
    _fields_ = [("hidden", C.c_int64), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("ctx", C.c_int32), ("window", C.c_int32),
                ("qk_norm", C.c_int32), ("sinks", C.c_int32), ("norm_eps", C.c_float),
                ("attn_scale", C.c_float), ("wq", MhWT), ("wk", MhWT), ("wv", MhWT), ("wo", MhWT),
                ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("bo", C.c_void_p),
                ("attn_norm", C.c_void_p), ("qn", C.c_void_p), ("kn", C.c_void_p), ("sink", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("kc", C.c_void_p), ("vc", C.c_void_p)]


class MhModelDesc(C.Structure):
    """mh_model_desc: the tensors forward() reads (engine/midge.c:552-565)."""
    _fields_ = [("hidden", C.c_int64), ("vocab", C.c_int64), ("n_layers", C.c_int32), ("norm_eps", C.c_float),
                ("embed", MhWT), ("lm_head", MhWT), ("final_norm", C.c_void_p),
                ("attn", C.POINTER(MhAttnLayer)), ("moe", C.POINTER(MhMoeLayer))]


_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64
_U64 = C.c_uint64
_F = C.c_float

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGS = {
    "mh_init": [_I],
    "mh_shutdown": [],
    "mh_last_error": [],
    "mh_set_stream": [_P],
    "mh_set_switch": [C.c_char_p, _I],
    "mh_get_stream": [],
    "mh_sync": [],
    "mh_profile_enable": [_I],
    "mh_profile_reset": [],
    "mh_profile_query": [C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)],
    "mh_register_region": [_P, _U64, C.POINTER(_P)],
    "mh_unregister_region": [_P],
    "mh_alloc": [_U64, C.POINTER(_P)],
    "mh_free": [_P],
    "mh_h2d": [_P, _P, _U64],
    "mh_d2h": [_P, _P, _U64],
    "mh_matvec": [C.POINTER(MhWT), _P, _P],
    "mh_row": [C.POINTER(MhWT), _I64, _P],
    "mh_matvec_dev": [C.POINTER(MhWT), _P, _P, _I],
    "mh_dequant_dev": [C.POINTER(MhWT), _I64, _I64, _P],
    "mh_rmsnorm_dev": [_P, _P, _P, _I64, _F, _I],
    "mh_moe": [C.POINTER(MhMoeLayer), _P, _P, _P],
    "mh_moe_dev": [C.POINTER(MhMoeLayer), _P, _I, _P, _P],
    "mh_moe_prefill": [C.POINTER(MhMoeLayer), _I, _P, _P, _P],
    "mh_moe_prefill_dev": [C.POINTER(MhMoeLayer), _I, _P, _P, _P],
    "mh_topk_dev": [_P, _I, _I, _I, _I, _P, _P],
    "mh_sample_dev": [_P, _I64, _F, _F, _F, _P],
    "mh_sample_dev_static": [_P, _I64, _F, _F, _F, _P],
    "mh_attention_dev": [C.POINTER(MhAttnLayer), _P, _I],
    "mh_expert_major_dev": [C.POINTER(MhMoeLayer), _I, _P, _P, _P, _P],
    "mh_stack_create": [C.POINTER(MhMoeLayer), _I, _I, C.POINTER(_P)],
    "mh_stack_decode": [_P, _P, _I, _P, _P, _P],
    "mh_stack_apply_dev": [_P, _I, _P, _P, _P, _P],
    "mh_stack_destroy": [_P],
    "mh_model_create": [C.POINTER(MhModelDesc), C.POINTER(_P)],
    "mh_forward_dev": [_P, _I, _I, _P, _P, _P, _P],
    "mh_model_destroy": [_P],
    "mh_synth_bytes_dev": [_P, _U64, _U64],
    "mh_synth_scales_dev": [_P, _U64, _U64, _I, _I],
    "mh_synth_i8_dev": [_P, _U64, _U64],
    "mh_synth_normal_dev": [_P, _U64, _U64, _F],
    "mh_synth_uniform_dev": [_P, _U64, _U64, _F, _F],
    "mh_synth_expert_table_dev": [_P, C.POINTER(MhMoeLayer), _I, _U64, _I, _I, _F],
}
_RESTYPES = {"mh_last_error": C.c_char_p, "mh_get_stream": C.c_void_p}

_lib = None


def load() -> C.CDLL:
    """Load libmidge_hip.so from the package directory (raises if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.isfile(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m midge_amd.build` "
                          "(there is no CPU fallback)")
    lib = C.CDLL(LIB_PATH)
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib


def symbols() -> list[str]:
    return list(_SIGS)


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise MidgeHipError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != MH_OK:
        msg = lib.mh_last_error()
        raise MidgeHipError(rc, name, msg.decode() if msg else "")


def raw(name: str):
    return getattr(load(), name)
