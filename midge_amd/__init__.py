"""midge_amd — MI355X (gfx950) implementation of midge's quantized-MoE hot path.

The compute lives in libmidge_hip.so (HIP kernels behind the C ABI in
include/midge_hip.h). This package is the host-side mirror of the
reference's interface for that path: kern (engine/mkern.h's wk_matvec /
wk_row), moe (engine/midge.c's moe / route_topk / expert-major prefill),
layout (engine/mten.h's expert layout) and synth (seeded inputs).
"""
from ._lib import (DT_F32, DT_MXFP4, DT_Q4G32, DT_Q8R, LIB_PATH, MidgeHipError, load)
from .device import DevBuf, Region, init, set_switch, shutdown, stream, switch, sync
from .layout import ExpertLayout

__all__ = ["DT_F32", "DT_Q8R", "DT_Q4G32", "DT_MXFP4", "LIB_PATH", "MidgeHipError", "load", "DevBuf",
           "Region", "init", "set_switch", "shutdown", "stream", "switch", "sync", "ExpertLayout"]
