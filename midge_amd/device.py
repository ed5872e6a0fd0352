"""Device runtime plumbing: init, streams and device buffers over the C ABI."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

_inited = False


def init(device: int = 0) -> None:
    """mh_init(device); idempotent."""
    global _inited
    _lib.call("mh_init", device)
    _inited = True


def shutdown() -> None:
    global _inited
    _lib.call("mh_shutdown")
    _inited = False


def sync() -> None:
    _lib.call("mh_sync")


def stream() -> int:
    """The hipStream_t every _dev call is launched on."""
    return _lib.raw("mh_get_stream")() or 0


def set_switch(name: str, on: bool) -> None:
    """mh_set_switch: a path switch ("NO_MFMA", "NO_FUSED", "ATTN_SPLIT",
    "COOP", "Q8_NO_ROWS", "BATCH_GEMV", "SPLIT_ROUTE") on or off for the
    calls that follow."""
    _lib.call("mh_set_switch", name.encode(), 1 if on else 0)


class switch:
    """`with switch("NO_FUSED"):` runs the block with a path switch on."""

    def __init__(self, name: str, on: bool = True):
        self.name, self.on = name, on

    def __enter__(self):
        set_switch(self.name, self.on)
        return self

    def __exit__(self, *exc):
        set_switch(self.name, not self.on)
        return False


def profile_enable(on: bool = True) -> None:
    _lib.call("mh_profile_enable", 1 if on else 0)


def profile_reset() -> None:
    _lib.call("mh_profile_reset")


def profile_query(name: str) -> tuple[float, int]:
    """(total ms, launches) of kernel `name` since the last reset."""
    ms = C.c_double()
    n = C.c_uint64()
    _lib.call("mh_profile_query", name.encode(), C.byref(ms), C.byref(n))
    return float(ms.value), int(n.value)


class DevBuf:
    """A device allocation (mh_alloc) with numpy upload/download helpers."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        _lib.call("mh_alloc", int(nbytes), C.byref(p))
        self.ptr = int(p.value)
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError(f"upload of {a.nbytes} B at {offset} overruns {self.nbytes} B buffer")
        if a.nbytes:
            _lib.call("mh_h2d", self.ptr + offset, a.ctypes.data, a.nbytes)

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError(f"download of {out.nbytes} B at {offset} overruns {self.nbytes} B buffer")
        if out.nbytes:
            _lib.call("mh_d2h", out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def free(self) -> None:
        if self.ptr:
            _lib.call("mh_free", self.ptr)
            self.ptr = 0

    def __int__(self) -> int:
        return self.ptr


class Region:
    """A host byte range uploaded to HBM with identical offsets
    (mh_register_region); host pointers inside it are translated."""

    def __init__(self, host: np.ndarray):
        self.host = np.ascontiguousarray(host)
        if not self.host.flags["C_CONTIGUOUS"]:
            raise ValueError("region must be contiguous")
        p = C.c_void_p()
        _lib.call("mh_register_region", self.host.ctypes.data, self.host.nbytes, C.byref(p))
        self.dev = int(p.value)
        self.base = int(self.host.ctypes.data)

    def release(self) -> None:
        if self.base:
            _lib.call("mh_unregister_region", self.base)
            self.base = 0
