"""Kernel-level interface, named as the reference's engine/mkern.h.

    wk_matvec(t, x)      y = W x           (engine/mkern.h:180-198)
    wk_row(t, r)         dequantized row   (engine/mkern.h:201-236)

`WT` mirrors the reference's tensor view (engine/mten.h:67-72). Its data and
scales are numpy arrays (uploaded through a registered region, the way the
reference's mmap'd blobs are) or device pointers. The _dev functions take
device buffers and run asynchronously on the library stream.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .device import DevBuf, Region


@dataclass
class WT:
    dt: int
    rows: int
    cols: int
    data: object            # numpy array (host) or int device pointer
    scales: object = None   # numpy array, int device pointer or None (f32)
    _regions: list = field(default_factory=list, repr=False)

    def _ptr(self, a) -> int:
        if a is None:
            return 0
        if isinstance(a, np.ndarray):
            return int(a.ctypes.data)
        return int(a)

    def register(self) -> "WT":
        """Upload host data/scales to HBM (mh_register_region), as the engine's
        mmap'd blobs are; later calls translate the host pointers."""
        for a in (self.data, self.scales):
            if isinstance(a, np.ndarray) and a.nbytes:
                self._regions.append(Region(a))
        return self

    def release(self) -> None:
        for r in self._regions:
            r.release()
        self._regions.clear()

    def c(self) -> _lib.MhWT:
        return _lib.MhWT(self.dt, self.rows, self.cols, self._ptr(self.data), self._ptr(self.scales))


def wk_matvec(t: WT, x: np.ndarray) -> np.ndarray:
    """y[rows] = W x (host arrays, synchronous)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.shape != (t.cols,):
        raise ValueError(f"x has shape {x.shape}, expected ({t.cols},)")
    y = np.empty(t.rows, dtype=np.float32)
    ct = t.c()
    _lib.call("mh_matvec", C.byref(ct), x.ctypes.data, y.ctypes.data)
    return y


def wk_row(t: WT, r: int) -> np.ndarray:
    out = np.empty(t.cols, dtype=np.float32)
    ct = t.c()
    _lib.call("mh_row", C.byref(ct), int(r), out.ctypes.data)
    return out


def matvec_dev(t: WT, x: DevBuf | int, y: DevBuf | int, batch: int = 1) -> None:
    ct = t.c()
    _lib.call("mh_matvec_dev", C.byref(ct), int(x), int(y), int(batch))


def dequant_dev(t: WT, r0: int, n: int, out: DevBuf | int) -> None:
    ct = t.c()
    _lib.call("mh_dequant_dev", C.byref(ct), int(r0), int(n), int(out))


def rmsnorm_dev(x, w, out, n: int, eps: float, batch: int = 1) -> None:
    _lib.call("mh_rmsnorm_dev", int(x), _ptr(w), int(out), int(n), float(eps), int(batch))


def _ptr(a) -> int:
    if isinstance(a, np.ndarray):
        return int(a.ctypes.data)
    return int(a)
