"""The kernel-level drop-in at model scale. The header registers a tensor's
data and scales as two regions the first time the engine uses it
(include/midge_hip_kern.h, wk_gpu_resident, on engine/mkern.h:180-198's
wk_matvec): a lazily driven gpt-oss-120b holds about 28,000 of them, and
every GEMV resolves its host pointers among them. Here 28,000 regions cut
from one host arena (blobs of 256 B to 2 KB), then q8r GEMVs whose data and
scales sit in regions at the start, the middle and the end of the table,
against the oracle's mv_q8r restatement; the host time per call is
reported."""
import ctypes as C
import time

import numpy as np
import pytest

from conftest import rel_l2, say
from midge_amd import DT_Q8R, _lib
from midge_amd.kern import WT, wk_matvec
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu

N_REGIONS = 28000
COLS = 64


def test_gemv_among_28000_regions(mh):
    rng = np.random.default_rng(4)
    sizes = rng.integers(4, 33, N_REGIONS) * 64            # 256 B .. 2 KB per blob
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    arena = rng.integers(-127, 128, int(offs[-1]), dtype=np.int8)
    # tensors: data in region k (rows x 64 int8), scales in region k + 1
    picks = (0, 1, N_REGIONS // 2, N_REGIONS - 2)
    shapes = {}
    for k in picks:
        rows = int(sizes[k]) // COLS
        sc = (rng.random(rows) * 6e-3 + 2e-3).astype(np.float32)
        arena[offs[k + 1]:offs[k + 1] + 4 * rows] = sc.view(np.int8)
        shapes[k] = rows
    base = arena.ctypes.data
    registered = []
    t0 = time.perf_counter()
    try:
        for i in range(N_REGIONS):
            p = C.c_void_p()
            _lib.call("mh_register_region", base + int(offs[i]), int(sizes[i]), C.byref(p))
            registered.append(base + int(offs[i]))
        t_reg = time.perf_counter() - t0
        x = rng.standard_normal(COLS).astype(np.float32)
        for k in picks:
            rows = shapes[k]
            w = arena[offs[k]:offs[k] + rows * COLS]
            s = arena[offs[k + 1]:offs[k + 1] + 4 * rows].view(np.float32)
            t = WT(DT_Q8R, rows, COLS, w, s)
            got = wk_matvec(t, x)
            want = po.matvec(DT_Q8R, w.reshape(rows, COLS), s, x, rows, COLS)
            assert rel_l2(got, want) < 1e-5, (k, rel_l2(got, want))
        # the lookup cost: host calls on the last tensor (two resolves each)
        k = picks[-1]
        rows = shapes[k]
        t = WT(DT_Q8R, rows, COLS, arena[offs[k]:offs[k] + rows * COLS],
               arena[offs[k + 1]:offs[k + 1] + 4 * rows].view(np.float32))
        n = 500
        t1 = time.perf_counter()
        for _ in range(n):
            wk_matvec(t, x)
        per_call = (time.perf_counter() - t1) / n
        say(f"{N_REGIONS} regions registered in {t_reg:.2f} s; a host mh_matvec among them "
            f"(upload x, GEMV, download y, two lookups) {per_call * 1e6:.1f} us per call")
        # a pointer between regions is not resolved (the arena's padding
        # gaps do not exist here, so use one past the last region's end)
        end = base + int(offs[-1])
        bad = _lib.MhWT(DT_Q8R, 1, COLS, end, end)
        xs, ys = np.zeros(COLS, np.float32), np.zeros(1, np.float32)
        assert _lib.load().mh_matvec(C.byref(bad), xs.ctypes.data, ys.ctypes.data) == _lib.MH_E_UNREGISTERED
    finally:
        for b in registered:
            _lib.call("mh_unregister_region", b)
