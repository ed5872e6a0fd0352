"""Child process of test_sample_static_allocates_nothing: in a fresh
initialisation, mh_sample_dev_static runs before anything else has used the
sampling path, under an allocation cap of one byte (MIDGE_HIP_MAX_BYTES=1:
any device allocation the library attempted would fail with MH_E_NOMEM),
on two vocabularies in a row, the second smaller; then, without the cap,
mh_sample_dev must pick the same tokens. Prints "no-alloc ok"."""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

import midge_amd  # noqa: E402
from midge_amd import DevBuf  # noqa: E402
from midge_amd.moe import sample_dev, sample_dev_static  # noqa: E402

CASES = ((0.0, 1.0, 0.0), (1.0, 0.9, 0.37), (0.7, 0.5, 0.91), (1.3, 1.0, 0.05))


def main() -> int:
    midge_amd.init(0)
    rng = np.random.default_rng(7)
    bufs = []
    for V, spread in ((201088, 0.2), (50000, 20.0)):
        bufs.append((V, DevBuf.from_array((rng.standard_normal(V) * spread).astype(np.float32))))
    out = DevBuf(4)
    os.environ["MIDGE_HIP_MAX_BYTES"] = "1"
    try:
        got = []
        for V, ld in bufs:
            print(f"[case] no-alloc: mh_sample_dev_static V {V} under a 1-byte cap", flush=True)
            for temp, topp, u in CASES:
                sample_dev_static(ld, V, temp, topp, u, out)
                got.append(int(out.download(np.int32, (1,))[0]))
        midge_amd.sync()
    finally:
        del os.environ["MIDGE_HIP_MAX_BYTES"]
    want = []
    for V, ld in bufs:
        for temp, topp, u in CASES:
            sample_dev(ld, V, temp, topp, u, out)
            want.append(int(out.download(np.int32, (1,))[0]))
    assert got == want, (got, want)
    print("no-alloc ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
