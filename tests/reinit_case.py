"""Child process of test_reinit_attention_and_sampling: the library is
initialised, used, shut down and initialised again, twice over, and the
one-launch attention (its exchange words, launch tags and error flag) and
temperature sampling (its workspace counters) must give bit-identical results
in both initialisations, with mh_sync clean after each. Prints "reinit ok"."""
from __future__ import annotations

import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.dirname(HERE), HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

import midge_amd  # noqa: E402
from midge_amd import DevBuf, _lib  # noqa: E402
from midge_amd.moe import sample_dev  # noqa: E402
from attn_dev import attn_device_layer  # noqa: E402
from test_oracle_kernels import GPT_OSS_ATTN, GPT_OSS_ROPE, AttnHost  # noqa: E402

POSITIONS = 24
VOCAB = 201088


def once(host, cfg):
    midge_amd.init(0)
    D, bufs, kc_d, vc_d = attn_device_layer(host, cfg)
    H = cfg["hidden"]
    rng = np.random.default_rng(5)
    xd = DevBuf(H * 4)
    outs = []
    for pos in range(POSITIONS):
        xd.upload(rng.standard_normal(H).astype(np.float32))
        _lib.call("mh_attention_dev", ctypes.byref(D), xd.ptr, pos)
        outs.append(xd.download(np.float32, (H,)))
    logits = (rng.standard_normal(VOCAB) * 3.0).astype(np.float32)
    ld, od = DevBuf.from_array(logits), DevBuf(4)
    picks = []
    for u in (0.05, 0.37, 0.61, 0.93):
        sample_dev(ld.ptr, VOCAB, 1.0, 0.9, u, od.ptr)
        picks.append(int(od.download(np.int32, (1,))[0]))
    midge_amd.sync()   # raises if an error flag was set
    caches = (kc_d.download(np.uint16, host.kc.shape), vc_d.download(np.uint16, host.vc.shape))
    for d in bufs + [xd, ld, od]:
        d.free()
    midge_amd.shutdown()
    return outs, picks, caches


def main() -> int:
    cfg = GPT_OSS_ATTN
    host = AttnHost(**cfg, seed=13, rope=GPT_OSS_ROPE)
    print("[case] reinit: first initialisation", flush=True)
    a = once(host, cfg)
    print("[case] reinit: second initialisation", flush=True)
    b = once(host, cfg)
    for i, (x, y) in enumerate(zip(a[0], b[0])):
        assert np.array_equal(x, y), f"attention output differs at position {i}"
    assert a[1] == b[1], (a[1], b[1])
    assert all(np.array_equal(x, y) for x, y in zip(a[2], b[2])), "f16 caches differ"
    print("reinit ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
