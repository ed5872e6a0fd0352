"""mh_sample_dev_static (the allocation-free sampling entry point) against
mh_sample_dev through the C ABI: two calls in a row, the second over a
smaller vocabulary, on every selection path (greedy, the candidate sort,
the radix select over the whole vocabulary); and, in a fresh process, that
it allocates nothing when it runs before anything else has sampled."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("spread", [20.0, 0.2])
def test_sample_static_matches_sample_dev(mh, spread):
    from midge_amd import DevBuf
    from midge_amd.moe import sample_dev, sample_dev_static
    rng = np.random.default_rng(int(spread * 10))
    out_a, out_b = DevBuf(4), DevBuf(4)
    for V in (201088, 50000):      # the second call smaller than the first
        say(f"sample_dev_static spread {spread} V {V}")
        lg = (rng.standard_normal(V) * spread).astype(np.float32)
        ld = DevBuf.from_array(lg)
        for temp, topp, u in ((0.0, 1.0, 0.0), (1.0, 0.9, 0.37), (0.7, 0.5, 0.91), (1.3, 1.0, 0.05)):
            sample_dev(ld, V, temp, topp, u, out_a)
            sample_dev_static(ld, V, temp, topp, u, out_b)
            a = int(out_a.download(np.int32, (1,))[0])
            b = int(out_b.download(np.int32, (1,))[0])
            assert 0 <= b < V and a == b, (spread, V, temp, topp, u, a, b)
        ld.free()
    out_a.free()
    out_b.free()


def test_sample_static_allocates_nothing():
    # a child process: a fresh initialisation, the static entry point first,
    # under a one-byte allocation cap
    say("sample_dev_static first in a fresh process under MIDGE_HIP_MAX_BYTES=1")
    r = subprocess.run([sys.executable, "-u", os.path.join(os.path.dirname(os.path.abspath(__file__)), "no_alloc_case.py")],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "no-alloc ok" in r.stdout

