"""Write tests/golden/attn_divergence.npz: the reference's own AVX2-vs-scalar
divergence on attention() per decode position at the gpt-oss shape (the
bar the GPU attention test holds each position to).

The reference engine is compiled from its own sources by `make -C oracle ref`
(oracle/_ref/, where the reference checkout exists).

    python tests/golden/make_attn_divergence.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.dirname(HERE)]

from test_oracle_kernels import ATTN_DIV_FIXTURE, GPT_OSS_ATTN, attn_divergence_gptoss  # noqa: E402

if __name__ == "__main__":
    div = attn_divergence_gptoss()
    np.savez(ATTN_DIV_FIXTURE, div=div, cfg=np.array(sorted(GPT_OSS_ATTN.items()), dtype=object).astype(str),
             seeds=np.array([13, 14]))
    print(f"wrote {ATTN_DIV_FIXTURE}: {len(div)} positions, max {div.max():.3g} at {int(div.argmax())}, "
          f"mean {div.mean():.3g}, > 1e-3 at {np.flatnonzero(div > 1e-3).tolist()}")
