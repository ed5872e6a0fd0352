"""The reference engine's own host (engine/midge.c, built from its sources
by oracle/Makefile) on a gpt-oss-shaped model written through
midge_amd.container: the containers load and the protocol answers (CPU)."""
import json
import os

import numpy as np
import pytest

import engine_model as em
from midge_amd.container import expert_layout_of, map_data, read_header

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MIDGED = os.path.join(ROOT, "oracle", "_ref", "midged")


def test_containers_round_trip(tmp_path):
    sp = em.write_model(str(tmp_path), n_layers=2, vocab=512, n_experts=4)
    hdr, base = read_header(str(tmp_path / "dense.midge"))
    assert hdr["kind"] == "dense" and hdr["spec"] == json.loads(json.dumps(sp)) and base % 64 == 0
    t = hdr["tensors"]
    assert t["embed"] == {"dt": "q8r", "shape": [512, 2880], "off": 0, "soff": 512 * 2880}
    assert all(e["off"] % 64 == 0 and e.get("soff", 0) % 64 == 0 for e in t.values())
    assert t["L1.router.w"]["dt"] == "f32" and "soff" not in t["L1.router.w"]
    ehdr, data = map_data(str(tmp_path / "experts.midge"))
    lay = expert_layout_of(sp, ehdr)
    assert ehdr == {"midge": 1, "kind": "experts", "dt": "mxfp4"} and data.size == 2 * lay.layer_stride
    sc = data[lay.offset(1, 3, 2, 1):][:16].view(np.uint16)     # down scales of layer 1, expert 3
    assert ((sc >> 10) >= 7).all() and ((sc >> 10) <= 11).all() and not (sc & 0x3FF).any()


@pytest.mark.skipif(not os.path.exists(MIDGED), reason="reference engine not built (oracle/_ref)")
def test_reference_engine_runs_the_model(tmp_path):
    sp = em.write_model(str(tmp_path), n_layers=2, vocab=1024)
    ids = em.prompt(40, sp["vocab"])
    lg, toks, done, err = em.run_engine(MIDGED, str(tmp_path), f"tfall: {' '.join(map(str, ids))}\ngen: 4\nquit\n",
                                        ctx=128)
    assert "layers=2 experts=32 topk=4 hidden=2880" in err
    assert len(lg) == 40 and all(r.shape == (1024,) and np.isfinite(r).all() for r in lg)
    assert len(toks) == 4 and toks[0] == int(np.argmax(lg[-1]))
    assert done[0][:2] == [40, 0] and done[1][1] == 4
