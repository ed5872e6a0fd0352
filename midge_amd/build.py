"""Build libmidge_hip.so (gfx950) in-tree, plus the oracle libraries.

    python -m midge_amd.build            # HIP library + oracle (+ reference shim if present)

The HIP library is compiled with hipcc for gfx950 only; every object is
rebuilt on each call (the build check must compile, not reuse). Objects go
to midge_amd/_build/, the library to midge_amd/libmidge_hip.so.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmidge_hip.so")
ORACLE = os.path.join(ROOT, "oracle")
REFERENCE = os.environ.get("MIDGE_REFERENCE", "/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["mh_runtime.hip", "mh_gemv.hip", "mh_moe.hip", "mh_decode.hip", "mh_prefill.hip", "mh_grouped.hip", "mh_synth.hip",
           "mh_sample.hip", "mh_attn.hip", "mh_forward.hip"]
HIPFLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
]


def _run(cmd: list[str], cwd: str | None = None) -> None:
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip(jobs: int = 8) -> str:
    """Compile every csrc/*.hip for gfx950 and link libmidge_hip.so."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    procs = []
    objs = []
    for s in srcs:
        obj = os.path.join(BUILD, s.replace(".hip", ".o"))
        objs.append(obj)
        cmd = [HIPCC, *HIPFLAGS, "-c", os.path.join(CSRC, s), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _wait(procs)
            procs = []
    _wait(procs)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def _wait(procs) -> None:
    for cmd, p in procs:
        out, _ = p.communicate()
        out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed ({p.returncode}): {' '.join(cmd)}\n{out}")
        if out.strip():
            print(out)


def build_oracle() -> None:
    """The C oracle always; the reference shim when the reference checkout exists."""
    _run(["make", "-s", "-B", "libmidge_oracle.so"], cwd=ORACLE)
    if os.path.isfile(os.path.join(REFERENCE, "engine", "midge.c")):
        _run(["make", "-s", "-B", "ref", "engines", f"REF={REFERENCE}"], cwd=ORACLE)


def main() -> int:
    build_hip()
    build_oracle()
    print(f"built {LIB}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
