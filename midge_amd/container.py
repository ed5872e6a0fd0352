"""midge's container files: dense.midge and experts.midge.

The format is the reference's (engine/mten.h:1-31, read by wf_open at
engine/mten.h:84-98, written by tools/midgepack.py's writers):

    [u64 LE header_len][header JSON][zero pad to a 64-byte boundary][data ...]

    dense.midge    {"midge": 1, "kind": "dense", "spec": {...},
                    "tensors": {name: {"dt": ..., "shape": [r, c] | [n],
                                       "off": o, "soff": s}}}
                   offsets relative to the data start; every blob 64-aligned
    experts.midge  {"midge": 1, "kind": "experts", "dt": "mxfp4" | ...}
                   blobs at wt_expert_layout() offsets (midge_amd.layout)

Used to hand the GPU-linked engine and the CPU engine the same model, and to
read the expert region of a real container for upload (mh_register_region).
"""
from __future__ import annotations

import json
import struct

import numpy as np

from ._lib import DT_F32, DT_MXFP4, DT_Q4G32, DT_Q8R
from .layout import ExpertLayout, align64, blob_sizes

DT_STR = {DT_F32: "f32", DT_Q8R: "q8r", DT_Q4G32: "q4g32", DT_MXFP4: "mxfp4"}
STR_DT = {v: k for k, v in DT_STR.items()}


def header_bytes(hdr: dict) -> bytes:
    blob = json.dumps(hdr).encode()
    head = struct.pack("<Q", len(blob)) + blob
    return head + b"\0" * (align64(len(head)) - len(head))


class DenseFile:
    """Collects dense tensors (already encoded blobs) and writes dense.midge."""

    def __init__(self, spec: dict):
        self.spec = spec
        self.index: dict = {}
        self.parts: list[bytes] = []
        self.off = 0

    def _put(self, blob: bytes) -> int:
        at = self.off
        self.parts.append(blob + b"\0" * (align64(len(blob)) - len(blob)))
        self.off = align64(self.off + len(blob))
        return at

    def add_vector(self, name: str, v: np.ndarray) -> None:
        v = np.ascontiguousarray(v, np.float32)
        self.index[name] = {"dt": "f32", "shape": [int(v.size)], "off": self._put(v.tobytes())}

    def add_matrix(self, name: str, dt: int, rows: int, cols: int, data: bytes, scales: bytes = b"") -> None:
        db, sb = blob_sizes(dt, rows, cols)
        if len(data) != db or len(scales) != sb:
            raise ValueError(f"{name}: blob sizes {len(data)}/{len(scales)}, expected {db}/{sb}")
        e = {"dt": DT_STR[dt], "shape": [rows, cols], "off": self._put(data)}
        if sb:
            e["soff"] = self._put(scales)
        self.index[name] = e

    def write(self, path: str) -> None:
        hdr = {"midge": 1, "kind": "dense", "spec": self.spec, "tensors": self.index}
        with open(path, "wb") as f:
            f.write(header_bytes(hdr))
            for p in self.parts:
                f.write(p)


def write_experts(path: str, dt: int, layers) -> None:
    """experts.midge whose data is the concatenation of `layers` (byte arrays,
    e.g. one per layer, in wt_expert_layout order), written as they come."""
    with open(path, "wb") as f:
        f.write(header_bytes({"midge": 1, "kind": "experts", "dt": DT_STR[dt]}))
        for t in layers:
            f.write(memoryview(np.ascontiguousarray(t, np.uint8)))


def read_header(path: str) -> tuple[dict, int]:
    """(header, byte offset of the 64-aligned data start)."""
    with open(path, "rb") as f:
        (hl,) = struct.unpack("<Q", f.read(8))
        hdr = json.loads(f.read(hl))
    return hdr, align64(8 + hl)


def map_data(path: str) -> tuple[dict, np.ndarray]:
    """Header and a read-only memory map of the data region."""
    hdr, base = read_header(path)
    return hdr, np.memmap(path, dtype=np.uint8, mode="r", offset=base)


def expert_layout_of(spec: dict, experts_hdr: dict) -> ExpertLayout:
    moe = spec["moe"]
    return ExpertLayout(STR_DT[experts_hdr["dt"]], int(spec["hidden"]), int(moe["ffn"]), int(moe["experts"]))
