"""The deterministic expert layout of experts.midge.

Mirrors wt_expert_layout() (engine/mten.h:101-150) and ExpertLayout
(tools/midgepack.py:166-205): per layer, per expert, for each matrix of
(gate, up, down) the data blob, the scales blob and an f32 bias, each
64-byte aligned; the expert stride is the 64-aligned end.
"""
from __future__ import annotations

from dataclasses import dataclass

from ._lib import DT_F32, DT_MXFP4, DT_Q4G32, DT_Q8R

MATS = ("gate", "up", "down")
PARTS = ("data", "scales", "bias")


def align64(x: int) -> int:
    return (x + 63) & ~63


def blob_sizes(dt: int, rows: int, cols: int) -> tuple[int, int]:
    """(data bytes, scale bytes) of a [rows x cols] matrix (engine/mten.h:101-109)."""
    if dt == DT_F32:
        return rows * cols * 4, 0
    if dt == DT_Q8R:
        return rows * cols, rows * 4
    if dt in (DT_Q4G32, DT_MXFP4):
        if cols % 32:
            raise ValueError(f"4-bit g32 matrix needs cols % 32 == 0, got {cols}")
        return rows * cols // 2, rows * (cols // 32) * 2
    raise ValueError(f"unknown dtype {dt}")


@dataclass(frozen=True)
class ExpertLayout:
    dt: int
    hidden: int
    ffn: int
    n_experts: int

    @property
    def rows(self) -> tuple[int, int, int]:
        return (self.ffn, self.ffn, self.hidden)

    @property
    def cols(self) -> tuple[int, int, int]:
        return (self.hidden, self.hidden, self.ffn)

    def _walk(self) -> tuple[tuple[int, ...], int]:
        o, out = 0, []
        for m in range(3):
            db, sb = blob_sizes(self.dt, self.rows[m], self.cols[m])
            out.append(o)
            o = align64(o + db)
            out.append(o)
            o = align64(o + sb)
            out.append(o)
            o = align64(o + self.rows[m] * 4)
        return tuple(out), align64(o)

    @property
    def off(self) -> tuple[int, ...]:
        """off[3*m + p] for m in (gate, up, down), p in (data, scales, bias)."""
        return self._walk()[0]

    @property
    def expert_stride(self) -> int:
        return self._walk()[1]

    @property
    def layer_stride(self) -> int:
        return self.expert_stride * self.n_experts

    def offset(self, layer: int, expert: int, mat: int, part: int) -> int:
        return layer * self.layer_stride + expert * self.expert_stride + self.off[3 * mat + part]
