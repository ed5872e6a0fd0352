"""Seeded synthetic inputs, bit-identical on the host (numpy) and the device
(include/midge_hip_synth.h). Each value is a pure function of (key, index):

    hash(key, i) = SplitMix64 finaliser of key + (i + 1) * 0x9e3779b97f4a7c15
    bytes        byte i = byte (i % 8) of hash(key, i // 8), little endian
    scales       f16 2^e, e = emin + (hash(key, i) >> 32) % (emax - emin + 1)
    int8         (16-bit field i % 4 of hash(key, i // 4)) % 255 - 127
    normal       f32(sum of the 4 16-bit fields of hash(key, i) - 131070) * c,
                 c = std / 37837.23 (Irwin-Hall(4) stand-in for N(0, std^2))
    uniform      lo + f32(hash(key, i) >> 40) * c, c = (hi - lo) / 2^24

The workload helpers build gpt-oss-shaped MoE inputs from one seed with the
distributions of the benchmark configurations: MXFP4 experts with uniform
nibbles and scales 2^e, e in [-8, -4]; expert biases ~N(0, 0.02); int8
routers uniform in [-127, 127] with row scales U(1e-3, 1e-2) and biases
~N(0, 0.2); hidden states ~N(0, 1); mlp_norm weights U[0.8, 1.2).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import DT_MXFP4, DT_Q8R
from .layout import ExpertLayout, blob_sizes

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
IH_STD = 37837.23   # std of the sum of four uniform 16-bit fields: sqrt((2^32 - 1) / 3)


def mix64(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def hash64(key: int, i) -> np.ndarray:
    i = np.asarray(i, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(key) + (i + np.uint64(1)) * _G)


def hash64_int(key: int, i: int) -> int:
    return int(hash64(key, np.uint64(i)))


def synth_bytes(key: int, n: int) -> np.ndarray:
    words = hash64(key, np.arange((n + 7) // 8, dtype=np.uint64))
    return words.view(np.uint8)[:n].copy()


def synth_scales(key: int, n: int, emin: int = -8, emax: int = -4) -> np.ndarray:
    span = np.uint64(emax - emin + 1)
    e = emin + ((hash64(key, np.arange(n, dtype=np.uint64)) >> np.uint64(32)) % span).astype(np.int64)
    return ((e + 15) << 10).astype(np.uint16)


def synth_i8(key: int, n: int) -> np.ndarray:
    i = np.arange(n, dtype=np.uint64)
    f = (hash64(key, i >> np.uint64(2)) >> (np.uint64(16) * (i & np.uint64(3)))) & np.uint64(0xFFFF)
    return ((f % np.uint64(255)).astype(np.int64) - 127).astype(np.int8)


def normal_c(std: float) -> np.float32:
    return np.float32(std / IH_STD)


def synth_normal(key: int, n: int, c) -> np.ndarray:
    h = hash64(key, np.arange(n, dtype=np.uint64))
    m = np.uint64(0xFFFF)
    s = ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m) + (h >> np.uint64(48))).astype(np.int64)
    return (s - 131070).astype(np.float32) * np.float32(c)


def uniform_c(lo: float, hi: float) -> np.float32:
    return np.float32((hi - lo) / float(1 << 24))


def synth_uniform(key: int, n: int, lo, c) -> np.ndarray:
    h = hash64(key, np.arange(n, dtype=np.uint64))
    return np.float32(lo) + (h >> np.uint64(40)).astype(np.float32) * np.float32(c)


# ------------------------------------------------------------ workloads

EXPERT_EMIN, EXPERT_EMAX = -8, -4
EXPERT_BIAS_STD = 0.02
ROUTER_SCALE_LO, ROUTER_SCALE_HI = 1e-3, 1e-2
ROUTER_BIAS_STD = 0.2
NORM_LO, NORM_HI = 0.8, 1.2


@dataclass(frozen=True)
class MoEShape:
    hidden: int = 2880
    ffn: int = 2880
    n_experts: int = 32
    top_k: int = 4
    n_layers: int = 1
    expert_dt: int = DT_MXFP4
    router_dt: int = DT_Q8R
    alpha: float = 1.702
    limit: float = 7.0
    norm_eps: float = 1e-5
    act_plain: int = 0
    router_norm: int = 1

    @property
    def layout(self) -> ExpertLayout:
        return ExpertLayout(self.expert_dt, self.hidden, self.ffn, self.n_experts)


class Keys:
    """Per-purpose keys derived from one seed."""

    def __init__(self, seed: int):
        self.seed = seed
        self.table = hash64_int(seed, 1)
        self.router_w = hash64_int(seed, 2)
        self.router_s = hash64_int(seed, 3)
        self.router_b = hash64_int(seed, 4)
        self.norm = hash64_int(seed, 5)
        self.x = hash64_int(seed, 6)

    def layer(self, base: int, layer: int) -> int:
        return hash64_int(base, layer)


def expert_blob_keys(table_key: int, n_experts: int, layer: int, expert: int, mat: int) -> tuple[int, int, int]:
    kb = ((layer * n_experts + expert) * 3 + mat) * 3
    return tuple(hash64_int(table_key, kb + p) for p in range(3))


def host_expert(shape: MoEShape, keys: Keys, layer: int, expert: int) -> np.ndarray:
    """One expert's bytes (gate, up, down blobs at the layout offsets)."""
    L = shape.layout
    out = np.zeros(L.expert_stride, dtype=np.uint8)
    for m in range(3):
        kd, ks, kb = expert_blob_keys(keys.table, shape.n_experts, layer, expert, m)
        db, sb = blob_sizes(shape.expert_dt, L.rows[m], L.cols[m])
        off = L.off[3 * m:3 * m + 3]
        out[off[0]:off[0] + db] = synth_bytes(kd, db)
        out[off[1]:off[1] + sb] = synth_scales(ks, sb // 2, EXPERT_EMIN, EXPERT_EMAX).view(np.uint8)
        out[off[2]:off[2] + 4 * L.rows[m]] = synth_normal(kb, L.rows[m], normal_c(EXPERT_BIAS_STD)).view(np.uint8)
    return out


def host_layer_experts(shape: MoEShape, keys: Keys, layer: int) -> np.ndarray:
    L = shape.layout
    out = np.empty(L.layer_stride, dtype=np.uint8)
    for e in range(shape.n_experts):
        out[e * L.expert_stride:(e + 1) * L.expert_stride] = host_expert(shape, keys, layer, e)
    return out


def host_router(shape: MoEShape, keys: Keys, layer: int):
    """(int8 weights [E][hidden], f32 row scales [E], f32 bias [E], f32 mlp_norm [hidden])."""
    E, H = shape.n_experts, shape.hidden
    w = synth_i8(keys.layer(keys.router_w, layer), E * H).reshape(E, H)
    s = synth_uniform(keys.layer(keys.router_s, layer), E, ROUTER_SCALE_LO,
                      uniform_c(ROUTER_SCALE_LO, ROUTER_SCALE_HI))
    b = synth_normal(keys.layer(keys.router_b, layer), E, normal_c(ROUTER_BIAS_STD))
    nw = synth_uniform(keys.layer(keys.norm, layer), H, NORM_LO, uniform_c(NORM_LO, NORM_HI))
    return w, s, b, nw


def host_x(shape: MoEShape, keys: Keys, batch: int, step: int = 0) -> np.ndarray:
    return synth_normal(keys.layer(keys.x, step), batch * shape.hidden, normal_c(1.0)).reshape(batch, shape.hidden)
