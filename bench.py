"""Benchmark: gpt-oss-120b-shape MoE expert-stack decode on one MI355X.

Workload (one step): 36 MoE layers x 128 MXFP4 experts (2880 x 2880 gate, up,
down; ~60 GiB resident in HBM, generated on the device from a seeded hash),
int8 routers 128 x 2880 with f32 row scales, top-4 softmax routing, clamped
SwiGLU, weighted sum and residual, for a batch of tokens (default 1).
Attention and the dense trunk are excluded. Every step starts from a fresh
seeded hidden state, so routing - and the experts read - differ per step.

Prints ONE JSON line. `value` is decode tokens per second. `roofline` is the
dominant kernel: at batch 1 the whole step is one launch (k_decode_step),
timed with HIP events on the library stream over the timed region;
algorithmic bytes per launch (every weight, scale, bias and router byte the
step must read, once) / launch duration, against 8 TB/s. `traffic` is the
HBM bytes per launch measured by rocprofv3 (profiles/). `cpu_baseline` is the
reference engine (built from its own sources into oracle/_ref) running moe()
on the host cores over one resident 128-expert layer, scaled to 36 layers.

    python bench.py [--steps K] [--warmup W] [--batch B] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "MoE decode tok/s (gpt-oss-120b shape, 1 GPU) + MXFP4 GEMV % HBM peak"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent timing on a given stream (the library's), via the HIP runtime
    the library already loaded."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]
        self.hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.hip.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream: int) -> None:
        assert self.hip.hipEventRecord(e, C.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.hip.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return float(ms.value)


def gu_bytes_grouped(shape, assignments: int, unique: float) -> float:
    """Algorithmic bytes of one expert-grouped gate/up launch: the gate and
    up data + f16 scales + f32 biases of each routed expert once, the normed
    inputs and the activations written per assignment."""
    L = shape.layout
    per_mat = L.rows[0] * L.cols[0] // 2 + L.rows[0] * (L.cols[0] // 32) * 2 + L.rows[0] * 4
    return unique * 2 * per_mat + assignments * (shape.ffn * 4 + shape.hidden * 4)


def gu_bytes_per_launch(shape, assignments: int) -> int:
    """Algorithmic bytes of one expert gate/up launch: per routed (token,
    expert) pair the gate and up data + f16 scales + f32 bias, the normed input
    and the activation written."""
    L = shape.layout
    per_mat = L.rows[0] * L.cols[0] // 2 + L.rows[0] * (L.cols[0] // 32) * 2 + L.rows[0] * 4
    return assignments * (2 * per_mat + shape.ffn * 4) + assignments * shape.hidden * 4


def step_bytes(shape, batch: int, unique_per_layer: float) -> float:
    """Algorithmic HBM bytes of one decode step: every routed expert's three
    matrices (data + scales + bias) once, plus the routers and norm weights."""
    L = shape.layout
    router = shape.n_experts * shape.hidden + shape.n_experts * 4 * 2 + shape.hidden * 4
    return shape.n_layers * (unique_per_layer * L.expert_stride + router) + 2 * batch * shape.hidden * 4


def run_gpu(args, shape):
    import midge_amd
    from midge_amd import DevBuf, _lib, synth
    from midge_amd.device import profile_enable, profile_query, profile_reset, stream

    midge_amd.init(0)
    t0 = time.time()
    from midge_amd.moe import Stack
    st, bufs, keys = Stack.synthetic(shape, args.seed, max(args.batch, 16))
    midge_amd.sync()
    log(f"expert table {shape.n_layers} x {shape.n_experts} experts "
        f"({shape.layout.layer_stride * shape.n_layers / 2**30:.2f} GiB) generated in {time.time() - t0:.1f}s")
    ev = HipEvents()
    s = stream()
    if args.copy_calib_mib:
        # a plain device-to-device copy of known size (the runtime's copy
        # kernel), for scaling the HBM byte counters of a --pmc run
        n = args.copy_calib_mib << 20
        src, dst = DevBuf(n), DevBuf(n)
        for _ in range(2):
            assert ev.hip.hipMemcpy(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), n, 3) == 0   # device to device
        assert ev.hip.hipDeviceSynchronize() == 0
        src.free()
        dst.free()
        log(f"copy calibration: 2 x {args.copy_calib_mib} MiB device-to-device")

    def inputs(n_steps: int, batch: int, salt: int) -> DevBuf:
        xs = DevBuf(n_steps * batch * shape.hidden * 4)
        _lib.call("mh_synth_normal_dev", xs.ptr, n_steps * batch * shape.hidden,
                  synth.hash64_int(keys.x, salt), float(synth.normal_c(1.0)))
        return xs

    def timed(batch: int, steps: int, warmup: int, salt: int, sel=None):
        xs = inputs(steps + warmup, batch, salt)
        stride = batch * shape.hidden * 4
        for i in range(warmup):
            st.decode(xs.ptr + i * stride, batch)
        midge_amd.sync()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for i in range(steps):
            st.decode(xs.ptr + (warmup + i) * stride, batch, sel)
        ev.record(b, s)
        ms = ev.elapsed_ms(a, b)
        midge_amd.sync()
        xs.free()
        return ms

    ms = timed(args.batch, args.steps, args.warmup, 1)
    log(f"batch {args.batch}: {ms / args.steps:.3f} ms/step")

    # unique experts per layer actually touched (for the step's algorithmic bytes)
    nl, k = shape.n_layers, shape.top_k
    sel = DevBuf(nl * args.batch * k * 4)
    xs = inputs(1, args.batch, 7)
    st.decode(xs.ptr, args.batch, sel.ptr)
    routed = sel.download(np.int32, (nl, args.batch, k))
    unique = float(np.mean([len(np.unique(routed[l])) for l in range(nl)]))
    sel.free()
    xs.free()

    extra = {}
    if args.batch == 1 and not args.no_b16:
        ms16 = timed(16, max(args.steps // 2, 5), 2, 2)
        sel = DevBuf(nl * 16 * k * 4)
        xs = inputs(1, 16, 8)
        st.decode(xs.ptr, 16, sel.ptr)
        r16 = sel.download(np.int32, (nl, 16, k))
        u16 = float(np.mean([len(np.unique(r16[l])) for l in range(nl)]))
        sel.free()
        xs.free()
        n16 = max(args.steps // 2, 5)
        extra["batch16"] = {"tok_per_s": 16 * n16 / (ms16 / 1e3), "ms_per_step": ms16 / n16,
                            "unique_experts_per_layer": u16,
                            "hbm_GBps": step_bytes(shape, 16, u16) / (ms16 / n16 / 1e3) / 1e9}
        log(f"batch 16: {ms16 / n16:.3f} ms/step, {u16:.1f} unique experts/layer")

    # dominant kernel: per-launch HIP-event timing on the library stream
    profile_reset()
    profile_enable(True)
    xs = inputs(args.prof_steps, args.batch, 3)
    for i in range(args.prof_steps):
        st.decode(xs.ptr + i * args.batch * shape.hidden * 4, args.batch)
    midge_amd.sync()
    kern = {}
    # per-layer phase spans of the one-launch step: mean over blocks, and the slowest block
    # (k_decode_grp's spans, then k_decode_step's; a name the run's kernel does not stamp is absent)
    spans = ("layer", "x_wait", "router", "route", "route0_gather", "route0_rank", "route0_weights",
             "route0_publish", "gu_issue", "gu_math", "gu_reduce", "h_publish", "dn_stage", "h_wait", "dn_math",
             "y_publish", "combine", "gate_up", "gu_epilogue", "barrier_arrive_prefetch", "barrier_wait",
             "down_combine", "dn_hload", "dn_reduce", "dn_combine", "tail", "gu_first_pair", "gu_mid_pair",
             "gu_last_pair", "gu_wave7_lag", "gu_barrier")
    phases = tuple(f"decode_step/{n}{m}" for n in spans for m in ("", ".max")) + tuple(
        f"decode_step/crit_{n}" for n in ("logits", "routed", "h", "x")) + tuple(
        f"decode_step/t{st:02d}.{w}" for st in (0, 15, 1, 16, 17, 18, 2, 9, 19, 20, 10, 21, 22, 11, 3, 4, 5, 12, 13,
                                                14, 6, 7)
        for w in ("first", "last"))
    for name in ("decode_step", "grouped_gu", "grouped_down", "expert_gu", "expert_down", "combine_route", "gemv",
                 "topk", "rmsnorm", "combine_norm", "combine_decode") + phases:
        tot, n = profile_query(name)
        if n:
            kern[name] = {"avg_us": 1e3 * tot / n, "launches": n}
    profile_enable(False)
    xs.free()
    if "decode_step" in kern:
        # one launch per step: the timed region's event time per step is the
        # launch's average duration (the profiled launches also write phase
        # stamps and run a few percent slower)
        dom = {"name": "k_decode_grp (all layers of a step in one launch)",
               "bytes": step_bytes(shape, args.batch, unique), "avg_us": ms / args.steps * 1e3,
               "profiled_avg_us": kern["decode_step"]["avg_us"]}
        tpath = os.path.join(ROOT, "profiles", "decode_step_120b_b1_traffic.json")
        if args.batch == 1 and shape.n_layers == 36 and shape.n_experts == 128 and os.path.exists(tpath):
            with open(tpath) as f:
                dom["traffic"] = json.load(f)["traffic_bytes"]
            dom["traffic_source"] = "profiles/decode_step_120b_b1_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE)"
    elif "grouped_gu" in kern:
        # each routed expert's gate/up read once per group of its tokens
        dom = {"name": "k_grouped<0> (expert-grouped gate/up on the f16 matrix cores + clamped SwiGLU)",
               "bytes": gu_bytes_grouped(shape, args.batch * k, unique), "avg_us": kern["grouped_gu"]["avg_us"]}
    else:
        dom = {"name": "expert_gu (fused gate/up MXFP4 GEMV + clamped SwiGLU)",
               "bytes": gu_bytes_per_launch(shape, args.batch * k), "avg_us": kern["expert_gu"]["avg_us"]}
    dom["GBps"] = dom["bytes"] / (dom["avg_us"] * 1e-6) / 1e9
    extra["gemv"] = gemv_probe(ev, s)
    if not args.no_refbench:
        extra["reference_bench"] = reference_bench(ev, s)
    if not args.no_configs:
        extra["configs"] = config_probes(ev, s, args.seed)
    if not args.no_prefill:
        extra["prefill"] = prefill_probe(ev, s, args.seed)
    if not args.no_configs:
        extra["lm_head_sample"] = lm_head_sample_probe(ev, s)
        extra["attention"] = attention_probe(ev, s)
        extra["full_token"] = full_token_probe(ev, s, st, shape)
    if not args.no_engine:
        extra["engine_host"] = engine_host_probe()
    for b in bufs:
        b.free()
    st.destroy()
    return ms, unique, kern, dom, extra


class DeviceSampler:
    """Samples the GPU's power, clock level and temperatures from sysfs
    (amdgpu hwmon and pp_dpm_sclk of the first card that has them) on a
    background thread, every `period` seconds, with host timestamps."""

    def __init__(self, period: float = 0.002):
        import glob
        import threading
        self.period, self.samples, self.stop_ev = period, [], threading.Event()
        self.dev = next((d for d in sorted(glob.glob("/sys/class/drm/card*/device"))
                         if glob.glob(d + "/hwmon/hwmon*/power1_input")), None)
        self.hw = glob.glob(self.dev + "/hwmon/hwmon*")[0] if self.dev else None
        self.th = threading.Thread(target=self._run, daemon=True)

    def _read(self, path: str) -> str | None:
        try:
            with open(path) as f:
                return f.read()
        except OSError:
            return None

    def _run(self) -> None:
        while not self.stop_ev.is_set():
            t = time.perf_counter()
            p = self._read(self.hw + "/power1_input")
            t2, t3 = self._read(self.hw + "/temp2_input"), self._read(self.hw + "/temp3_input")
            sclk = None
            txt = self._read(self.dev + "/pp_dpm_sclk") or ""
            for ln in txt.splitlines():
                if ln.strip().endswith("*"):
                    sclk = float(ln.split(":")[1].strip().rstrip("*").strip().lower().rstrip("mhz"))
            self.samples.append((t, float(p) / 1e6 if p else None, sclk, float(t2) / 1e3 if t2 else None,
                                 float(t3) / 1e3 if t3 else None))
            self.stop_ev.wait(self.period)

    def __enter__(self):
        if self.hw:
            self.th.start()
        return self

    def __exit__(self, *a):
        self.stop_ev.set()
        if self.hw:
            self.th.join()


def gemv_probe(ev, s, rows: int = 524288, cols: int = 2880, reps: int = 8, sustain: int = 30,
               sustain_s: float = 0.8) -> dict:
    """The MXFP4 GEMV engine alone: y = W x over a 524288 x 2880 matrix
    (849 MB of nibbles + f16 scales, over three times the 256 MB Infinity
    Cache).

    `avg_us` is per launch over `reps` back-to-back launches (~1.2 ms)
    between one pair of HIP events, the few microseconds between launches
    included. A longer back-to-back run (`sustain` launches, ~4.5 ms of
    streaming) is reported beside it, timed in groups of 5, first and last
    group. `sustained_1s` streams for `sustain_s` seconds, timed in groups of
    10, with the device's power, clock level and temperatures sampled from
    sysfs meanwhile, in windows of 5 ms (the first 50 ms) and 50 ms;
    `control_2x` does the same over a
    matrix twice as large (1.7 GB), so that no cache holds a useful part of
    either."""
    import midge_amd
    from midge_amd import DT_MXFP4, DevBuf, _lib, synth
    from midge_amd.kern import WT, matvec_dev

    def make(r: int):
        data, sc = DevBuf(r * cols // 2), DevBuf(r * cols // 32 * 2)
        y = DevBuf(r * 4)
        _lib.call("mh_synth_bytes_dev", data.ptr, r * cols // 2, 11)
        _lib.call("mh_synth_scales_dev", sc.ptr, r * cols // 32, 12, -8, -4)
        return WT(DT_MXFP4, r, cols, data.ptr, sc.ptr), [data, sc, y], y

    x = DevBuf(cols * 4)
    _lib.call("mh_synth_normal_dev", x.ptr, cols, 13, float(synth.normal_c(1.0)))
    t, bufs, y = make(rows)
    for _ in range(3):
        matvec_dev(t, x, y)
    midge_amd.sync()

    def launches(tt, yy, n: int, group: int) -> list:
        """Per-launch us of each group of `group` back-to-back launches."""
        evs = [ev.event() for _ in range(n // group + 1)]
        ev.record(evs[0], s)
        for i in range(n // group):
            for _ in range(group):
                matvec_dev(tt, x, yy)
            ev.record(evs[i + 1], s)
        midge_amd.sync()
        return [1e3 * ev.elapsed_ms(evs[i], evs[i + 1]) / group for i in range(n // group)]

    def nbytes_of(r: int) -> int:
        return r * cols // 2 + r * cols // 32 * 2 + cols * 4 + r * 4

    def sustained(tt, yy, r: int) -> dict:
        """`sustain_s` seconds of back-to-back launches with device samples,
        folded into 50 ms windows of GPU time."""
        group = 10
        n = max(group, int(sustain_s / (nbytes_of(r) / 5.5e12)) // group * group)
        time.sleep(0.3)   # idle first
        with DeviceSampler() as smp:
            time.sleep(0.02)
            t0 = time.perf_counter()
            per = launches(tt, yy, n, group)
            time.sleep(0.02)
        out, acc, w0, gt = [], 0.0, 0, 0.0
        for i, us in enumerate(per):
            acc += us * group
            if acc >= (5e3 if gt < 50e3 else 50e3) or i == len(per) - 1:   # 5 ms windows for the first 50 ms
                gt += acc
                g0 = sum(per[:w0]) * group * 1e-6   # window start, s of GPU time
                g1 = g0 + acc * 1e-6
                sm = [q for q in smp.samples if t0 + g0 <= q[0] < t0 + g1]

                def mean(k):
                    v = [q[k] for q in sm if q[k] is not None]
                    return round(sum(v) / len(v), 1) if v else None

                out.append({"t_ms": round(g0 * 1e3, 1), "GBps": round(nbytes_of(r) * (i + 1 - w0) * group /
                                                                      (acc * 1e-6) / 1e9, 1),
                            "power_W": mean(1), "sclk_MHz": mean(2), "temp2_C": mean(3), "temp3_C": mean(4),
                            "samples": len(sm)})
                acc, w0 = 0.0, i + 1
        return {"launches": n, "bytes_per_launch": nbytes_of(r), "windows": out}

    avg = launches(t, y, reps, reps)[0]
    time.sleep(0.2)
    long = launches(t, y, sustain, 5)
    nbytes = nbytes_of(rows)
    sus = sustained(t, y, rows)
    for d in bufs:
        d.free()
    t2, bufs2, y2 = make(2 * rows)
    ctl = sustained(t2, y2, 2 * rows)
    for d in bufs2 + [x]:
        d.free()
    gbs = nbytes / (avg * 1e-6) / 1e9
    first, last = long[0], long[-1]
    return {"kernel": "gemv (MXFP4)", "shape": [rows, cols], "bytes": nbytes, "launches": reps, "avg_us": avg,
            "GBps": gbs, "frac_of_peak": gbs / HBM_PEAK_GBS,
            "sustained": {"launches": sustain, "first5_us": first, "last5_us": last,
                          "first5_frac_of_peak": nbytes / (first * 1e-6) / 1e9 / HBM_PEAK_GBS,
                          "last5_frac_of_peak": nbytes / (last * 1e-6) / 1e9 / HBM_PEAK_GBS},
            "sustained_1s": sus, "control_2x": ctl}


def lm_head_sample_probe(ev, s, reps: int = 20) -> dict:
    """The token after the last layer on the device (the next component of
    the decode path): final rmsnorm, the int8 lm_head GEMV (201088 x 2880)
    and sample() over the 201088 logits, greedy and temperature 1 / top-p
    0.9, HIP-event timed per token over `reps` back-to-back tokens."""
    import midge_amd
    from midge_amd import DT_Q8R, DevBuf, _lib, synth
    from midge_amd.kern import WT, matvec_dev, rmsnorm_dev
    from midge_amd.moe import sample_dev
    V, H = 201088, 2880
    w, sc = DevBuf(V * H), DevBuf(V * 4)
    _lib.call("mh_synth_i8_dev", w.ptr, V * H, 911)
    _lib.call("mh_synth_uniform_dev", sc.ptr, V, 912, 1e-3, float(synth.uniform_c(1e-3, 1e-2)))
    nw, x, xb, lg, out = DevBuf(H * 4), DevBuf(H * 4), DevBuf(H * 4), DevBuf(V * 4), DevBuf(4)
    _lib.call("mh_synth_uniform_dev", nw.ptr, H, 913, 0.5, float(synth.uniform_c(0.5, 1.5)))
    _lib.call("mh_synth_normal_dev", x.ptr, H, 914, float(synth.normal_c(1.0)))
    t = WT(DT_Q8R, V, H, w.ptr, sc.ptr)
    res = {"workload": "final rmsnorm + int8 lm_head 201088x2880 + sample(), one token", "vocab": V}
    for name, temp, topp in (("greedy", 0.0, 1.0), ("temp1_topp0.9", 1.0, 0.9)):
        def token(i):
            rmsnorm_dev(x, nw, xb, H, 1e-5)
            matvec_dev(t, xb, lg)
            sample_dev(lg, V, temp, topp, (i * 0.618034) % 1.0, out)
        for i in range(3):
            token(i)
        midge_amd.sync()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for i in range(reps):
            token(i)
        ev.record(b, s)
        res[name + "_us"] = 1e3 * ev.elapsed_ms(a, b) / reps
    # sample() alone at temperature 1 / top-p 0.9 on normal logits of other
    # spreads: the nucleus from a few tokens (20) to most of the vocabulary
    # (0.2), which decides the selection's way (fast list, sorted
    # candidates, radix select)
    alone = {}
    for sd in (20.0, 6.0, 3.0, 0.2):
        _lib.call("mh_synth_normal_dev", lg.ptr, V, 915, float(synth.normal_c(sd)))
        sample_dev(lg, V, 1.0, 0.9, 0.5, out)
        midge_amd.sync()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for i in range(10):
            sample_dev(lg, V, 1.0, 0.9, (i * 0.618034) % 1.0, out)
        ev.record(b, s)
        alone[f"sd{sd:g}_us"] = 1e3 * ev.elapsed_ms(a, b) / 10
    res["sample_alone_temp1_topp0.9"] = alone
    midge_amd.sync()
    for d in (w, sc, nw, x, xb, lg, out):
        d.free()
    return res


def attention_probe(ev, s, fill: int = 1024, reps: int = 20) -> dict:
    """The trunk's attention for one decode token at the gpt-oss-120b shape
    (hidden 2880, 64 query / 8 key-value heads of 64, int8 projections,
    sinks): a full-attention layer with `fill` cached positions and a
    sliding layer (window 128), HIP-event timed per token over `reps`
    back-to-back positions. Synthetic weights and RoPE tables."""
    import ctypes as C

    import midge_amd
    from midge_amd import DT_Q8R, DevBuf, _lib, synth
    H, nh, nkv, hd, ctx = 2880, 64, 8, 64, fill + reps + 8
    qd, kvd = nh * hd, nkv * hd
    keep = []

    def buf(n, kind, key, a=0.0, b=1.0):
        d = DevBuf(n * 4 if kind != "i8" else n)
        if kind == "i8":
            _lib.call("mh_synth_i8_dev", d.ptr, n, key)
        elif kind == "u":
            _lib.call("mh_synth_uniform_dev", d.ptr, n, key, a, float(synth.uniform_c(a, b)))
        else:
            _lib.call("mh_synth_normal_dev", d.ptr, n, key, float(synth.normal_c(b)))
        keep.append(d)
        return d.ptr

    def wt(rows, cols, key):
        return _lib.MhWT(DT_Q8R, rows, cols, buf(rows * cols, "i8", key), buf(rows, "u", key + 1, 5e-4, 2.5e-3))

    res = {"workload": "attention(), one decode token, gpt-oss-120b shape (2880, 64/8 heads x 64, int8 q/k/v/o)"}
    for name, window in (("full", 0), ("sliding128", 128)):
        L = _lib.MhAttnLayer()
        L.hidden, L.n_heads, L.n_kv_heads, L.head_dim, L.ctx, L.window = H, nh, nkv, hd, ctx, window
        L.qk_norm, L.sinks, L.norm_eps, L.attn_scale = 0, 1, 1e-5, 0.125
        L.wq, L.wk, L.wv, L.wo = wt(qd, H, 920), wt(kvd, H, 922), wt(kvd, H, 924), wt(H, qd, 926)
        L.bq, L.bk, L.bv, L.bo = buf(qd, "n", 930, b=0.1), buf(kvd, "n", 931, b=0.1), buf(kvd, "n", 932, b=0.1), \
            buf(H, "n", 933, b=0.1)
        L.attn_norm = buf(H, "u", 934, 0.5, 1.5)
        L.sink = buf(nh, "n", 935)
        L.rope_cos, L.rope_sin = buf(ctx * hd // 2, "u", 936, -1.0, 1.0), buf(ctx * hd // 2, "u", 937, -1.0, 1.0)
        cap = window if 0 < window < ctx else ctx
        kc, vc = DevBuf(cap * kvd * 2), DevBuf(cap * kvd * 2)
        keep += [kc, vc]
        L.kc, L.vc = kc.ptr, vc.ptr
        xs = DevBuf((fill + reps) * H * 4)
        keep.append(xs)
        _lib.call("mh_synth_normal_dev", xs.ptr, (fill + reps) * H, 938, float(synth.normal_c(1.0)))
        for pos in range(fill):   # fill the cache
            _lib.call("mh_attention_dev", C.byref(L), xs.ptr + pos * H * 4, pos)
        midge_amd.sync()
        a, b = ev.event(), ev.event()
        t0 = time.perf_counter()
        ev.record(a, s)
        for i in range(reps):
            _lib.call("mh_attention_dev", C.byref(L), xs.ptr + (fill + i) * H * 4, fill + i)
        ev.record(b, s)
        host = (time.perf_counter() - t0) / reps * 1e6
        res[name + "_us"] = 1e3 * ev.elapsed_ms(a, b) / reps
        res[name + "_host_enqueue_us"] = host
        res[name + "_cached"] = min(fill + reps, cap)
    midge_amd.sync()
    for d in keep:
        d.free()
    return res


def full_token_probe(ev, s, st, shape, fill: int = 256, reps: int = 10) -> dict:
    """A whole decode token on the device at the gpt-oss-120b shape
    (mh_forward_dev, forward() of engine/midge.c:552-565): the embedding row,
    36 x (attention, then the MoE layer as its one-launch kernel), the final
    rmsnorm, the int8 lm_head (201088 x 2880) and the greedy pick. Layers
    alternate sliding (window 128) and full attention, each with its own
    synthetic int8 q/k/v/o and f16 cache; the MoE layers are the bench's
    resident expert stack. The caches are filled by running `fill` tokens
    first; then `reps` tokens are HIP-event timed back to back."""
    import ctypes as C

    import midge_amd
    from midge_amd import DT_Q8R, DevBuf, _lib, synth
    H, V, nh, nkv, hd, NL = 2880, 201088, 64, 8, 64, shape.n_layers
    ctx = fill + reps + 8
    qd, kvd = nh * hd, nkv * hd
    keep = []

    def buf(n, kind, key, a=0.0, b=1.0):
        d = DevBuf(n * 4 if kind != "i8" else n)
        if kind == "i8":
            _lib.call("mh_synth_i8_dev", d.ptr, n, key)
        elif kind == "u":
            _lib.call("mh_synth_uniform_dev", d.ptr, n, key, a, float(synth.uniform_c(a, b)))
        else:
            _lib.call("mh_synth_normal_dev", d.ptr, n, key, float(synth.normal_c(b)))
        keep.append(d)
        return d.ptr

    def wt(rows, cols, key, lo=1e-4, hi=4e-4):
        return _lib.MhWT(DT_Q8R, rows, cols, buf(rows * cols, "i8", key), buf(rows, "u", key + 1, lo, hi))

    co, si = buf(ctx * hd // 2, "u", 1936, -1.0, 1.0), buf(ctx * hd // 2, "u", 1937, -1.0, 1.0)
    layers = []
    for l in range(NL):
        k0 = 2000 + 40 * l
        L = _lib.MhAttnLayer()
        window = 128 if l % 2 == 0 else 0
        L.hidden, L.n_heads, L.n_kv_heads, L.head_dim, L.ctx, L.window = H, nh, nkv, hd, ctx, window
        L.qk_norm, L.sinks, L.norm_eps, L.attn_scale = 0, 1, 1e-5, 0.125
        L.wq, L.wk, L.wv, L.wo = wt(qd, H, k0), wt(kvd, H, k0 + 2), wt(kvd, H, k0 + 4), wt(H, qd, k0 + 6)
        L.bq, L.bk, L.bv, L.bo = (buf(qd, "n", k0 + 8, b=0.02), buf(kvd, "n", k0 + 9, b=0.02),
                                  buf(kvd, "n", k0 + 10, b=0.02), buf(H, "n", k0 + 11, b=0.02))
        L.attn_norm = buf(H, "u", k0 + 12, 0.5, 1.5)
        L.sink = buf(nh, "n", k0 + 13)
        L.rope_cos, L.rope_sin = co, si
        cap = window if 0 < window < ctx else ctx
        kc, vc = DevBuf(cap * kvd * 2), DevBuf(cap * kvd * 2)
        keep += [kc, vc]
        L.kc, L.vc = kc.ptr, vc.ptr
        layers.append(L)
    attn = (_lib.MhAttnLayer * NL)(*layers)
    d = _lib.MhModelDesc()
    d.hidden, d.vocab, d.n_layers, d.norm_eps = H, V, NL, 1e-5
    d.embed = wt(V, H, 1900, 2e-3, 8e-3)
    d.lm_head = wt(V, H, 1902, 1e-3, 1e-2)
    d.final_norm = buf(H, "u", 1904, 0.5, 1.5)
    d.attn, d.moe = attn, st._cl
    model = C.c_void_p()
    _lib.call("mh_model_create", C.byref(d), C.byref(model))
    x, lg, tok = DevBuf(H * 4), DevBuf(V * 4), DevBuf(4)
    keep += [x, lg, tok]
    toks = np.random.default_rng(77).integers(0, V, fill + reps)

    def token(i):
        _lib.call("mh_forward_dev", model, int(toks[i]), i, x.ptr, lg.ptr, None, None)
        _lib.call("mh_sample_dev", lg.ptr, V, 0.0, 1.0, 0.0, tok.ptr)

    for i in range(fill):
        token(i)
    midge_amd.sync()
    a, b = ev.event(), ev.event()
    t0 = time.perf_counter()
    ev.record(a, s)
    for i in range(fill, fill + reps):
        token(i)
    ev.record(b, s)
    host = (time.perf_counter() - t0) / reps * 1e3
    ms = ev.elapsed_ms(a, b) / reps
    midge_amd.sync()
    _lib.call("mh_model_destroy", model)
    for dd in keep:
        dd.free()
    log(f"full decode token (36 x attention + MoE, lm_head, greedy): {ms:.3f} ms")
    return {"workload": "one decode token on the device, gpt-oss-120b shape: embedding, 36 x (attention "
                        "(alternately sliding 128 / full) + MoE (128 MXFP4 experts, top-4)), final norm, int8 "
                        "lm_head 201088x2880, greedy pick",
            "ms_per_token": ms, "tok_per_s": 1e3 / ms, "host_enqueue_ms": host, "cached_positions": fill + reps}


def reference_bench(ev, s, seconds: float = 1.0) -> dict:
    """The reference's own kernel figure, run_bench (engine/midge.c:687-720):
    a q4g32 2880x2880 matvec over fixed synthetic data (byte i = (i *
    2654435761) >> 24, every scale 0x2c00, x = 0.5), looped for >= 1 s,
    reported as GiB/s of data + scales. Three numbers:
      cpu          the reference engine compiled from its sources
                   (oracle/_ref/midged --bench), AVX2 + OpenMP on the host
      drop_in_gpu  the same engine source with this library's drop-in
                   header (oracle/_ref/midged_hip --bench): the reference's
                   own loop, x and y crossing PCIe on every call
      device       this library's GEMV on the same data with x and y
                   resident in HBM, timed with HIP events over the loop.
    The 4.7 MB matrix stays cache-resident on both sides."""
    import re
    import subprocess
    import midge_amd
    from midge_amd import DT_Q4G32, DevBuf
    from midge_amd.kern import WT, matvec_dev
    out = {"workload": "run_bench: q4g32 2880x2880, data + scales GiB/s (engine/midge.c:687-720)"}
    for key, exe in (("cpu", "midged"), ("drop_in_gpu", "midged_hip")):
        path = os.path.join(ROOT, "oracle", "_ref", exe)
        if not os.path.exists(path):
            out[key] = None
            continue
        r = subprocess.run([path, "--bench"], capture_output=True, text=True, timeout=120)
        m = re.search(r"BENCH q4g32_gbps=([0-9.]+) threads=(\d+)", r.stdout)
        out[key] = {"GiBps": float(m.group(1)), "threads": int(m.group(2)), "line": m.group(0)} if m else {
            "error": (r.stdout + r.stderr)[-300:]}
    rows = cols = 2880
    db, sb = rows * cols // 2, rows * (cols // 32) * 2
    data = ((np.arange(db, dtype=np.uint64) * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)) >> np.uint64(24)
    dd = DevBuf.from_array(data.astype(np.uint8))
    sd = DevBuf.from_array(np.full(sb // 2, 0x2C00, np.uint16))
    xd = DevBuf.from_array(np.full(cols, 0.5, np.float32))
    yd = DevBuf(rows * 4)
    t = WT(DT_Q4G32, rows, cols, dd.ptr, sd.ptr)
    for _ in range(3):
        matvec_dev(t, xd, yd)
    midge_amd.sync()
    a, b = ev.event(), ev.event()
    iters, el = 0, 0.0
    while el < seconds:
        ev.record(a, s)
        for _ in range(200):
            matvec_dev(t, xd, yd)
        ev.record(b, s)
        el += ev.elapsed_ms(a, b) * 1e-3
        iters += 200
    out["device"] = {"GiBps": iters * (db + sb) / el / 2**30, "iters": iters, "seconds": el,
                     "us_per_call": el / iters * 1e6}
    for d in (dd, sd, xd, yd):
        d.free()
    return out


def engine_host_probe(n_gen: int = 384) -> dict:
    """The reference engine's own host (its protocol, forward, forward_batch,
    sample; engine/midge.c:552-622, 654-679, 790-831), built from its sources
    three ways, decoding on a 4-layer model at gpt-oss's layer shapes (32
    MXFP4 experts 2880x2880, int8 attention and router, vocab 8192) written
    to a temporary directory by the tests' model writer:
      cpu          oracle/_ref/midged: the engine on its CPU kernels
      kernel_level oracle/_ref/midged_hip: every wk_matvec / wk_row through
                   the drop-in header (host activations, a GEMV round trip
                   per projection)
      layer_level  oracle/_ref/midged_hip_layer: the containers resident in
                   HBM, forward() one mh_forward_dev call per token (device
                   attention, the one-launch MoE kernel per layer, lm_head),
                   sample() on the device logits
    Greedy decode tok/s from the engine's own DONE line (its timer around the
    gen loop), after a 16-token prefill; the layer level also at temperature
    0.8 / top-p 0.9 (set: ... seed 5)."""
    import shutil
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import engine_model as em
    out = {"workload": "4-layer gpt-oss-shaped model (32 MXFP4 experts, int8 attention/router, vocab 8192), "
                       f"16-token prefill then {n_gen} generated tokens; tok/s from the engine's DONE line"}
    d = tempfile.mkdtemp(prefix="midge_engine_")
    try:
        sp = em.write_model(d, n_layers=4)
        ids = " ".join(map(str, em.prompt(16, sp["vocab"], seed=9)))
        greedy = f"ids: {ids}\ngen: {n_gen}\nquit\n"
        sampled = f"set: 0.8 0.9 5\nids: {ids}\ngen: {n_gen}\nquit\n"
        runs = [("cpu", "midged", greedy), ("kernel_level", "midged_hip", greedy),
                ("layer_level", "midged_hip_layer", greedy), ("layer_level_sampled", "midged_hip_layer", sampled),
                ("cpu_sampled", "midged", sampled)]
        toks = {}
        for key, exe, script in runs:
            path = os.path.join(ROOT, "oracle", "_ref", exe)
            if not os.path.exists(path):
                out[key] = None
                continue
            log(f"engine host: {key}")
            _, t, done, _ = em.run_engine(path, d, script, ctx=512, timeout=300)
            gen = [x for x in done if x[1] > 0]
            toks[key] = t
            out[key] = {"tok_per_s": gen[-1][1] / gen[-1][2], "generated": int(gen[-1][1]),
                        "seconds": gen[-1][2]} if gen else {"error": "no DONE line"}
        if "cpu" in toks and "layer_level" in toks:
            out["greedy_tokens_equal"] = toks["cpu"] == toks["layer_level"] == toks.get("kernel_level", toks["cpu"])
        if "cpu_sampled" in toks and "layer_level_sampled" in toks:
            # the logits differ from the CPU engine's in the last bits, so a
            # draw that lands that close to a cumulative boundary picks the
            # neighbour and the sequences part from there: the common prefix
            a, b = toks["cpu_sampled"], toks["layer_level_sampled"]
            same = next((i for i, (p, q) in enumerate(zip(a, b)) if p != q), min(len(a), len(b)))
            out["sampled_tokens_common_prefix"] = same
        if out.get("cpu") and out.get("layer_level"):
            out["layer_level_vs_cpu"] = out["layer_level"]["tok_per_s"] / out["cpu"]["tok_per_s"]
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return out


def config_probes(ev, s, seed: int, reps: int = 40) -> dict:
    """Configurations 0-2 of the measurement plan beside the headline (cfg 4)
    and the prefill (cfg 3), each with synthetic device-generated inputs and
    weights that rotate over more than the 256 MB memory-side cache, so that
    every call streams its weights from HBM (the same figures for one set of
    weights, cache-resident, are given beside them):
      cfg0  one gpt-oss expert FFN for one token: expert_apply with the
            routing given (mh_stack_apply_dev: one launch, no router, as the
            reference's own configuration times the expert alone), call i on
            expert i mod 40 of a 40-expert table (561 MB); the same through a
            routed one-layer step (top-1 router) beside it
      cfg1  one gpt-oss-20b MoE layer (32 experts, top-4), batch 1, a fresh
            hidden state per call, rotating over 4 such layers (1.8 GB)
      cfg2  the int8 (q8r) trunk GEMVs QKV 5120x2880 and O 2880x4096 over 24
            copies of the weights (354 / 283 MB), lm_head 201088x2880 (579 MB,
            one copy), at batch 1 (the GEMV engine) and 32 (one pass over the
            weights on the int8 matrix cores)."""
    import midge_amd
    from midge_amd import DT_Q8R, DevBuf, _lib, synth
    from midge_amd.kern import WT, matvec_dev
    from midge_amd.moe import Stack
    from midge_amd.synth import MoEShape
    out = {}

    def timed(call, n) -> float:
        for i in range(3):
            call(i)
        midge_amd.sync()
        a, b = ev.event(), ev.event()
        ev.record(a, s)
        for i in range(n):
            call(3 + i)
        ev.record(b, s)
        return ev.elapsed_ms(a, b) / n

    def xs_of(keys, H, n):
        xs = DevBuf(n * H * 4)
        _lib.call("mh_synth_normal_dev", xs.ptr, n * H, synth.hash64_int(keys.x, 5), float(synth.normal_c(1.0)))
        return xs

    # cfg0: one expert FFN, one token
    E0 = 40
    shp = MoEShape(hidden=2880, ffn=2880, n_experts=E0, top_k=1, n_layers=1)
    st, bufs, keys = Stack.synthetic(shp, seed, 1)
    H = shp.hidden
    xs = xs_of(keys, H, reps + 3)
    xo = DevBuf(H * 4)
    _lib.call("mh_synth_normal_dev", xo.ptr, H, 907, float(synth.normal_c(1.0)))
    sels = DevBuf.from_array(np.arange(E0, dtype=np.int32))
    wd = DevBuf.from_array(np.ones(1, np.float32))
    rot = timed(lambda i: st.apply(0, xs.ptr + i * H * 4, sels.ptr + 4 * (i % E0), wd.ptr, xo.ptr), reps)
    one = timed(lambda i: st.apply(0, xs.ptr + i * H * 4, sels.ptr, wd.ptr, xo.ptr), reps)
    routed = timed(lambda i: st.decode(xs.ptr + i * H * 4, 1), reps)
    nbytes = shp.layout.expert_stride + 2 * H * 4   # the expert's three matrices, xb in, x out
    out["cfg0"] = {"workload": "one expert FFN (2880x2880 MXFP4 gate/up/down), one token; call i on expert i mod 40",
                   "path": "expert_apply, routing given (mh_stack_apply_dev, one launch)",
                   "us_per_token": rot * 1e3, "tok_per_s": 1e3 / rot, "hbm_bytes": nbytes,
                   "GBps": nbytes / (rot * 1e-3) / 1e9, "frac_of_peak": nbytes / (rot * 1e-3) / 1e9 / HBM_PEAK_GBS,
                   "cache_resident_us": one * 1e3, "routed_one_layer_us": routed * 1e3}
    for d in (xs, xo, sels, wd):
        d.free()
    st.destroy()
    for d in bufs:
        d.free()
    # cfg1: one gpt-oss-20b MoE layer at batch 1, rotating over 4 layers' tables
    shp = MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4, n_layers=1)
    stacks = [Stack.synthetic(shp, seed + 10 * j, 1) for j in range(4)]
    xs = xs_of(stacks[0][2], H, reps + 3)
    rot = timed(lambda i: stacks[i % 4][0].decode(xs.ptr + i * H * 4, 1), reps)
    one = timed(lambda i: stacks[0][0].decode(xs.ptr + i * H * 4, 1), reps)
    nbytes = step_bytes(shp, 1, float(shp.top_k))
    out["cfg1"] = {"workload": "one gpt-oss-20b MoE layer, 32 MXFP4 experts, top-4, batch 1; call i on layer i mod 4",
                   "us_per_token": rot * 1e3, "tok_per_s": 1e3 / rot, "hbm_bytes": nbytes,
                   "GBps": nbytes / (rot * 1e-3) / 1e9, "frac_of_peak": nbytes / (rot * 1e-3) / 1e9 / HBM_PEAK_GBS,
                   "cache_resident_us": one * 1e3}
    xs.free()
    for st_, bufs_, _ in stacks:
        st_.destroy()
        for d in bufs_:
            d.free()
    # cfg2: the int8 trunk GEMVs
    gemvs = []
    for gname, R, Cc, ncopy in (("qkv", 5120, 2880, 24), ("o", 2880, 4096, 24), ("lm_head", 201088, 2880, 1)):
        ws = []
        for j in range(ncopy):
            w, sc = DevBuf(R * Cc), DevBuf(R * 4)
            _lib.call("mh_synth_i8_dev", w.ptr, R * Cc, 901 + 17 * j)
            _lib.call("mh_synth_uniform_dev", sc.ptr, R, 902 + 17 * j, 1e-3, float(synth.uniform_c(1e-3, 1e-2)))
            ws.append((w, sc, WT(DT_Q8R, R, Cc, w.ptr, sc.ptr)))
        for B in (1, 32):
            x, y = DevBuf(B * Cc * 4), DevBuf(B * R * 4)
            _lib.call("mh_synth_normal_dev", x.ptr, B * Cc, 903, float(synth.normal_c(1.0)))
            ms = timed(lambda i: matvec_dev(ws[i % ncopy][2], x, y, B), reps)
            nbytes = R * Cc + 4 * R + 4 * Cc * B + 4 * R * B
            rec = {"gemv": gname, "shape": [R, Cc], "batch": B, "weight_copies": ncopy, "us": ms * 1e3,
                   "path": "int8 matrix cores, x as 3 int8 digits" if B > 1 else "GEMV",
                   "GBps": nbytes / (ms * 1e-3) / 1e9, "frac_of_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                   "GFLOPs": 2.0 * R * Cc * B / (ms * 1e-3) / 1e9}
            if ncopy > 1:
                rec["cache_resident_us"] = timed(lambda i: matvec_dev(ws[0][2], x, y, B), reps) * 1e3
            gemvs.append(rec)
            x.free()
            y.free()
        for w, sc, _ in ws:
            w.free()
            sc.free()
    out["cfg2"] = {"workload": "int8 (q8r) trunk GEMVs, batch 1 and 32, weights rotating over more than 256 MB",
                   "gemvs": gemvs}
    return out


MFMA_FP6_PEAK_TFLOPS = 10100.0  # dense fp6 / fp4 MFMA (the rate of fp4 x fp6 operands, the prefill GEMM's)


def prefill_probe(ev, s, seed: int, n: int = 512, reps: int = 10) -> dict:
    """Expert-major prefill of one gpt-oss-20b MoE layer (32 MXFP4 experts
    2880x2880, top-4) for 512 tokens routed by N(0,1) logits: the grouped
    scaled-MFMA GEMM path and, for comparison, the per-assignment GEMV path.
    Timed with HIP events over `reps` calls of mh_expert_major_dev."""
    import midge_amd
    from midge_amd import DevBuf, _lib, set_switch, synth
    from midge_amd.device import profile_enable, profile_query, profile_reset
    from midge_amd.moe import Stack, expert_major_dev, topk_dev
    from midge_amd.synth import MoEShape
    shape = MoEShape(hidden=2880, ffn=2880, n_experts=32, top_k=4, n_layers=1)
    st, bufs, keys = Stack.synthetic(shape, seed + 3, 1)
    lay = st.layers[0]
    H, E, k = shape.hidden, shape.n_experts, shape.top_k
    logits, xb, x = DevBuf(n * E * 4), DevBuf(n * H * 4), DevBuf(n * H * 4)
    _lib.call("mh_synth_normal_dev", logits.ptr, n * E, synth.hash64_int(keys.x, 77), float(synth.normal_c(1.0)))
    _lib.call("mh_synth_normal_dev", xb.ptr, n * H, synth.hash64_int(keys.x, 78), float(synth.normal_c(1.0)))
    _lib.call("mh_synth_normal_dev", x.ptr, n * H, synth.hash64_int(keys.x, 79), float(synth.normal_c(1.0)))
    sel, w = DevBuf(n * k * 4), DevBuf(n * k * 4)
    topk_dev(logits, n, E, k, 1, sel, w)
    counts = np.bincount(sel.download(np.int32, (n, k)).ravel(), minlength=E)
    out = {"workload": f"one gpt-oss-20b MoE layer, {n} tokens, {E} MXFP4 experts 2880x2880, top-{k}",
           "tokens_per_expert": {"min": int(counts.min()), "max": int(counts.max()), "mean": float(counts.mean())}}
    weights = E * shape.layout.expert_stride
    useful_flops = 2.0 * n * k * 3 * shape.hidden * shape.ffn
    for path in ("mfma", "gemv"):
        if path == "gemv":
            set_switch("NO_MFMA", True)
        try:
            r = reps if path == "mfma" else 2
            expert_major_dev(lay, n, xb, sel, w, x)
            midge_amd.sync()
            a, b = ev.event(), ev.event()
            ev.record(a, s)
            for _ in range(r):
                expert_major_dev(lay, n, xb, sel, w, x)
            ev.record(b, s)
            ms = ev.elapsed_ms(a, b) / r
            res = {"ms": ms, "tok_per_s": n / (ms * 1e-3), "weight_GBps": weights / (ms * 1e-3) / 1e9}
            if path == "mfma":
                profile_reset()
                profile_enable(True)
                expert_major_dev(lay, n, xb, sel, w, x)
                midge_amd.sync()
                kern = {}
                for name in ("plist", "quant_x", "moe_gu_mfma", "quant_h", "moe_down_mfma", "combine_prefill"):
                    tot, cnt = profile_query(name)
                    if cnt:
                        kern[name] = {"us": 1e3 * tot, "launches": cnt}
                profile_enable(False)
                gemm_us = sum(kern[n_]["us"] for n_ in ("moe_gu_mfma", "moe_down_mfma") if n_ in kern)
                tiles = int(sum(-(-int(c) // 32) for c in counts))          # 32-token tiles over experts
                issued = 2.0 * tiles * 32 * 3 * shape.hidden * shape.ffn * 3   # 3 matrices x 3 activation terms
                res.update({"kernels": kern, "useful_TFLOPs": useful_flops / (ms * 1e-3) / 1e12,
                            "gemm_issued_TFLOPs": issued / (gemm_us * 1e-6) / 1e12 if gemm_us else None,
                            "mfma_util_of_fp6_peak": issued / (gemm_us * 1e-6) / 1e12 / MFMA_FP6_PEAK_TFLOPS
                            if gemm_us else None})
            out[path] = res
        finally:
            set_switch("NO_MFMA", False)
    out["speedup_mfma_vs_gemv"] = out["gemv"]["ms"] / out["mfma"]["ms"]
    for d in (logits, xb, x, sel, w):
        d.free()
    st.destroy()
    for d in bufs:
        d.free()
    log(f"prefill cfg3: mfma {out['mfma']['ms']:.3f} ms, gemv {out['gemv']['ms']:.3f} ms")
    return out


def run_cpu(shape, seed: int, seconds: float, threads: int) -> dict:
    """The reference engine's moe() (AVX2+OpenMP, built from its sources) over
    one resident gpt-oss-120b layer (128 experts, 1.8 GB host RAM), in this
    process (a child of the bench: its OpenMP team is set up from the
    environment the parent gives it)."""
    from midge_amd import synth
    from oracle import pyoracle as po

    kind = "reference" if po.have_ref() else "port"
    keys = synth.Keys(seed)
    L = shape.layout
    table = np.empty(L.layer_stride, np.uint8)
    lib = po.oracle()

    def gen(e: int) -> int:   # ctypes releases the GIL: experts generate in parallel
        sl = table[e * L.expert_stride:(e + 1) * L.expert_stride]
        return lib.mo_synth_expert(sl.ctypes.data, shape.expert_dt, shape.hidden, shape.ffn, shape.n_experts, 0, e,
                                   keys.table, synth.EXPERT_EMIN, synth.EXPERT_EMAX,
                                   float(synth.normal_c(synth.EXPERT_BIAS_STD)))

    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as pool:
        assert all(rc == 0 for rc in pool.map(gen, range(shape.n_experts)))
    w, s, b, nw = synth.host_router(shape, keys, 0)
    Ls = po.layer_struct(shape, table, w, s, b, nw)
    xs = synth.host_x(shape, keys, 64, step=11)
    run = (lambda x: po.ref_moe_decode(Ls, x)) if kind == "reference" else (lambda x: po.moe_decode(Ls, x))
    for i in range(3):
        run(xs[i])
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        run(xs[n % 64])
        n += 1
    dt = time.perf_counter() - t0
    layer_b = step_bytes(shape, 1, shape.top_k) / shape.n_layers   # the bytes one moe() call reads
    return {"value": n / dt / shape.n_layers, "unit": "tok/s", "cores": threads if kind == "reference" else 1,
            "kind": kind, "GBps": n / dt * layer_b / 1e9,
            "sample": f"{n} moe() calls on one resident 128-expert gpt-oss-120b layer (batch 1, {dt:.1f}s), "
                      f"tok/s = calls/s / 36 layers"}


def physical_cores() -> int | None:
    """Physical cores of the host (distinct (core, socket) pairs of lscpu)."""
    import subprocess
    try:
        r = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=20)
    except (OSError, subprocess.SubprocessError):
        return None
    pairs = {ln.strip() for ln in r.stdout.splitlines() if ln.strip() and not ln.startswith("#")}
    return len(pairs) or None


def cpu_baseline(shape, seed: int, seconds: float) -> dict:
    """The CPU baseline in two child processes: one OpenMP thread (beside the
    reference's published per-core figure, 3.98 GB/s on AVX2, README.md:84-86)
    and the threads this process may use (its affinity mask, at most
    OMP_NUM_THREADS), each pinned to its own physical core (OMP_PROC_BIND=close,
    OMP_PLACES=cores)."""
    import subprocess
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    team = max(1, min(avail, int(os.environ.get("OMP_NUM_THREADS", avail))))
    rows = {}
    for threads, secs in ((1, seconds / 2), (team, seconds)):
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PROC_BIND="close", OMP_PLACES="cores")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", str(threads),
                            "--cpu-seconds", str(secs), "--seed", str(seed)],
                           env=env, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            raise RuntimeError(f"cpu baseline child ({threads} threads) failed: {r.stderr[-500:]}")
        rows[threads] = json.loads(r.stdout.strip().splitlines()[-1])
    out = dict(rows[team])
    one = rows[1]
    out.update({"physical_cores": physical_cores(), "affinity_cpus": avail,
                "binding": "OMP_PROC_BIND=close OMP_PLACES=cores",
                "one_thread": {"value": one["value"], "unit": "tok/s", "GBps": one["GBps"],
                               "published_GBps_per_core": 3.98, "sample": one["sample"]}})
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--experts", type=int, default=128)
    ap.add_argument("--seed", type=int, default=120)
    ap.add_argument("--prof-steps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b16", action="store_true", help="skip the extra batch-16 measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the expert-major prefill measurement")
    ap.add_argument("--no-refbench", action="store_true", help="skip the reference's run_bench figure")
    ap.add_argument("--no-configs", action="store_true", help="skip the configuration 0-2 measurements")
    ap.add_argument("--no-engine", action="store_true", help="skip the reference engine's host on the library")
    ap.add_argument("--cpu-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device twice (byte-counter calibration)")
    args = ap.parse_args()
    from midge_amd.synth import MoEShape
    if args.cpu_child:   # the CPU baseline's child process: no GPU
        shape = MoEShape(hidden=2880, ffn=2880, n_experts=args.experts, top_k=4, n_layers=args.layers)
        print(json.dumps(run_cpu(shape, args.seed, args.cpu_seconds, args.cpu_child)), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the expert stack "
              "fits one MI355X); run with --gpus 1", file=sys.stderr)
        return 2

    shape = MoEShape(hidden=2880, ffn=2880, n_experts=args.experts, top_k=4, n_layers=args.layers)
    ms, unique, kern, dom, extra = run_gpu(args, shape)
    ms_step = ms / args.steps
    value = args.batch * args.steps / (ms / 1e3)
    step_b = step_bytes(shape, args.batch, unique)
    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(shape, args.seed, args.cpu_seconds)
    out = {
        "metric": METRIC, "value": value, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"gpt-oss-120b expert-stack decode: {shape.n_layers} layers x {shape.n_experts} "
                               f"MXFP4 experts (2880x2880 gate/up/down), int8 routers, top-4, "
                               f"batch {args.batch}; attention/trunk excluded",
                   "layers": shape.n_layers, "experts": shape.n_experts, "top_k": 4, "hidden": 2880,
                   "ffn": 2880, "batch": args.batch, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["GBps"] / HBM_PEAK_GBS, "traffic": dom.get("traffic"),
                     "kernel": dom["name"], "bytes_per_launch": dom["bytes"], "avg_us": dom["avg_us"],
                     **({"traffic_source": dom["traffic_source"]} if "traffic_source" in dom else {}),
                     **({"profiled_avg_us": dom["profiled_avg_us"]} if "profiled_avg_us" in dom else {})},
        "step": {"hbm_bytes": step_b, "hbm_GBps": step_b / (ms_step / 1e3) / 1e9,
                 "hbm_frac": step_b / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS,
                 "unique_experts_per_layer": unique, "kernels": kern},
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)
    import midge_amd
    midge_amd.shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
