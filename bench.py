#!/usr/bin/env python3
"""Benchmark of the routed-MoE layer on one MI355X.

Default workload: BASELINE config 1 at the 17-token speculative-verify batch
(Q4_K gate/up, IQ4_NL down, shared Q4_K expert with sigmoid gate, correlated
RMS-normed inputs).  A step is one layer forward (router -> top-10 -> experts
-> router-rank combine -> shared expert) through the C ABI's qg_moe_forward,
rotating over 16 distinct seeded layers (14.5 GB) so expert weights stream
from HBM, not from the 256 MB Infinity Cache.  Inputs are resident in HBM
before the timed region.

--config 0: one token, Q4_K experts, no shared expert.
--config 2: the 48-layer stack at one token, h <- h + MoE(RMSNorm(h)) per
            layer, replayed as one captured graph (43.5 GB of experts).
--config 4: config 1 with 128 of 512 experts resident per layer and the 90 %
            coverage flags.
--config 3: the 2048-token prefill (Zipf(1.1)-biased router, Q4_K gate/up,
            IQ4_NL down): value = tokens/s of the layer; roofline = the
            matrix-core utilisation of the grouped gate/up GEMM (one launch
            over every expert) against the int8 peak; the dense experts
            (>= 256 rows) are also timed in a launch of their own, on fp16
            and on int8 matrix cores.
--matmul:   qg_matmul (exact reference order) on the D = 2560 dense
            projections in Q4_K at --batch tokens (default 1): value = weight
            GB/s; cpu_baseline = the reference's qc_matmul.

Printed: one JSON line.  value = tokens/s (batch / step time), the step being
one layer forward inside a captured graph of the whole 16-layer rotation
(replayed back to back); roofline = the gate/up kernel's
algorithmic bytes over its average duration, from HIP events recorded by the
kernel dispatches themselves on the library's launch stream
(hipExtLaunchKernelGGL) over the same number of eagerly launched steps; cpu_baseline = the reference's own
cpu.c (router qc_matmul, qc_moe, shared-expert qc_matmul; built from
/root/reference into oracle/_ref) on the same inputs, on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import gc
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from nebula_amd import qg, synth  # noqa: E402

D, FF, TOP, EXPERTS = 2048, 512, 10, 512
EXPERT_BYTES = 1_769_472
GATEUP_BYTES = 1_179_648          # gate + up rows of one Q4_K expert (2 x 512 x 1152 B)
ROUTER_BYTES = EXPERTS * D * 4
HBM_PEAK_GBS = 8000.0
METRIC = "routed-MoE tokens/s + % HBM peak at B=1/17; int8 MFMA util at 2048-tok prefill"
KERNELS = ["router", "route", "gate_up", "down", "combine"]
PF_KERNELS = ["router", "route", "scan", "fill", "gate_up_dense", "gate_up", "down_dense", "down",
              "down_shared", "combine", "count"]
INT8_PEAK_TOPS = 5000.0           # MI355X dense int8 MFMA (POP/s x 1e3)
FP16_PEAK_TFLOPS = 2500.0         # MI355X dense fp16 MFMA
DENSE_MIN = 256                   # rows from which an expert is dense


def layer_bytes(nt: int, unique: float, shared: bool) -> float:
    """Algorithmic HBM bytes of one layer forward (each touched expert once)."""
    b = ROUTER_BYTES + unique * EXPERT_BYTES + nt * (2 * D * 4 + 80)
    if shared:
        b += EXPERT_BYTES + D * 4
    return b


def gateup_bytes(nt: int, unique: float, shared: bool) -> float:
    return (unique + (1 if shared else 0)) * GATEUP_BYTES + nt * D * 4


def down_bytes(nt: int, unique: float, shared: bool) -> float:
    """The down kernel's algorithmic bytes: each touched expert's down rows
    once, the mid rows read (fp16 hi and lo planes, one row per selection and
    shared-expert token) and the weighted rows written to the selection slots."""
    rows = nt * TOP + (nt if shared else 0)
    return (unique + (1 if shared else 0)) * (EXPERT_BYTES - GATEUP_BYTES) + rows * FF * 4 + rows * D * 4


def resident_set(layer: synth.DeviceLayer, batch_seed: int, noise_seed: int, count: int = 128) -> np.ndarray:
    """Config 4's resident experts: the `count` best-ranked over 4096 seeded
    synthetic tokens from 8 correlated contexts, one of them the verify
    batch's own (synth.ranking_inputs), routed on the device, ranked by the
    reference's rule: activation count, then routed weight, then id
    (synth.resident_ranking, qwen/README.md:38)."""
    xs = synth.ranking_inputs(batch_seed, noise_seed, width=D)
    n = xs.shape[0]
    dx = qg.Device(xs)
    logits = qg.Device(shape=(n, EXPERTS), dtype=np.float32)
    ids = qg.Device(shape=(n, TOP), dtype=np.int32)
    w = qg.Device(shape=(n, TOP), dtype=np.float32)
    qg.call("matmul", logits.p, layer.bufs["router"].p, 0, EXPERTS, D, dx.p, n)
    qg.call("route", ids.p, w.p, logits.p, n)
    return synth.resident_ranking(ids.get(), w.get(), count)


class Workload:
    def __init__(self, config: int, batch: int, layers: int, seed: int):
        self.config, self.nt = config, batch
        self.shared = config in (1, 4)
        dt = 20 if config in (1, 4) else 12
        self.specs = [synth.LayerSpec(seed=seed + l, down_type=dt, shared=self.shared) for l in range(layers)]
        t0 = time.time()
        self.layers = []
        for s in self.specs:
            L = synth.build_layer(s)
            if config == 4:
                mask = resident_set(L, batch_seed=seed + 1000, noise_seed=s.seed + 77)
                L.bufs["resident"] = qg.Device(mask)
                L.desc.resident, L.desc.threshold = L.bufs["resident"].p, 0.10
            self.layers.append(L)
        qg.call("sync")
        self.build_s = time.time() - t0
        self.fw = synth.Forward(D, FF, batch)
        self.x = synth.inputs(seed + 1000, batch, D, correlated=config in (1, 4))
        self.fw.x.set(self.x)

    def step(self, i: int) -> None:
        self.fw.run(self.layers[i % len(self.layers)], self.nt)

    def routing(self, i: int):
        self.step(i)
        qg.call("sync")
        ids = self.fw.ids.get()[:self.nt]
        flags = self.fw.flags.get()[:self.nt]
        return ids, flags

    def unique_experts(self, i: int) -> int:
        ids, flags = self.routing(i)
        ok = (ids >= 0) & (ids < EXPERTS) & (flags[:, None] < 2)
        return len(np.unique(ids[ok]))


def capture_steps(wl, layers) -> C.c_void_p:
    """One captured graph of consecutive layer forwards (rotated layers
    `layers`, in order): a replay runs them back to back with one host call,
    as a serving loop replays a whole captured decode step (qwen.c:726-734
    captures per batch size), so the device time per layer is measured rather
    than the host's graph-launch rate."""
    g = C.c_void_p()
    qg.call("graph_begin", C.byref(g))
    for i in layers:
        wl.step(i)
    qg.call("graph_end", g)
    return g


def time_decode(wl: Workload, steps: int, warmup: int):
    """Step time over exactly `steps` timed layer forwards: steps // n replays
    of one graph of all n rotated layers, then one graph of the first
    steps % n; then the average duration of each kernel of the step from
    dispatch-timestamped events (qg_moe_kernel_events,
    hipExtLaunchKernelGGL) over the same number of eagerly launched steps."""
    n = len(wl.layers)
    full = capture_steps(wl, range(n))
    part = capture_steps(wl, range(steps % n)) if steps % n else None
    for _ in range(max(1, -(-warmup // n))):
        qg.call("graph_launch", full)
    qg.call("sync")
    b, e = qg.Event(), qg.Event()
    b.record()
    for _ in range(steps // n):
        qg.call("graph_launch", full)
    if part is not None:
        qg.call("graph_launch", part)
    e.record()
    qg.call("sync")
    ms = qg.elapsed_ms(b, e) / steps
    for g in (full, part):
        if g is not None:
            qg.lib().qg_graph_destroy(g)
    return ms, kernel_times(wl.step, KERNELS, steps)


def kernel_times(step, names, steps) -> dict:
    """Average duration (ms) of each named kernel of a step over `steps`
    eagerly launched steps, from events the dispatches record themselves
    (qg_moe_kernel_events); kernels that did not run are left out."""
    n = 2 * len(names)
    evs = [[qg.Event() for _ in range(n)] for _ in range(steps)]
    arrs = [(C.c_void_p * n)(*[ev.p for ev in evs_i]) for evs_i in evs]
    for i in range(steps):
        qg.call("moe_kernel_events", arrs[i], n)
        step(i)
    qg.call("moe_kernel_events", None, 0)
    qg.call("sync")
    kern = {}
    for k, name in enumerate(names):
        vals = []
        for ev in evs:
            t = C.c_float()
            if qg.lib().qg_event_elapsed(C.byref(t), ev[2 * k].p, ev[2 * k + 1].p) == 0:
                vals.append(t.value)
        if vals:
            kern[name] = float(np.mean(vals))
    return kern


_HOST_CPUS = None


def host_cpus() -> dict:
    """This process's CPUs: model name, sockets, physical cores and logical
    CPUs among the CPUs it may run on, from /proc and /sys.  Read once, at
    the first call, which main() makes before the OpenMP runtime starts (with
    OMP_PROC_BIND set the runtime binds the calling thread to one place,
    which would shrink sched_getaffinity afterwards)."""
    global _HOST_CPUS
    if _HOST_CPUS is not None:
        return _HOST_CPUS
    cpus = sorted(os.sched_getaffinity(0))
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    cores, sockets = set(), set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            pkg = int((base / "physical_package_id").read_text())
            core = int((base / "core_id").read_text())
        except (OSError, ValueError):
            pkg, core = 0, c
        sockets.add(pkg)
        cores.add((pkg, core))
    _HOST_CPUS = {"model": model, "sockets": len(sockets), "physical_cores": len(cores), "logical_cpus": len(cpus)}
    return _HOST_CPUS


def cpu_threads() -> int:
    """min(28, physical cores available): 28 is cpu.c's own cap (cpu.c:121,150,164)."""
    return max(1, min(28, host_cpus()["physical_cores"]))


def cpu_baseline(wl, budget_s: float, tokens: int | None = None) -> dict | None:
    """The reference's cpu.c on layer 0 of the workload: router qc_matmul (F32),
    qc_moe on the routed experts, shared expert through qc_matmul x 3 plus the
    sigmoid-gated add.  Routing ids/weights come from the GPU run of the same
    inputs (the reference's CPU path receives them from the GPU,
    qwen.c:665-669); routing itself is not timed (a top-10 of 512 per token)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    try:
        import oracle as O
    except Exception:
        return None
    ref = O.ref_lib(D)
    if ref is None:
        return None
    L = wl.layers[0]
    nt = min(wl.nt, tokens or wl.nt)
    ids, _ = wl.routing(0)
    ids = np.ascontiguousarray(ids[:nt])
    w = np.ascontiguousarray(wl.fw.w.get()[:nt])
    s = L.spec
    per = {"gate": FF * qg.row_bytes(s.gate_type, D), "up": FF * qg.row_bytes(s.up_type, D), "down": D * qg.row_bytes(s.down_type, FF)}
    host = {k: np.zeros(EXPERTS * v, np.uint8) for k, v in per.items()}
    for e in np.unique(ids[ids >= 0]):
        for k in host:
            host[k][e * per[k]:(e + 1) * per[k]] = synth.read_expert(L, k, int(e))
    router = np.empty(EXPERTS * D * 4, np.uint8)
    qg.call("read", router.ctypes.data, L.bufs["router"].p, router.nbytes)
    shared = {}
    if wl.shared:
        for name in ("sh_gate", "sh_up", "sh_down", "sh_inp"):
            buf = np.empty(L.bufs[name].nbytes, np.uint8)
            qg.call("read", buf.ctypes.data, L.bufs[name].p, buf.nbytes)
            shared[name] = buf
    hc = host_cpus()
    threads = cpu_threads()
    ws = ref.qc_create(max(nt, 1), threads)
    out = np.empty((nt, D), np.float32)
    logits = np.empty((nt, EXPERTS), np.float32)
    g = np.empty((nt, FF), np.float32)
    u = np.empty((nt, FF), np.float32)
    so = np.empty((nt, D), np.float32)
    lg = np.empty((nt, 1), np.float32)
    x = np.ascontiguousarray(wl.x[:nt], np.float32)

    def run():
        assert ref.qc_matmul(logits.ctypes.data, router.ctypes.data, 0, EXPERTS, D, x.ctypes.data, nt, threads) == 0
        assert ref.qc_moe(ws, out.ctypes.data, x.ctypes.data, ids.ctypes.data, w.ctypes.data, nt,
                          host["gate"].ctypes.data, s.gate_type, host["up"].ctypes.data, s.up_type,
                          host["down"].ctypes.data, s.down_type) == 0
        if wl.shared:
            st = s.sh_types
            assert ref.qc_matmul(g.ctypes.data, shared["sh_gate"].ctypes.data, st[0], FF, D, x.ctypes.data, nt, threads) == 0
            assert ref.qc_matmul(u.ctypes.data, shared["sh_up"].ctypes.data, st[1], FF, D, x.ctypes.data, nt, threads) == 0
            mid = (g / (1 + np.exp(-g))) * u
            assert ref.qc_matmul(so.ctypes.data, shared["sh_down"].ctypes.data, st[2], D, FF, mid.ctypes.data, nt, threads) == 0
            assert ref.qc_matmul(lg.ctypes.data, shared["sh_inp"].ctypes.data, 0, 1, D, x.ctypes.data, nt, threads) == 0
            out[:] += so / (1 + np.exp(-lg))

    for _ in range(3):
        run()
    times = []
    t_end = time.time() + budget_s
    while len(times) < 20 or (time.time() < t_end and len(times) < 2000):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    ref.qc_destroy(ws)
    med = float(np.median(times))
    parts = "router qc_matmul + qc_moe" + (" + shared expert (3 qc_matmul + gate)" if wl.shared else "")
    return {"value": round(nt / med, 1), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"cpu.c {parts} on layer 0, {nt} tokens"
                      f"{f' (the first {nt} of the {wl.nt}-token batch, their GPU routing)' if nt < wl.nt else ''}, "
                      f"isa={ref.qc_backend_name().decode()}; "
                      f"median of {len(times)} runs after 3 warm-ups; {threads} OpenMP threads "
                      f"(OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND')}, OMP_PLACES={os.environ.get('OMP_PLACES')}) on "
                      f"{hc['physical_cores']} physical cores / {hc['logical_cpus']} logical CPUs, {hc['sockets']} socket(s), "
                      f"{hc['model']}",
            "host": hc, "isa": ref.qc_backend_name().decode()}


def bench_stack(args, cpu_budget: float | None = None) -> dict:
    """Config 2: 48 seeded config-0 layers, one token, replayed as one graph.
    With cpu_budget, also the reference's cpu.c on the same stack
    (cpu_stack_baseline)."""
    n_layers = args.layers if args.layers != 16 else 48
    specs = [synth.LayerSpec(seed=9000 + l) for l in range(n_layers)]
    layers = [synth.build_layer(s) for s in specs]
    arr = (qg.MoeLayer * n_layers)(*[l.desc for l in layers])
    h = qg.host()
    stack = h.nm_stack_create(arr, n_layers, 1, 0)
    if not stack:
        raise RuntimeError(h.nm_last_error().decode())
    x0 = synth.inputs(31, 1, D)
    hid = h.nm_stack_hidden(stack)
    for _ in range(max(1, args.warmup // 10)):
        qg.call("write", hid, x0.ctypes.data, x0.nbytes)
        if h.nm_stack_forward(stack, 1, 1):
            raise RuntimeError(h.nm_last_error().decode())
    qg.call("sync")
    steps = max(1, args.steps // 10)
    b, e = qg.Event(), qg.Event()
    b.record()
    for _ in range(steps):
        if h.nm_stack_forward(stack, 1, 1):
            raise RuntimeError(h.nm_last_error().decode())
    e.record()
    qg.call("sync")
    ms = qg.elapsed_ms(b, e) / steps
    h.nm_stack_destroy(stack)
    nbytes = n_layers * layer_bytes(1, 10, False)
    r = {"ms": ms, "layers": n_layers, "bytes": nbytes, "steps": steps}
    if cpu_budget:
        r["cpu"] = cpu_stack_baseline(layers, arr, x0, cpu_budget)
    return r


def cpu_stack_baseline(layers, arr, x0: np.ndarray, budget_s: float) -> dict | None:
    """The reference's cpu.c on the config-2 stack, one token: per layer
    h <- h + qc_moe(RMSNorm(h)) after the router's qc_matmul, over all 48
    layers.  Each layer's routing is the GPU stack's own (a recorded eager
    forward from the same input; the reference's CPU MoE receives its ids
    from the GPU, qwen.c:665-669), and only the 10 routed experts of a layer
    are copied to the host, renumbered 0..9 (qc_moe's work depends only on
    the selected experts)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    try:
        import oracle as O
    except Exception:
        return None
    ref = O.ref_lib(D)
    if ref is None:
        return None
    n_layers = len(layers)
    h = qg.host()
    rec = h.nm_stack_create(arr, n_layers, 1, 1)
    if not rec:
        raise RuntimeError(h.nm_last_error().decode())
    qg.call("write", h.nm_stack_hidden(rec), x0.ctypes.data, x0.nbytes)
    if h.nm_stack_forward(rec, 1, 0):
        raise RuntimeError(h.nm_last_error().decode())
    qg.call("sync")
    per = {"gate": FF * qg.row_bytes(12, D), "up": FF * qg.row_bytes(12, D), "down": D * qg.row_bytes(12, FF)}
    cpu_layers = []
    for l, L in enumerate(layers):
        pi, pw = C.c_void_p(), C.c_void_p()
        if h.nm_stack_record(rec, l, None, C.byref(pi), C.byref(pw), None):
            raise RuntimeError(h.nm_last_error().decode())
        ids = np.empty((1, TOP), np.int32)
        w = np.empty((1, TOP), np.float32)
        qg.call("read", ids.ctypes.data, pi.value, ids.nbytes)
        qg.call("read", w.ctypes.data, pw.value, w.nbytes)
        host = {k: np.empty(TOP * v, np.uint8) for k, v in per.items()}
        for slot, ex in enumerate(ids[0]):
            for k in host:
                host[k][slot * per[k]:(slot + 1) * per[k]] = synth.read_expert(L, k, int(ex))
        router = np.empty(EXPERTS * D * 4, np.uint8)
        qg.call("read", router.ctypes.data, L.bufs["router"].p, router.nbytes)
        cpu_layers.append((router, host, np.arange(TOP, dtype=np.int32)[None, :].copy(), w))
    h.nm_stack_destroy(rec)
    threads = cpu_threads()
    ws = ref.qc_create(1, threads)
    logits = np.empty((1, EXPERTS), np.float32)
    out = np.empty((1, D), np.float32)

    def run():
        hs = x0.astype(np.float32).copy()
        for router, host, ids, w in cpu_layers:
            xn = synth.rmsnorm(hs)
            assert ref.qc_matmul(logits.ctypes.data, router.ctypes.data, 0, EXPERTS, D, xn.ctypes.data, 1, threads) == 0
            assert ref.qc_moe(ws, out.ctypes.data, xn.ctypes.data, ids.ctypes.data, w.ctypes.data, 1,
                              host["gate"].ctypes.data, 12, host["up"].ctypes.data, 12, host["down"].ctypes.data, 12) == 0
            hs += out
    for _ in range(3):
        run()
    times, t_end = [], time.time() + budget_s
    while len(times) < 20 or (time.time() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    ref.qc_destroy(ws)
    med = float(np.median(times))
    hc = host_cpus()
    return {"value": round(1 / med, 2), "unit": "tokens/s", "ms_per_token": round(med * 1e3, 3), "cores": threads,
            "kind": "reference",
            "sample": f"cpu.c router qc_matmul + qc_moe per layer over the {n_layers}-layer stack, 1 token, the GPU "
                      f"stack's routing, isa={ref.qc_backend_name().decode()}; median of {len(times)} runs after 3 "
                      f"warm-ups; {threads} OpenMP threads on {hc['physical_cores']} physical cores, {hc['model']}"}


class PrefillWorkload:
    """Config 3: one layer (906 MB of experts, above the 256 MB Infinity
    Cache), 2048 seeded RMS-normed tokens, Zipf(1.1)-biased router."""

    def __init__(self, nt: int, seed: int):
        self.nt, self.shared = nt, False
        self.spec = synth.LayerSpec(seed=seed, gate_type=12, up_type=12, down_type=20, bias_seed=seed + 1)
        self.layers = [synth.build_layer(self.spec)]
        self.fw = synth.Forward(D, FF, nt)
        self.x = synth.inputs(seed + 2, nt, D)
        self.fw.x.set(self.x)

    def step(self, i: int = 0) -> None:
        self.fw.run(self.layers[0], self.nt)

    def routing(self, i: int = 0):
        self.step()
        qg.call("sync")
        return self.fw.ids.get()[:self.nt], self.fw.flags.get()[:self.nt]


def bench_prefill(args, data: str) -> dict:
    nt = args.batch if args.batch is not None else 2048
    wl = PrefillWorkload(nt, seed=9300)
    ids, _ = wl.routing()
    n_e = np.bincount(ids[ids >= 0].ravel(), minlength=EXPERTS)
    dense = n_e >= DENSE_MIN
    g = C.c_void_p()
    qg.call("graph_begin", C.byref(g))
    wl.step()
    qg.call("graph_end", g)
    for _ in range(args.warmup):
        qg.call("graph_launch", g)
    qg.call("sync")
    b, e = qg.Event(), qg.Event()
    b.record()
    for _ in range(args.steps):
        qg.call("graph_launch", g)
    e.record()
    qg.call("sync")
    ms = qg.elapsed_ms(b, e) / args.steps
    qg.lib().qg_graph_destroy(g)
    kern = kernel_times(wl.step, PF_KERNELS, args.steps)
    # the dense experts' gate/up in a launch of their own, on fp16 (mode 2)
    # and on int8 matrix cores (mode 1), timed the same way
    split = {}
    for mode in () if getattr(args, "no_split", False) else (2, 1):
        prev = qg.lib().qg_prefill_int8_dense(mode)
        try:
            split[mode] = kernel_times(wl.step, PF_KERNELS, args.steps).get("gate_up_dense")
        finally:
            qg.lib().qg_prefill_int8_dense(prev)
    # algorithmic matrix-core work: 2 ops per multiply-add of the useful products
    ops_gu = lambda rows: 2.0 * rows * 2 * D * FF
    ops_dn = lambda rows: 2.0 * rows * D * FF
    rows_dense, rows_all = int(n_e[dense].sum()), int(n_e.sum())
    t_gu = kern.get("gate_up")
    achieved = ops_gu(rows_all) / (t_gu * 1e-3) / 1e12 if t_gu else None
    t_experts = sum(kern.get(k, 0) for k in ("gate_up", "down"))
    util = lambda ops, t: round(ops / (t * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4) if t and ops else None
    touched = int(np.count_nonzero(n_e))
    layer_b = ROUTER_BYTES + touched * EXPERT_BYTES + nt * (2 * D * 4 + 80)
    line = {
        "metric": METRIC, "value": round(nt / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": DTYPE, "data": data,
        "config": {"workload": f"config3: routed-MoE prefill, B={nt}, D=2048, 512 experts top-10, F=512, Q4_K gate/up, "
                               "IQ4_NL down, router biased to Zipf(1.1) expert popularity; one captured graph per step",
                   "batch_tokens": nt, "experts_touched": touched, "dense_experts": int(dense.sum()),
                   "dense_rows": rows_dense, "rows": rows_all, "max_rows": int(n_e.max()),
                   "matrix_cores": "fp16 16x16x32 MFMA, exact integer weights x fp16 hi/lo activation planes, fp32 accumulate",
                   "expert_gemms_int8_util_algorithmic": util(ops_gu(rows_all) + ops_dn(rows_all), t_experts),
                   "expert_gemms_fp16_util_issued": round(2 * (ops_gu(rows_all) + ops_dn(rows_all)) / (t_experts * 1e-3) / 1e12
                                                          / FP16_PEAK_TFLOPS, 4) if t_experts else None,
                   "dense_experts_gate_up": {
                       "rows": rows_dense,
                       "us_fp16": round(split[2] * 1000, 2) if split.get(2) else None,
                       "int8_util_algorithmic_fp16": util(ops_gu(rows_dense), split.get(2)),
                       "us_int8_variant": round(split[1] * 1000, 2) if split.get(1) else None,
                       "int8_util_algorithmic_int8_variant": util(ops_gu(rows_dense), split.get(1)),
                       "int8_variant_arithmetic": "int8 16x16x32 MFMA per Q4_K group and activation plane (two int8 "
                                                  "planes, row scale), per-group int32->fp32 scaling"},
                   "expert_gemm_TOPS_all": round((ops_gu(rows_all) + ops_dn(rows_all)) / (t_experts * 1e-3) / 1e12, 1) if t_experts else None,
                   "layer_bytes": int(layer_b), "layer_hbm_frac": round(layer_b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "kernel_us": {k: round(v * 1000, 2) for k, v in kern.items()}},
        "roofline": {"bound": "mfma", "kernel": "gate_up", "achieved": round(achieved, 1) if achieved else None,
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4) if achieved else None,
                     **load_traffic(f"gate_up_config3_B{nt}", 1), "algorithmic_ops": ops_gu(rows_all)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(wl, args.cpu_budget)
    return line


MM_SHAPES = (("qkv", 10240, 2560), ("z", 6144, 2560), ("out", 2560, 6144))


def bench_matmul(args, data) -> dict:
    """qg_matmul on the reference's dense projections at D = 2560 (the gated
    DeltaNet qkv, z and out matrices of qwen.c:533-543) in Q4_K, `batch`
    tokens (default 1): each shape's weights rotate over enough seeded copies
    (> 512 MB) that every launch streams from HBM.  value = weight bytes of the
    three projections / their summed time; roofline on the largest (qkv)."""
    nt = args.batch if args.batch is not None else 1
    rng = np.random.default_rng(5)
    per, total_bytes, total_us, cpu = {}, 0, 0.0, None
    for name, rows, cols in MM_SHAPES:
        nbytes = rows * qg.row_bytes(12, cols)
        copies = max(4, (512 << 20) // nbytes + 1)
        w = qg.Device(nbytes=nbytes * copies)
        for c in range(copies):
            qg.call("synth_matrix", w.p + c * nbytes, 12, 77, (9 << 32) | c, rows, cols, qg.F(0.02))
        x = qg.Device(rng.standard_normal((nt, cols)).astype(np.float32))
        out = qg.Device(shape=(nt, rows), dtype=np.float32)
        for i in range(args.warmup):
            qg.call("matmul", out.p, w.p + (i % copies) * nbytes, 12, rows, cols, x.p, nt)
        b, e = qg.Event(), qg.Event()
        qg.call("sync")
        b.record()
        for i in range(args.steps):
            qg.call("matmul", out.p, w.p + (i % copies) * nbytes, 12, rows, cols, x.p, nt)
        e.record()
        qg.call("sync")
        us = qg.elapsed_ms(b, e) * 1e3 / args.steps
        per[name] = {"rows": rows, "cols": cols, "us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1)}
        total_bytes += nbytes
        total_us += us
        if name == "qkv" and not args.no_cpu:
            cpu = cpu_matmul(w, rows, cols, x, nt, args.cpu_budget)
        w.free()
    q = per["qkv"]
    achieved = q["GBps"]
    return {"metric": "qg_matmul dense-projection weight streaming (Q4_K GEMV/GEMM, qkv+z+out)",
            "value": round(total_bytes / total_us / 1e3, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(total_us / 1e3, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": data,
            "config": {"workload": f"qg_matmul, Q4_K, D=2560 dense projections (qkv 10240x2560, z 6144x2560, out 2560x6144), "
                                   f"{nt} tokens, exact reference order", "batch_tokens": nt, "per_shape": per},
            "roofline": {"bound": "hbm", "kernel": "mm_tile_kernel (qkv)", "achieved": achieved, "peak": 8000.0, "unit": "GB/s",
                         "frac": round(achieved / 8000.0, 4), "traffic": None},
            "cpu_baseline": cpu}


def cpu_matmul(w, rows, cols, x, nt, budget_s) -> dict | None:
    """The reference's qc_matmul (cpu.c:119-148) on the same Q4_K matrix and tokens."""
    sys.path.insert(0, str(ROOT / "oracle"))
    try:
        import oracle as O
    except Exception:
        return None
    ref = O.ref_lib(2048)
    if ref is None:
        return None
    nbytes = rows * qg.row_bytes(12, cols)
    hw = np.empty(nbytes, np.uint8)
    qg.call("read", hw.ctypes.data, w.p, nbytes)
    hx = x.get()
    out = np.empty((nt, rows), np.float32)
    threads = cpu_threads()
    run = lambda: ref.qc_matmul(out.ctypes.data, hw.ctypes.data, 12, rows, cols, hx.ctypes.data, nt, threads)
    for _ in range(3):
        assert run() == 0
    times, t_end = [], time.time() + budget_s
    while len(times) < 20 or (time.time() < t_end and len(times) < 2000):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"cpu.c qc_matmul, Q4_K {rows}x{cols}, {nt} tokens, isa={ref.qc_backend_name().decode()}; "
                      f"median of {len(times)} runs after 3 warm-ups (one host-resident matrix)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2, 3, 4))
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sections", action="store_true",
                    help="default workload only: leave out the other configurations of the metric (B=1/4/8, config 4, "
                         "the 48-layer stack, the prefill)")
    ap.add_argument("--matmul", action="store_true",
                    help="measure qg_matmul on the dense projections instead of the MoE layer (--batch tokens, default 1)")
    ap.add_argument("--no-split", action="store_true",
                    help="--config 3: skip the timings of the dense experts in launches of their own")
    ap.add_argument("--int8-dense", action="store_true",
                    help="with --counter-pass: the prefill dense experts' gate/up in a launch of their own on int8")
    ap.add_argument("--dense-split", action="store_true",
                    help="with --counter-pass: the prefill dense experts' gate/up in a launch of their own on fp16")
    ap.add_argument("--counter-pass", type=int, default=0, metavar="P",
                    help="for rocprofv3 counter runs: build the workload, print each layer's routing and algorithmic "
                         "bytes as one JSON line, then run P eager passes over the layers in order (dispatch k of a "
                         "kernel is layer k %% layers) and exit")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain copy kernel over MIB MiB 5 times (qg_unary identity: MIB read, MIB "
                         "written; the known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE to bytes) and exit")
    args = ap.parse_args()
    # the CPU baseline's OpenMP placement (read when the runtime starts)
    host_cpus()
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src, dst = qg.Device(nbytes=n), qg.Device(nbytes=n)
        for _ in range(5):
            qg.call("unary", dst.p, src.p, n // 4, 2, qg.F(1.0))
        qg.call("sync")
        print(json.dumps({"calibration_copy_bytes": n, "copies": 5, "kernel": "unary_kernel (identity)"}), flush=True)
        return 0
    if args.counter_pass:
        return counter_pass(args)
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the layer; --gpus {args.gpus} is not supported "
              "(this build runs on one MI355X; sharding the layer over several GPUs is designed, not built)",
              file=sys.stderr)
        return 2
    data = "synthetic (seeded N(0,0.02) weights quantised to Q4_K/IQ4_NL on the device; seeded RMS-normed inputs)"
    if args.matmul:
        if args.batch is not None and not 1 <= args.batch <= 8192:
            print("matmul batch must be 1..8192", file=sys.stderr)
            return 2
        print(json.dumps(bench_matmul(args, "synthetic (seeded N(0,0.02) weights quantised to Q4_K on the device; "
                                                "seeded N(0,1) inputs)")), flush=True)
        return 0
    if args.config == 3:
        if args.batch is not None and not 18 <= args.batch <= 8192:
            print("prefill batch must be 18..8192", file=sys.stderr)
            return 2
        print(json.dumps(bench_prefill(args, data)), flush=True)
        return 0
    batch = args.batch if args.batch is not None else (17 if args.config in (1, 4) else 1)
    if not 1 <= batch <= 17:
        print("decode batch must be 1..17", file=sys.stderr)
        return 2

    if args.config == 2:
        r = bench_stack(args, None if args.no_cpu else args.cpu_budget)
        ms = r["ms"]
        line = {
            "metric": METRIC, "value": round(1 / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": r["steps"], "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": DTYPE, "data": data,
            "config": {"workload": f"config2: {r['layers']}-layer routed-MoE stack, B=1, D=2048, 512 experts top-10, F=512, Q4_K; "
                                   "h <- h + MoE(RMSNorm(h)); one captured graph",
                       "layers": r["layers"], "stack_bytes": int(r["bytes"]),
                       "stack_hbm_GBps": round(r["bytes"] / (ms * 1e-3) / 1e9, 1),
                       "stack_hbm_frac": round(r["bytes"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                       "us_per_layer": round(ms * 1000 / r["layers"], 3)},
            "roofline": None, "cpu_baseline": r.get("cpu"),
        }
        print(json.dumps(line), flush=True)
        return 0

    wl = Workload(args.config, batch, args.layers, seed=9000)
    r = decode_result(wl, args.steps, args.warmup)
    names = {0: f"config0: routed-MoE layer, B={wl.nt}, D=2048, 512 experts top-10, F=512, Q4_K",
             1: f"config1: routed-MoE layer, B={wl.nt}, D=2048, 512 experts top-10, F=512, Q4_K gate/up, IQ4_NL down, shared Q4_K expert",
             4: f"config4: config 1 at B={wl.nt} with 128/512 resident experts per layer and 90% coverage flags"}
    line = {
        "metric": METRIC,
        "value": round(wl.nt / (r["ms"] * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "data": data,
        "config": {"workload": names[args.config], "arithmetic": ARITHMETIC,
                   "batch_tokens": wl.nt, "layers_rotated": len(wl.layers), "unique_experts_mean": r["U"],
                   "layer_bytes": int(r["nbytes"]), "layer_hbm_GBps": round(r["nbytes"] / (r["ms"] * 1e-3) / 1e9, 1),
                   "layer_hbm_frac": r["layer_frac"],
                   "kernel_us": {k: round(v * 1000, 2) for k, v in r["kern"].items()}},
        "roofline": {"bound": "hbm", "kernel": "gate_up", "achieved": round(r["achieved"], 1) if r["achieved"] else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["achieved"] / HBM_PEAK_GBS, 4) if r["achieved"] else None,
                     **load_traffic(f"gate_up_config{args.config}_B{wl.nt}", len(wl.layers)),
                     "algorithmic_bytes": int(r["gu_bytes"])},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(wl, args.cpu_budget)
    if args.config == 1 and args.batch is None and not args.no_sections:
        # the rest of the metric in the same line: B=4/8 on the same layers,
        # config 4, B=1 (config 0), the 48-layer stack and the prefill
        line["config"]["sections"] = sections(wl, args)
    print(json.dumps(line), flush=True)
    return 0


def counter_pass(args) -> int:
    """Eager passes over the workload's layers in order, for counter runs."""
    if args.int8_dense or args.dense_split:
        qg.lib().qg_prefill_int8_dense(1 if args.int8_dense else 2)
    if args.config == 3:
        nt = args.batch if args.batch is not None else 2048
        wl = PrefillWorkload(nt, seed=9300)
        ids, _ = wl.routing()
        n_e = np.bincount(ids[ids >= 0].ravel(), minlength=EXPERTS)
        dense = n_e >= DENSE_MIN
        touched = int(np.count_nonzero(n_e))
        info = {"config": 3, "batch": nt, "layers": [{"layer": 0, "experts_touched": touched, "dense_experts": int(dense.sum()),
                                                       "rows": int(n_e.sum()),
                                                       "gate_up_algorithmic_bytes": touched * GATEUP_BYTES + nt * D * 4}]}
    else:
        batch = args.batch if args.batch is not None else (17 if args.config in (1, 4) else 1)
        wl = Workload(args.config, batch, args.layers, seed=9000)
        layers = []
        for i in range(len(wl.layers)):
            u = wl.unique_experts(i)
            layers.append({"layer": i, "unique_experts": u, "gate_up_algorithmic_bytes": int(gateup_bytes(batch, u, wl.shared)),
                           "down_algorithmic_bytes": int(down_bytes(batch, u, wl.shared))})
        info = {"config": args.config, "batch": batch, "layers": layers}
    qg.call("sync")
    print(json.dumps(info), flush=True)
    for _ in range(args.counter_pass):
        for i in range(len(wl.layers)):
            wl.step(i)
    qg.call("sync")
    return 0


DTYPE = "f16x2+f32"
ARITHMETIC = ("router fp32 in the reference's order (ids bit-exact); experts on fp16 16x16x32 MFMA: exact integer "
              "weights x two fp16 activation planes (hi = fp16(x), lo = fp16(x - hi), ~22 significant bits), fp32 "
              "accumulate, fp32 group/superblock scales")


def decode_result(wl: Workload, steps: int, warmup: int) -> dict:
    uniq = [wl.unique_experts(i) for i in range(len(wl.layers))]
    U = float(np.mean(uniq))
    ms, kern = time_decode(wl, steps, warmup)
    gu_ms = kern.get("gate_up")
    nbytes = layer_bytes(wl.nt, U, wl.shared)
    gu_bytes = gateup_bytes(wl.nt, U, wl.shared)
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9 if gu_ms else None
    return {"ms": ms, "kern": kern, "U": U, "nbytes": nbytes, "gu_bytes": gu_bytes, "achieved": achieved,
            "layer_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def decode_section(wl: Workload, steps: int, warmup: int, cpu_budget: float | None) -> dict:
    r = decode_result(wl, steps, warmup)
    out = {"tokens_per_s": round(wl.nt / (r["ms"] * 1e-3), 1), "us_per_layer": round(r["ms"] * 1e3, 2),
           "unique_experts_mean": r["U"], "layer_bytes": int(r["nbytes"]), "layer_hbm_frac": r["layer_frac"],
           "gate_up_GBps": round(r["achieved"], 1) if r["achieved"] else None,
           "gate_up_hbm_frac": round(r["achieved"] / HBM_PEAK_GBS, 4) if r["achieved"] else None,
           "kernel_us": {k: round(v * 1000, 2) for k, v in r["kern"].items()}}
    if cpu_budget:
        c = cpu_baseline(wl, cpu_budget)
        if c:
            out["cpu_tokens_per_s"] = c["value"]
    return out


def graph_floor(reps: int = 50) -> dict:
    """What a chain of kernels costs whatever they compute: the device time
    per dependent one-block kernel (qg_zero of 256 bytes) inside one captured
    graph of 100 such kernels, the resulting floor of a 3- and a 5-kernel
    layer, and the host-side replay rate of a one-kernel graph (back-to-back
    hipGraphLaunch calls)."""
    buf = qg.Device(nbytes=256)

    def replay_us(n, r):
        g = C.c_void_p()
        qg.call("graph_begin", C.byref(g))
        for _ in range(n):
            qg.call("zero", buf.p, 256)
        qg.call("graph_end", g)
        for _ in range(5):
            qg.call("graph_launch", g)
        qg.call("sync")
        b, e = qg.Event(), qg.Event()
        b.record()
        for _ in range(r):
            qg.call("graph_launch", g)
        e.record()
        qg.call("sync")
        qg.lib().qg_graph_destroy(g)
        return qg.elapsed_ms(b, e) * 1e3 / r
    per = replay_us(100, reps) / 100
    return {"per_dependent_kernel_us": round(per, 2), "floor_3_kernels_us": round(3 * per, 2),
            "floor_5_kernels_us": round(5 * per, 2), "one_kernel_graph_replay_us": round(replay_us(1, 200), 2)}


def sections(wl1: Workload, args) -> dict:
    """Every other configuration of the metric, measured in the same run."""
    steps, warm = min(args.steps, 100), min(args.warmup, 10)
    cpu = None if args.no_cpu else min(args.cpu_budget, 3.0)
    out = {"graph_floor_us": graph_floor()}
    for nt in (4, 8):
        wl1.nt = nt
        wl1.fw = synth.Forward(D, FF, nt)
        wl1.x = synth.inputs(9000 + 1000 + nt, nt, D, correlated=True)
        wl1.fw.x.set(wl1.x)
        out[f"config1_B{nt}"] = decode_section(wl1, steps, warm, cpu)
    # config 4: the same layers with 128 resident experts each and the coverage flags
    wl1.nt = 17
    wl1.fw = synth.Forward(D, FF, 17)
    wl1.x = synth.inputs(9000 + 1000, 17, D, correlated=True)
    wl1.fw.x.set(wl1.x)
    for L in wl1.layers:
        mask = resident_set(L, batch_seed=9000 + 1000, noise_seed=L.spec.seed + 77)
        L.bufs["resident"] = qg.Device(mask)
        L.desc.resident, L.desc.threshold = L.bufs["resident"].p, 0.10
    flags = np.concatenate([wl1.routing(i)[1] for i in range(len(wl1.layers))])
    sec = decode_section(wl1, steps, warm, cpu)
    sec["flag_counts"] = np.bincount(flags, minlength=4).tolist()
    sec["resident_ranking"] = ("128 of 512 experts per layer by activation count, then routed weight, then id "
                               "(qwen/README.md:38), over 4096 tokens from 8 correlated contexts, one of them the batch's")
    out["config4_B17"] = sec
    del wl1.layers[:]
    gc.collect()
    wl0 = Workload(0, 1, args.layers, seed=9000)
    out["config0_B1"] = decode_section(wl0, steps, warm, cpu)
    del wl0
    gc.collect()
    a = argparse.Namespace(layers=48, warmup=20, steps=40)
    r = bench_stack(a, cpu)
    out["config2_stack48_B1"] = {"tokens_per_s": round(1 / (r["ms"] * 1e-3), 1), "us_per_layer": round(r["ms"] * 1000 / 48, 2),
                                 "stack_bytes": int(r["bytes"]),
                                 "stack_hbm_frac": round(r["bytes"] / (r["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if r.get("cpu"):
        out["config2_stack48_B1"]["cpu_tokens_per_s"] = r["cpu"]["value"]
        out["config2_stack48_B1"]["cpu_ms_per_token"] = r["cpu"]["ms_per_token"]
    gc.collect()
    a = argparse.Namespace(batch=2048, warmup=warm, steps=min(args.steps, 50), no_cpu=cpu is None, cpu_budget=cpu or 0)
    p = bench_prefill(a, "")
    pc = p["config"]
    out["config3_prefill_B2048"] = {
        "tokens_per_s": p["value"], "ms_per_layer": p["ms_per_step"],
        "gate_up_TOPS": p["roofline"]["achieved"], "gate_up_int8_frac": p["roofline"]["frac"],
        "expert_gemms_int8_util_algorithmic": pc["expert_gemms_int8_util_algorithmic"],
        "dense_experts_gate_up": pc["dense_experts_gate_up"],
        "dense_experts": pc["dense_experts"], "layer_hbm_frac": pc["layer_hbm_frac"], "kernel_us": pc["kernel_us"]}
    if p.get("cpu_baseline"):
        out["config3_prefill_B2048"]["cpu_tokens_per_s"] = p["cpu_baseline"]["value"]
        out["config3_prefill_B2048"]["cpu_sample"] = p["cpu_baseline"]["sample"]
    return out


def load_traffic(name: str, layers: int) -> dict:
    """HBM bytes per launch of the roofline kernel, measured with rocprofv3
    FETCH_SIZE/WRITE_SIZE counters scaled by a copy kernel of known size
    (profiles/traffic.json, written from the counter runs).  Reported only
    when the counter runs covered the same layers this run averages over
    (the first `layers` seeded layers of the workload), so `traffic` and
    `algorithmic_bytes` describe the same launches; the record's own
    algorithmic mean and the ratio ride along."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        rec = json.loads(p.read_text()).get(name) if p.exists() else None
    except (OSError, ValueError):
        rec = None
    if not rec or sorted(l["layer"] for l in rec.get("layers", [])) != list(range(layers)):
        return {"traffic": None}
    return {"traffic": rec["bytes"], "traffic_algorithmic_bytes": rec["algorithmic_bytes"],
            "traffic_over_algorithmic": rec["ratio"], "traffic_source": rec.get("profile")}


if __name__ == "__main__":
    sys.exit(main())
