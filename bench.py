#!/usr/bin/env python3
"""Benchmark of the routed-MoE layer on one MI355X.

Default workload: BASELINE config 1 at the 17-token speculative-verify batch
(Q4_K gate/up, IQ4_NL down, shared Q4_K expert with sigmoid gate, correlated
RMS-normed inputs).  A step is one layer forward (router -> top-10 -> experts
-> router-rank combine -> shared expert) through the C ABI's qg_moe_forward,
rotating over 16 distinct seeded layers (14.5 GB) so weights stream from HBM,
not from the 256 MB Infinity Cache.  Inputs are resident in HBM before the
timed region.

Printed: one JSON line.  value = tokens/s of the layer (batch / step time);
roofline = the dominant kernel's algorithmic bytes over its average duration,
timed with HIP events on the library's launch stream; cpu_baseline = the
reference's own cpu.c qc_moe (built from /root/reference into oracle/_ref) on
the same inputs, on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
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
ROUTER_BYTES = EXPERTS * D * 4
HBM_PEAK_GBS = 8000.0
METRIC = "routed-MoE tokens/s + % HBM peak at B=1/17; int8 MFMA util at 2048-tok prefill"


def layer_bytes(nt: int, unique: int, shared: bool) -> int:
    """Algorithmic HBM bytes of one layer forward (each touched expert once)."""
    b = ROUTER_BYTES + unique * EXPERT_BYTES + nt * (2 * D * 4 + 80)
    if shared:
        b += EXPERT_BYTES + D * 4
    return b


def gateup_bytes(nt: int, unique: int, shared: bool) -> int:
    per = FF * 1152 * 2  # gate + up rows of one Q4_K expert
    return (unique + (1 if shared else 0)) * per + nt * D * 4


class Workload:
    def __init__(self, config: int, batch: int, layers: int, seed: int):
        self.config, self.nt = config, batch
        shared = config in (1, 4)
        dt = 20 if config in (1, 3, 4) else 12
        self.shared = shared
        self.specs = [synth.LayerSpec(seed=seed + l, down_type=dt, shared=shared) for l in range(layers)]
        t0 = time.time()
        self.layers = [synth.build_layer(s) for s in self.specs]
        qg.call("sync")
        self.build_s = time.time() - t0
        self.fw = synth.Forward(D, FF, batch)
        self.x = synth.inputs(seed + 1000, batch, D, correlated=config in (1, 4))
        self.fw.x.set(self.x)

    def step(self, i: int) -> None:
        self.fw.run(self.layers[i % len(self.layers)], self.nt)

    def unique_experts(self, i: int) -> int:
        self.step(i)
        qg.call("sync")
        ids = self.fw.ids.get()[:self.nt]
        return len(np.unique(ids[(ids >= 0) & (ids < EXPERTS)]))


def time_steps(wl: Workload, steps: int, warmup: int) -> float:
    for i in range(warmup):
        wl.step(i)
    qg.call("sync")
    b, e = qg.Event(), qg.Event()
    b.record()
    for i in range(steps):
        wl.step(i)
    e.record()
    qg.call("sync")
    return qg.elapsed_ms(b, e) / steps


def time_phases(wl: Workload, steps: int) -> list[float]:
    """Average duration of each kernel phase (ms), from events recorded by the
    library between its launches on its own stream."""
    evs = [qg.Event() for _ in range(6)]
    arr = (C.c_void_p * 6)(*[e.p for e in evs])
    acc = np.zeros(5)
    for i in range(steps):
        qg.call("moe_phase_events", arr, 6)
        wl.step(i)
        qg.call("moe_phase_events", None, 0)
        qg.call("sync")
        acc += [qg.elapsed_ms(evs[k], evs[k + 1]) for k in range(5)]
    return list(acc / steps)


def cpu_baseline(wl: Workload, budget_s: float) -> dict | None:
    """The reference's qc_moe (cpu.c) on layer 0's routed experts for this batch,
    timed on the host cores; routing ids/weights from the GPU run of the same
    inputs (the reference's CPU path receives them from the GPU, qwen.c:665-669)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    try:
        import oracle as O
    except Exception:
        return None
    ref = O.ref_lib(D)
    if ref is None:
        return None
    L = wl.layers[0]
    wl.step(0)
    qg.call("sync")
    ids = wl.fw.ids.get()[:wl.nt].copy()
    w = wl.fw.w.get()[:wl.nt].copy()
    s = L.spec
    per = {"gate": FF * qg.row_bytes(s.gate_type, D), "up": FF * qg.row_bytes(s.up_type, D), "down": D * qg.row_bytes(s.down_type, FF)}
    host = {k: np.zeros(EXPERTS * v, np.uint8) for k, v in per.items()}
    for e in np.unique(ids[ids >= 0]):
        for k in host:
            host[k][e * per[k]:(e + 1) * per[k]] = synth.read_expert(L, k, int(e))
    cores = len(os.sched_getaffinity(0))
    threads = max(1, min(28, cores))
    ws = ref.qc_create(max(wl.nt, 1), threads)
    out = np.empty((wl.nt, D), np.float32)
    x = np.ascontiguousarray(wl.x, np.float32)

    def run():
        rc = ref.qc_moe(ws, out.ctypes.data, x.ctypes.data, ids.ctypes.data, w.ctypes.data, wl.nt,
                        host["gate"].ctypes.data, s.gate_type, host["up"].ctypes.data, s.up_type, host["down"].ctypes.data, s.down_type)
        assert rc == 0
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
    return {"value": round(wl.nt / med, 1), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"cpu.c qc_moe (routed experts of layer 0, {wl.nt} tokens, isa={ref.qc_backend_name().decode()}), "
                      f"median of {len(times)} runs after 3 warm-ups; OMP threads={threads} of {cores} host CPUs"}


def load_traffic(name: str):
    p = ROOT / "profiles" / "traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get(name)
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1))
    ap.add_argument("--batch", type=int, default=17)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the layer; --gpus {args.gpus} is not supported "
              "(this build runs on one MI355X; the multi-GPU sharding is described in DESIGN.md)", file=sys.stderr)
        return 2
    if not 1 <= args.batch <= 17:
        print("decode batch must be 1..17", file=sys.stderr)
        return 2

    wl = Workload(args.config, args.batch, args.layers, seed=9000)
    uniq = [wl.unique_experts(i) for i in range(len(wl.layers))]
    U = float(np.mean(uniq))
    ms = time_steps(wl, args.steps, args.warmup)
    phases = time_phases(wl, min(args.steps, 64))
    names = ["router", "route_dispatch", "gate_up", "down", "combine"]
    gu_ms = phases[2] if phases[2] > 0 else None
    nbytes = layer_bytes(wl.nt, U, wl.shared)
    gu_bytes = gateup_bytes(wl.nt, U, wl.shared)
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9 if gu_ms else None
    line = {
        "metric": METRIC,
        "value": round(wl.nt / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q4_K/IQ4_NL on the device; seeded RMS-normed inputs)",
        "config": {"workload": f"config{args.config}: routed-MoE layer, B={wl.nt}, D=2048, 512 experts top-10, F=512"
                               + (", Q4_K gate/up, IQ4_NL down, shared Q4_K expert" if args.config == 1 else ", Q4_K"),
                   "batch_tokens": wl.nt, "layers_rotated": len(wl.layers), "unique_experts_mean": U,
                   "layer_bytes": int(nbytes), "layer_hbm_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                   "layer_hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "phase_us": {n: round(v * 1000, 2) for n, v in zip(names, phases)}},
        "roofline": {"bound": "hbm", "kernel": "gate_up", "achieved": round(achieved, 1) if achieved else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
                     "traffic": load_traffic(f"gate_up_config{args.config}_B{wl.nt}"),
                     "algorithmic_bytes": int(gu_bytes)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(wl, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
