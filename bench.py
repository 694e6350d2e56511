"""Benchmark: neuron-steps/s and synaptic events/s of the fly-scale conductance-LIF
forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward call of the hot path over one batch of synthetic input: 8 trials
x 2000 time steps (dt 0.1 ms) of a 140k-neuron, ~50M-synapse network from rest, with
the input resident in HBM. Prints one JSON line (see the keys below), including the
roofline of the dominant kernel (``wt_cond_run``, timed with HIP events on its stream)
and the CPU baseline (the oracle, on a bounded slice of the same workload).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from wiretorch_amd import engine, synthetic  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "neuron-steps/s and synaptic events/s, fly-scale conductance LIF, 1 MI355X"


def algorithmic_bytes(B, T, N, S, events):
    """Bytes the step must move (per neuron-trial-step: v r/w 8, g rise+decay r/w 16*S,
    refractory counter r/w 8, spike write 4; per neuron-step: six parameter reads 24;
    per delivered event: target index + weight 8)."""
    return T * (B * N * (8 + 16 * S + 8 + 4) + 24 * N) + 8 * events


def delivered_events(spikes, x, drive):
    """Recurrent spikes x out-degree + input spikes x input out-degree, all trials/steps."""
    rec, ff = drive.sparse_recurrent, drive.sparse_feedforward
    out_rec = rec.out_degree().to(spikes.device, torch.float64)
    out_ff = ff.out_degree().to(x.device, torch.float64)
    per_src = spikes.double().sum(dim=(0, 1))
    per_in = (x != 0).double().sum(dim=(0, 1))
    return float(per_src @ out_rec + per_in @ out_ff)


def measured_traffic():
    """HBM bytes per launch of wt_cond_run on this workload, from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE summary (calibrated against a copy of known size), or None."""
    path = ROOT / "profiles" / "wt_cond_run_config2_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(wl, steps):
    """The oracle (the reference's PyTorch step restated, compressed propagation) on the
    first ``steps`` steps of the same workload, on this host's cores."""
    import oracle.dynamics as oracle_engine
    from wiretorch_amd.synthetic import sparse_drive

    rec = wl.drive.sparse_recurrent.to("cpu")
    ff = wl.drive.sparse_feedforward.to("cpu")
    drive, p = sparse_drive(rec, ff, wl.N, 0.1, "cpu")
    B = wl.x.shape[0]
    x = torch.from_numpy(wl.x[:, :steps]).float()
    v, g, c = synthetic.rest_state(B, wl.N, wl.S)
    with torch.no_grad():
        oracle_engine.simulate(v, g, x[:, :2], drive, p, refractory=c)  # warm-up
        t0 = time.perf_counter()
        oracle_engine.simulate(v, g, x, drive, p, refractory=c)
        dt = time.perf_counter() - t0
    return {
        "value": B * wl.N * steps / dt,
        "unit": "neuron-steps/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle on the first {steps} of {wl.x.shape[1]} steps, all {B} trials "
                  f"({dt:.1f} s)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-steps", type=int, default=int(os.environ.get("BENCH_CPU_STEPS", 400)))
    ap.add_argument("--T", type=int, default=2000)
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run one device-to-device copy of this many bytes (the "
                         "reference kernel for calibrating rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_bytes:
        src = torch.ones(args.copy_bytes // 4, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": args.copy_bytes}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(the hot path runs on a single GPU)", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    wl = synthetic.fly_scale(T=args.T, device=dev)
    x = torch.from_numpy(wl.x).float().to(dev)
    drive, p = wl.drive, wl.physiology
    B, T, N, S = x.shape[0], x.shape[1], wl.N, wl.S
    v0, g0, c0 = synthetic.rest_state(B, N, S, dev)
    print(f"# built config2 in {time.perf_counter() - t_build:.1f} s: N {N}, "
          f"{drive.sparse_recurrent.n_edges} synapses, B {B}, T {T}", file=sys.stderr, flush=True)

    def step():
        return engine.simulate(v0, g0, x, drive, p, refractory=c0)

    with torch.no_grad():
        for _ in range(args.warmup):
            run = step()
        torch.cuda.synchronize()
        engine.LAUNCH_EVENTS = []
        t0 = time.perf_counter()
        for _ in range(args.steps):
            run = step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        launches = engine.LAUNCH_EVENTS
        engine.LAUNCH_EVENTS = None
    kernel_ms = float(np.mean([a.elapsed_time(b) for a, b in launches]))
    events = delivered_events(run.spikes, x, drive)
    ms_per_step = wall * 1e3 / args.steps
    neuron_steps = B * N * T
    value = neuron_steps / (ms_per_step / 1e3)
    bytes_per_launch = algorithmic_bytes(B, T, N, S, events)
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    rate_hz = float(run.spikes.mean()) / (0.1e-3)
    print(f"# kernel {kernel_ms:.3f} ms/launch, wall {ms_per_step:.3f} ms/step, "
          f"rate {rate_hz:.2f} Hz, events/step {events / T:.0f}", file=sys.stderr, flush=True)
    cpu = cpu_baseline(wl, args.cpu_steps) if args.cpu_steps > 0 else None
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "neuron-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "synaptic_events_per_s": events / (ms_per_step / 1e3),
        "mean_rate_hz": rate_hz,
        "config": {
            "workload": "config2: fly-scale conductance-LIF forward",
            "neurons": N, "synapses": int(drive.sparse_recurrent.n_edges),
            "cell_types": 8000, "batch": B, "time_steps": T, "dt_ms": 0.1,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(),
            "kernel": "wt_cond_run",
            "kernel_ms": kernel_ms,
            "algorithmic_bytes_per_launch": bytes_per_launch,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
