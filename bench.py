"""Benchmark: neuron-steps/s and synaptic events/s of the fly-scale conductance-LIF
forward (configuration 2, the headline workload) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 0|1|2|3|4] [--phases]

A step is one forward call of the hot path over one batch of synthetic input: 8 trials
x 2000 time steps (dt 0.1 ms) of a 140k-neuron, ~50M-synapse network from rest, with
the input resident in HBM. Prints one JSON line (see the keys below), including the
roofline of the dominant kernel (``wt_cond_run``, timed with HIP events on its stream)
and the CPU baseline (the oracle, on a bounded slice of the same workload).

``--config 1`` measures configuration 1 the same way (10,000 neurons, ~2M synapses, 32
trials x 5,000 steps, through the network API). ``--config 3`` measures the training
step: forward + backward of 64 trials x 500 steps of configuration 3's network (learnt
per-synapse weights, tau_mem and theta), the loss a squared error of 20 ms-binned rates;
its roofline is that of the part (forward, backward, weight gradient) with the largest
share of the step. ``--config 4`` measures the dense rate network (configuration 4, the
matrix-core path): a step is one forward + backward of 256 trials x 1000 steps of 4096 tanh rate
neurons with bf16 weights, from rest, with a linear read-out's squared error as the loss;
the roofline is that of the kernel with the largest share of the step, against the
matrix cores' dense peak in its arithmetic type.
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
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f32": 157.3}
METRIC = "neuron-steps/s and synaptic events/s, fly-scale conductance LIF, 1 MI355X"


def algorithmic_bytes(B, T, N, S, events):
    """Bytes the step must move (per neuron-trial-step: v r/w 8, g rise+decay r/w 16*S,
    refractory counter r/w 8, spike write 4; per neuron-step: six parameter reads 24;
    per delivered event: target index + weight 8)."""
    return T * (B * N * (8 + 16 * S + 8 + 4) + 24 * N) + 8 * events


def measured_traffic(summary="wt_cond_run_config2_traffic.md"):
    """HBM bytes per launch of a kernel on its workload, from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE summary (calibrated against a copy of known size), or None."""
    path = ROOT / "profiles" / summary
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def er_events(wl, spikes, x):
    """Delivered events of an Erdős–Rényi workload: spikes x out-degree, recurrent and
    input, over all trials and steps."""
    out_rec = torch.from_numpy((wl.structure["w"] != 0).sum(1)).to(spikes.device, torch.float64)
    out_ff = torch.from_numpy((wl.structure["w_in"] != 0).sum(1)).to(x.device, torch.float64)
    return float(spikes.double().sum(dim=(0, 1)) @ out_rec
                 + (x != 0).double().sum(dim=(0, 1)) @ out_ff)


#: The phases of a forward step the in-kernel timer (``wt_cond_run_timed``) separates,
#: in its order.
PHASE_NAMES = ("loads", "listing", "lookups+update", "slowest wave", "publish+arrival",
               "barrier", "appends", "scan+push")


def phase_split(model, x, T):
    """One more forward of ``model`` under the in-kernel phase timer: microseconds per
    step of each phase (thread 0 of each workgroup, 100 MHz wall clock; averaged over the
    workgroups). Printed to stderr and returned."""
    engine.PHASE_TIMING = []
    try:
        with torch.no_grad():
            model.reset_state()
            model(x)
        torch.cuda.synchronize()
        ticks = engine.PHASE_TIMING[0].double().mean(dim=0).cpu().numpy()
    finally:
        engine.PHASE_TIMING = None
    us = {n: float(v) / 100.0 / T for n, v in zip(PHASE_NAMES, ticks)}
    print("# phases (us per step): " + ", ".join(f"{n} {v:.2f}" for n, v in us.items())
          + f"; total {sum(us.values()):.2f}", file=sys.stderr, flush=True)
    return us


def _part_ms(events):
    return {k: float(np.mean([a.elapsed_time(b) for a, b in v])) for k, v in events.items()}


def _er_cpu_baseline(model, x_np, steps, train):
    """The oracle on the first ``steps`` steps of the same workload (all trials), on a
    CPU copy of the benchmarked network, with this host's threads; and with one thread
    (the reference's test setting, ``tests/conftest.py:12``) on an eighth of those steps."""
    import copy

    import oracle.dynamics as oracle_engine

    engine_module, model._engine = model._engine, None  # (a module does not copy)
    try:
        cpu_model = copy.deepcopy(model).cpu()
    finally:
        model._engine = engine_module
    model = cpu_model
    model._engine = oracle_engine
    B, N = x_np.shape[0], model.n_neurons
    what = "forward + backward" if train else "forward"

    def timed(n):
        x = torch.from_numpy(x_np[:, :n]).float()
        model.reset_state()
        t0 = time.perf_counter()
        if train:
            model.zero_grad(set_to_none=True)
            spikes = model(x)
            dt = float(model.dt)
            target = torch.from_numpy(synthetic.gamma_targets(3, N, max(1, int(n * dt // 20))))
            synthetic.binned_rate_loss(spikes, target, dt).backward()
        else:
            with torch.no_grad():
                model(x)
        elapsed = time.perf_counter() - t0
        return {"value": B * N * n / elapsed, "unit": "neuron-steps/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"oracle {what} of the first {n} of {x_np.shape[1]} steps, all {B} "
                          f"trials ({elapsed:.1f} s)"}

    out = timed(steps)
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        out["one_thread"] = timed(max(1, steps // 8))
    finally:
        torch.set_num_threads(threads)
    return out


def _line(value, ms_per_step, args, dtype, config, roofline, cpu, **extra):
    line = {
        "metric": METRIC, "value": value, "unit": "neuron-steps/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic", **extra, "config": config, "roofline": roofline,
        "cpu_baseline": cpu,
    }  # fmt: skip
    print(json.dumps(line), flush=True)


def bench_config1(args):
    """Configuration 1 (or 0, ``--config 0``: 1,000 neurons, one trial, 1,000 steps — a
    latency-bound case, reported in absolute numbers), forward through the network API."""
    dev = torch.device("cuda:0")
    if args.config == 0:
        T = args.T if args.T != 2000 else 1000
        wl = synthetic.config0(T=T)
    else:
        T = args.T if args.T != 2000 else 5000
        wl = synthetic.config1(T=T)
    model = wl.model.to(dev)
    x = torch.from_numpy(wl.x).float().to(dev)
    B, N = x.shape[0], wl.N
    with torch.no_grad():
        for _ in range(args.warmup):
            model.reset_state()
            model(x)
        torch.cuda.synchronize()
        engine.PART_EVENTS = {}
        t0 = time.perf_counter()
        for _ in range(args.steps):
            model.reset_state()
            spikes = model(x)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    parts, engine.PART_EVENTS = _part_ms(engine.PART_EVENTS), None
    ms_per_step = wall * 1e3 / args.steps
    events = er_events(wl, spikes, x)
    S = wl.S
    bytes_per_launch = algorithmic_bytes(B, T, N, S, events)
    achieved = bytes_per_launch / (parts["forward"] / 1e3) / 1e9
    rate_hz = float(spikes.mean()) / 0.1e-3
    print(f"# config{args.config}: kernel {parts['forward']:.3f} ms, wall {ms_per_step:.3f} ms/step, "
          f"rate {rate_hz:.2f} Hz", file=sys.stderr, flush=True)
    extra = {"phases_us_per_step": phase_split(model, x, T)} if args.phases else {}
    cpu = _er_cpu_baseline(model, wl.x, args.cpu_steps, False) if args.cpu_steps > 0 else None
    _line(B * N * T / (ms_per_step / 1e3), ms_per_step, args, "f32",
          {"workload": ("config1: mid-size conductance-LIF forward" if args.config == 1 else
                        "config0: small conductance-LIF forward (latency-bound)"), "neurons": N,
           "synapses": int((wl.structure["w"] != 0).sum()), "batch": B, "time_steps": T,
           "dt_ms": 0.1, "parallelism": "single GPU"},
          {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "wt_cond_run",
           "kernel_ms": parts["forward"], "algorithmic_bytes_per_launch": bytes_per_launch},
          cpu, synaptic_events_per_s=events / (ms_per_step / 1e3), mean_rate_hz=rate_hz, **extra)


def bench_config3(args):
    dev = torch.device("cuda:0")
    T = args.T if args.T != 2000 else 500
    wl = synthetic.config3(T=T)
    model = wl.model.to(dev)
    model.recurrent_gradients = bool(args.recurrent_gradients)
    x = torch.from_numpy(wl.x).float().to(dev)
    B, N, S = x.shape[0], wl.N, wl.S
    dt = float(model.dt)
    target = torch.from_numpy(synthetic.gamma_targets(3, N, max(1, int(T * dt // 20)))).to(dev)

    def step():
        model.reset_state()
        model.zero_grad(set_to_none=True)
        spikes = model(x)
        synthetic.binned_rate_loss(spikes, target, dt).backward()
        return spikes

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    engine.PART_EVENTS = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        spikes = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    parts, engine.PART_EVENTS = _part_ms(engine.PART_EVENTS), None
    ms_per_step = wall * 1e3 / args.steps
    events = er_events(wl, spikes.detach(), x)
    K = 3  # pathways: recurrent E, recurrent I, input
    n_edges = int((wl.structure["w"] != 0).sum() + (wl.structure["w_in"] != 0).sum())
    # algorithmic bytes: the forward moves the state and saves v, G, held, A; the backward
    # reads what was saved (and the spikes and dL/ds) and writes dL/dA; the weight
    # gradient reads dL/dA of each delivered event's target (and its index) and writes
    # one gradient per synapse; with gradients through the recurrent spikes the backward
    # also reads the recurrent synapses (target and weight) once per step
    n_rec = int((wl.structure["w"] != 0).sum())
    nbytes = {
        "forward": T * (B * N * (8 + 16 * S + 8 + 4 + 4 + 4 * S + 1 + 4 * K) + 24 * N)
                   + 8 * events,
        "backward": T * B * N * (4 + 4 + 4 + 4 * S + 1 + 4 * K + 4 * K)
                    + (T * 8 * n_rec if args.recurrent_gradients else 0),
        "weight_gradient": 8 * events + 4 * n_edges,
    }
    dominant = max(parts, key=parts.get)
    achieved = nbytes[dominant] / (parts[dominant] / 1e3) / 1e9
    rate_hz = float(spikes.detach().mean()) * 1000.0 / dt
    print(f"# config3: wall {ms_per_step:.2f} ms/step; " + ", ".join(
        f"{k} {v:.2f} ms ({nbytes[k] / (v / 1e3) / 1e9:.0f} GB/s)" for k, v in parts.items())
        + f"; rate {rate_hz:.1f} Hz", file=sys.stderr, flush=True)
    cpu = _er_cpu_baseline(model, wl.x, args.cpu_steps, True) if args.cpu_steps > 0 else None
    _line(B * N * T / (ms_per_step / 1e3), ms_per_step, args, "f32",
          {"workload": "config3: conductance-LIF training step (BPTT, surrogate gradient)",
           "neurons": N, "synapses": n_rec, "batch": B,
           "time_steps": T, "dt_ms": dt, "learnt": "per-synapse weights, tau_mem, theta",
           "recurrent_gradients": bool(args.recurrent_gradients),
           "loss": "MSE of 20 ms-binned rates vs gamma(2, 5 Hz) targets",
           "parallelism": "single GPU"},
          {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": achieved / HBM_PEAK_GBS, "traffic": None,
           "kernel": {"forward": "wt_cond_run",
                      "backward": ("wt_cond_recurrent_backward" if args.recurrent_gradients
                                   else "wt_cond_scan_backward"),
                      "weight_gradient": "wt_weight_gradient"}[dominant],
           "kernel_ms": parts[dominant], "algorithmic_bytes_per_launch": nbytes[dominant],
           "per_part_ms": parts},
          cpu, synaptic_events_per_s=events / (ms_per_step / 1e3), mean_rate_hz=rate_hz)


def rate_cpu_baseline(wl, steps):
    """The oracle (the reference's PyTorch rate step restated, float32 as the reference's
    CPU path computes) on forward + backward of the first ``steps`` steps, all trials."""
    import oracle.rate as oracle_rate

    wl_cpu = synthetic.dense_rate(B=wl.x.shape[0], T=steps, storage_dtype=torch.float32)
    model = wl_cpu.model
    model._engine = oracle_rate
    readout = _readout(wl.N, "cpu")
    x = torch.from_numpy(wl.x[:, :steps])
    target = torch.zeros((x.shape[0], steps, readout.shape[1]))
    _rate_step(model, x[:, :2], readout, target[:, :2])  # warm-up
    t0 = time.perf_counter()
    _rate_step(model, x, readout, target)
    dt = time.perf_counter() - t0
    B = x.shape[0]
    return {
        "value": B * wl.N * steps / dt,
        "unit": "neuron-steps/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle (float32) forward + backward of the first {steps} of "
                  f"{wl.x.shape[1]} steps, all {B} trials ({dt:.1f} s)",
    }


def _readout(N, device, n_out=16):
    g = torch.Generator().manual_seed(5)
    return (torch.randn((N, n_out), generator=g) / N**0.5).to(device)


def _rate_step(model, x, readout, target):
    """One training step's forward + backward: rates, a linear read-out, squared error."""
    model.reset_state()
    model.zero_grad(set_to_none=True)
    rates = model(x)
    loss = ((rates @ readout - target) ** 2).mean()
    loss.backward()
    return rates


def bench_config4(args):
    from wiretorch_amd import rate_engine

    dev = torch.device("cuda:0")
    T = args.T if args.T != 2000 else 1000
    wl = synthetic.config4(T=T)
    model = wl.model.to(dev)
    x = torch.from_numpy(wl.x).to(dev)
    B, N = x.shape[0], wl.N
    n_in = x.shape[2]
    readout = _readout(N, dev)
    target = torch.randn((B, T, readout.shape[1]), generator=torch.Generator().manual_seed(6))
    target = target.to(dev)
    for _ in range(args.warmup):
        _rate_step(model, x, readout, target)
    torch.cuda.synchronize()
    rate_engine.LAUNCH_EVENTS = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rates = _rate_step(model, x, readout, target)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    events, rate_engine.LAUNCH_EVENTS = rate_engine.LAUNCH_EVENTS, None
    ms = {k: float(np.mean([a.elapsed_time(b) for a, b in v])) for k, v in events.items()}
    ms_per_step = wall * 1e3 / args.steps
    # algorithmic flops: per time step the recurrent product and the input product forward,
    # the recurrent product's transpose backward; per call the weight gradients
    flops = {
        "forward": 2.0 * B * N * (N + n_in) * T,
        "backward": 2.0 * B * N * N * T,
        "grad_w": 2.0 * B * T * N * (N + n_in),
    }
    # (the recurrent weight gradient runs as three bf16 products of the operands' hi/lo
    # split, wt_split_bf16: its algorithmic flops are those of the one float32 product)
    peak = {"forward": "bf16", "backward": "bf16", "grad_w": "bf16"}
    kernel = {"forward": "rate_step_kernel (wt_rate_forward)",
              "backward": "rate_back_elem_kernel + rate_back_gemm_kernel (wt_rate_backward)",
              "grad_w": "weight-gradient products: wt_split_bf16 + three bf16 GEMMs with "
                        "float32 accumulation (torch.mm / addmm, out_dtype float32)"}
    dominant = max(ms, key=ms.get)
    achieved = flops[dominant] / (ms[dominant] / 1e3) / 1e12
    peak_tf = MFMA_PEAK_TFLOPS[peak[dominant]]
    print(f"# config4: wall {ms_per_step:.2f} ms/step; " + ", ".join(
        f"{k} {ms[k]:.2f} ms ({flops[k] / (ms[k] / 1e3) / 1e12:.0f} TFLOP/s)" for k in ms),
        file=sys.stderr, flush=True)
    mean_rate = float(rates.detach().abs().mean())
    cpu = rate_cpu_baseline(wl, args.cpu_steps) if args.cpu_steps > 0 else None
    line = {
        "metric": METRIC,
        "value": B * N * T / (ms_per_step / 1e3),
        "unit": "neuron-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "tflops": sum(flops.values()) / (ms_per_step / 1e3) / 1e12,
        "mean_abs_rate": mean_rate,
        "config": {
            "workload": "config4: dense rate network, forward + backward",
            "neurons": N, "inputs": n_in, "batch": B, "time_steps": T, "dt_ms": synthetic.RATE_DT,
            "products": "bf16 operands, f32 accumulation; f32 state; weight gradients as "
                        "bf16 hi/lo split products (float32-accurate)",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": peak_tf,
            "unit": "TFLOP/s",
            "frac": achieved / peak_tf,
            "traffic": None,
            "kernel": kernel[dominant],
            "kernel_ms": ms[dominant],
            "algorithmic_flops_per_launch": flops[dominant],
            "per_part_ms": ms,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_filter(args):
    """The spike-train losses' double-exponential filter (forward + backward) on spike
    trains of config 3's training shape: 64 trials x 500 steps x 10,000 neurons."""
    from wiretorch_amd.filtering import VanRossumLoss, double_exponential

    dev = torch.device("cuda:0")
    B, T, N = 64, (args.T if args.T != 2000 else 500), 10_000
    gen = torch.Generator(device=dev).manual_seed(0)
    x = (torch.rand((B, T, N), device=dev, generator=gen) < 0.002).float().requires_grad_(True)
    g = torch.randn((B, T, N), device=dev, generator=gen)
    loss = VanRossumLoss(5.0, 20.0, 0.1, T, device=dev)
    kernels = loss.kernel_rise, loss.kernel_decay
    fwd, bwd = [], []
    for i in range(args.warmup + args.steps):
        if i == args.warmup:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record()
        _, smooth = double_exponential(x, *kernels, None, None)
        e[1].record()
        e[2].record()
        (grad,) = torch.autograd.grad(smooth, x, g)
        e[3].record()
        if i >= args.warmup:
            fwd.append((e[0], e[1]))
            bwd.append((e[2], e[3]))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    parts = _part_ms({"forward": fwd, "backward": bwd})
    ms_per_step = wall * 1e3 / args.steps
    elems = B * T * N
    bytes_fwd, bytes_bwd = 12 * elems, 8 * elems  # x in, rise + smooth out; g in, dL/dx out
    achieved = bytes_fwd / (parts["forward"] / 1e3) / 1e9
    print(f"# filter: forward {parts['forward']:.3f} ms ({achieved:.0f} GB/s), backward "
          f"{parts['backward']:.3f} ms ({bytes_bwd / parts['backward'] / 1e6:.0f} GB/s)",
          file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_steps > 0:
        import oracle.filtering as of

        steps = min(args.cpu_steps, T)
        xs = x.detach()[:, :steps].cpu().numpy()
        gs = g[:, :steps].cpu().numpy()
        a_r, a_d = float(kernels[0][1]), float(kernels[1][1])
        c0 = time.perf_counter()
        of.forward(xs, a_r, a_d)
        of.backward(gs, a_r, a_d)
        elapsed = time.perf_counter() - c0
        cpu = {"value": B * N * steps / elapsed, "unit": "neuron-steps/s", "cores": 1,
               "kind": "port", "sample": f"oracle forward + backward of the first {steps} of "
                                         f"{T} steps, all {B} trials ({elapsed:.1f} s)"}
    _line(elems / (ms_per_step / 1e3), ms_per_step, args, "f32",
          {"workload": "double-exponential spike-train filter, forward + backward",
           "neurons": N, "batch": B, "time_steps": T, "tau_rise_ms": 5.0,
           "tau_decay_ms": 20.0, "dt_ms": 0.1, "parallelism": "single GPU"},
          {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": achieved / HBM_PEAK_GBS,
           "traffic": measured_traffic("wt_filter_config3_shape_traffic.md") if T == 500 else None,
           "kernel": "wt_filter_forward",
           "kernel_ms": parts["forward"], "algorithmic_bytes_per_launch": bytes_fwd},
          cpu, per_part_ms=parts)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-steps", type=int, default=int(os.environ.get("BENCH_CPU_STEPS", 400)))
    ap.add_argument("--T", type=int, default=2000)
    ap.add_argument("--config", type=int, choices=(0, 1, 2, 3, 4), default=2)
    ap.add_argument("--recurrent-gradients", action="store_true",
                    help="configuration 3 with gradients through the recurrent spikes")
    ap.add_argument("--poisson", action="store_true",
                    help="configuration 2 with its input drawn on the device")
    ap.add_argument("--filter", action="store_true",
                    help="measure the spike-train loss filter instead of a configuration")
    ap.add_argument("--phases", action="store_true",
                    help="configurations 0-2: one more forward under the in-kernel phase "
                         "timer, its per-step split reported beside the line")
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
    default_cpu = "--cpu-steps" not in sys.argv and "BENCH_CPU_STEPS" not in os.environ
    if args.filter:
        if default_cpu:
            args.cpu_steps = 500
        return bench_filter(args)
    if args.config == 4:
        if default_cpu:
            args.cpu_steps = 100
        return bench_config4(args)
    if args.config in (0, 1):
        if default_cpu:
            args.cpu_steps = 50 if args.config == 1 else 1000
        return bench_config1(args)
    if args.config == 3:
        if default_cpu:
            args.cpu_steps = 5
        return bench_config3(args)
    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    wl = synthetic.config2(T=args.T, device=dev)
    model = wl.model
    if args.poisson:  # the 10 Hz sensory drive drawn inside the forward (no input tensor)
        from wiretorch_amd.inputs import PoissonInput

        x = PoissonInput(np.full(model.n_inputs, 10.0), 0.1, wl.x.shape[0], wl.x.shape[1],
                         seed=2)
    else:
        x = torch.from_numpy(wl.x).float().to(dev)
    B, T, N, S = x.shape[0], x.shape[1], wl.N, wl.S
    rec, ff = model.rec_projections, model.ff_projections
    print(f"# built config2 through ConductanceLIFNetwork in {time.perf_counter() - t_build:.1f} s: "
          f"N {N}, {model.n_cell_types} cell types, {rec.n_edges} synapses, B {B}, T {T}",
          file=sys.stderr, flush=True)

    def step():
        model.reset_state()
        return model(x)

    with torch.no_grad():
        for _ in range(args.warmup):
            spikes = step()
        torch.cuda.synchronize()
        engine.LAUNCH_EVENTS = []
        t0 = time.perf_counter()
        for _ in range(args.steps):
            spikes = step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        launches = engine.LAUNCH_EVENTS
        engine.LAUNCH_EVENTS = None
    kernel_ms = float(np.mean([a.elapsed_time(b) for a, b in launches]))
    out_rec = (rec.indptr[1:] - rec.indptr[:-1]).double()
    out_ff = (ff.indptr[1:] - ff.indptr[:-1]).double()
    x_dense = x.materialize() if args.poisson else x
    events = float(spikes.double().sum(dim=(0, 1)) @ out_rec
                   + (x_dense != 0).double().sum(dim=(0, 1)) @ out_ff)
    ms_per_step = wall * 1e3 / args.steps
    neuron_steps = B * N * T
    value = neuron_steps / (ms_per_step / 1e3)
    bytes_per_launch = algorithmic_bytes(B, T, N, S, events)
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    rate_hz = float(spikes.mean()) / (0.1e-3)
    print(f"# kernel {kernel_ms:.3f} ms/launch, wall {ms_per_step:.3f} ms/step, "
          f"rate {rate_hz:.2f} Hz, events/step {events / T:.0f}", file=sys.stderr, flush=True)
    x_cpu = x.replay() if args.poisson else wl.x
    cpu = _er_cpu_baseline(model, x_cpu, args.cpu_steps, False) if args.cpu_steps > 0 else None
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
            "neurons": N, "synapses": int(rec.n_edges),
            "cell_types": int(model.n_cell_types), "batch": B, "time_steps": T, "dt_ms": 0.1,
            "built": "ConductanceLIFNetwork, SparseProjection sides",
            "input": ("Poisson drawn on the device (Philox4x32-10)" if args.poisson
                      else "spike tensor resident in HBM"),
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
    if args.phases:
        line["phases_us_per_step"] = phase_split(model, x, T)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
