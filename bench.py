#!/usr/bin/env python3
"""Benchmark of the fp32 GRU training step (forward + backward) on one MI355X.

Workload = BASELINE config 2: 1-layer GRU, input 256, hidden 256, batch 64,
seq_len 512, fp32; x ~ N(0,1), PyTorch-uniform init, h0 ~ 0.1 N(0,1), MSE loss
against an N(0,1) target; a step is forward + loss + backward producing the
gradients of all four weight/bias tensors, x and h0 (no optimizer, as the
reference's published fwd+bwd numbers).  The MSE loss is the library's
(rnn_kernel_amd.mse_loss, the same mean squared error as F.mse_loss); the
torch.nn.GRU baselines use F.mse_loss.  Inputs are generated on the CPU with
seed 42, copied to the GPU, and resident in HBM before timing starts.

Timing protocol (the reference's, rnn_benchmark.py:642-694): W untimed
warm-up steps, then K timed steps bracketed by torch.cuda.synchronize();
ms_per_step is the wall-clock elapsed time over the K steps divided by K
(time.perf_counter), as the reference's run_case reports it.  An event is
also recorded on the stream after every step; the median of those K
per-step intervals is reported beside it (event_median_ms_per_step).

Prints ONE JSON line (rank 0).  Besides the contract fields it carries:
  roofline      - the dominant kernel (the slower recurrence): achieved rate
                  from the library's own per-stage hipEvents on the launch
                  stream over a separate pass of K steps, against the fp32
                  peak and, as a latency-bound kernel, against the measured
                  floor of its step structure;
  cpu_baseline  - torch.nn.GRU fp32 on this host's CPU cores (the
                  reference's CPU path), full workload, 1 warm-up + 5 timed
                  steps, median; thread count, CPU model and MKL / oneDNN
                  versions recorded;
  cpu_oracle_port - the C oracle (fp32, one thread), bounded sample;
  torch_gru_gpu - torch.nn.GRU (MIOpen/rocBLAS) on the same GPU, same protocol.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "fp32 GRU fwd+bwd timesteps/sec & µs/step, H=256 B=64 T=512, 1 MI355X"
B, T, I, H, L = 64, 512, 256, 256, 1
SEED = 42
MFMA_FP32_PEAK_TFLOPS = 157.3
# The recurrences' FMAs are non-packed v_fmac_f32 (this build disables packed
# fp32); the published 157.3 TFLOP/s vector figure assumes packed FMAs.  Their
# roof is measured in each run (rka_measure_fma_rate: every CU issuing
# independent FMA chains), and valu_frac and the step floor use that rate.
HBM_PEAK_GBS = 8000.0
RECURRENCES = ("forward_recurrence", "backward_recurrence")
CPU_THREAD_CAP = 16  # the GPU box's CPU share for one GPU, whatever os.cpu_count() reports


def flops_per_step(B, T, I, H):
    # 2*B*T*3H*(I+H) forward + backward (dh, dW_hh, dx, dW_ih): 18*B*T*H*(I+H).
    return 18.0 * B * T * H * (I + H)


def stage_flops(B, T, I, H):
    return {
        "input_gemm": 2.0 * B * T * 3 * H * I,
        "forward_recurrence": 2.0 * B * T * 3 * H * H,
        "backward_recurrence": 2.0 * B * T * 3 * H * H,
        "dw_gemm": 2.0 * B * T * 3 * H * (H + I),
        "dw_reduce": 0.0,
        "dx_gemm": 2.0 * B * T * 3 * H * I,
    }


def stage_bytes(B, T, I, H):
    """Algorithmic HBM bytes per launch of the recurrence kernels: every input
    read once, every output written once (fp32)."""
    return {
        # gx, W_hh, b_hh, h0 in; y, reserve (r, z, n, W_hn h + b_hn), hn out
        "forward_recurrence": 4.0 * (B * T * 3 * H + 3 * H * H + 3 * H + B * H + B * T * H + B * T * 4 * H + B * H),
        # dy, reserve, y (h_{t-1}), W_hh, h0 in; G = (da_n, dr, dz, dn), dh0 out
        "backward_recurrence": 4.0 * (B * T * H + B * T * 4 * H + B * T * H + 3 * H * H + B * H + B * T * 4 * H + B * H),
    }


TRAFFIC_FILE = os.path.join(REPO, "profiles", "gru_c2_recurrence_hbm_traffic.txt")


def measured_traffic(stage):
    """HBM bytes per launch of `stage` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (copy-calibrated), or None if it has no such line."""
    try:
        for line in open(TRAFFIC_FILE):
            f = line.split()
            if len(f) == 3 and f[0] == "traffic_bytes_per_launch" and f[1] == stage:
                return int(f[2])
    except OSError:
        pass
    return None


def make_inputs():
    import torch

    torch.manual_seed(SEED)
    gru = torch.nn.GRU(I, H, num_layers=L, batch_first=True)  # PyTorch-uniform init
    x = torch.randn(B, T, I)
    h0 = 0.1 * torch.randn(L, B, H)
    target = torch.randn(B, T, H)
    return gru, x, h0, target


def time_steps(model, x, h0, target, steps, warmup, sync, profile_cb=None, loss_fn=None):
    """(wall-clock mean seconds per step, median per-step seconds from
    stream events) of `steps` timed steps after `warmup` untimed ones."""
    import torch
    import torch.nn.functional as F

    loss_fn = loss_fn or F.mse_loss

    def step():
        for p in model.parameters():
            p.grad = None
        x.grad = None
        h0.grad = None
        out, hn = model(x, h0)
        loss = loss_fn(out, target)
        loss.backward()

    for _ in range(warmup):
        step()
    sync()
    if profile_cb:
        profile_cb(True)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    events[0].record()
    for i in range(steps):
        step()
        events[i + 1].record()
    sync()
    elapsed = time.perf_counter() - t0
    per_step = [events[i].elapsed_time(events[i + 1]) * 1e-3 for i in range(steps)]
    return elapsed / steps, statistics.median(per_step)


# The other BASELINE configs, measured with `--workload` (the default run is c2
# and keeps the one-line contract above; these print one JSON line each too).
OTHER_WORKLOADS = {
    # hidden sweep, I = H, B = 64, T = 512
    "c3": [dict(L=1, I=h, H=h, B=64, T=512, h0_scale=0.1) for h in (64, 96, 128, 129, 130, 160, 192)],
    # two stacked layers
    "c4": [dict(L=2, I=256, H=256, B=256, T=1024, h0_scale=0.1)],
    # 8 chunks of 512 carrying h without detach (gradients flow through all chunks)
    "c5": [dict(L=1, I=128, H=256, B=16, T=4096, h0_scale=0.5, chunks=8, saturate=True)],
    # the same with the carried state detached (truncated BPTT: a backward per chunk)
    "c5-detached": [dict(L=1, I=128, H=256, B=16, T=4096, h0_scale=0.5, chunks=8, saturate=True, detach=True)],
    # c2 forward only, no autograd (the inference path: no gate cache)
    "infer": [dict(L=1, I=256, H=256, B=64, T=512, h0_scale=0.1, infer=True)],
}


def workload_inputs(w):
    import torch

    torch.manual_seed(SEED)
    gru = torch.nn.GRU(w["I"], w["H"], num_layers=w["L"], batch_first=True)
    x = torch.randn(w["B"], w["T"], w["I"])
    if w.get("saturate"):
        # 5 % of the [B, T] rows of x scaled x10 (gate saturation)
        g = torch.Generator().manual_seed(SEED + 1)
        mask = torch.rand(w["B"], w["T"], generator=g) < 0.05
        x = torch.where(mask[..., None], x * 10.0, x)
    h0 = w["h0_scale"] * torch.randn(w["L"], w["B"], w["H"])
    target = torch.randn(w["B"], w["T"], w["H"])
    return gru, x, h0, target


def time_workload(model, w, x, h0, target, steps, warmup, sync, loss_fn):
    """Mean seconds of one step of workload w: forward over the chunks, MSE
    loss and backward (per chunk when the carried state is detached), or the
    forward alone without autograd for the inference workload."""
    import torch

    chunks = w.get("chunks", 1)

    def step():
        if w.get("infer"):
            with torch.no_grad():
                model(x, h0)
            return
        for p in model.parameters():
            p.grad = None
        x.grad = None
        h0.grad = None
        if chunks == 1:
            out, _ = model(x, h0)
            loss_fn(out, target).backward()
            return
        hidden = h0
        outs = []
        for xc, tc in zip(x.chunk(chunks, dim=1), target.chunk(chunks, dim=1)):
            if w.get("detach"):
                out, hidden = model(xc, hidden.detach())
                loss_fn(out, tc).backward()
            else:
                out, hidden = model(xc, hidden)
                outs.append(out)
        if outs:
            loss_fn(torch.cat(outs, dim=1), target).backward()

    for _ in range(warmup):
        step()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    sync()
    return (time.perf_counter() - t0) / steps


def run_other_workload(name, args):
    import torch
    import torch.nn.functional as F

    from rnn_kernel_amd import from_torch_gru, mse_loss

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    sync = torch.cuda.synchronize
    rows = []
    for w in OTHER_WORKLOADS[name]:
        gru, x_cpu, h0_cpu, target_cpu = workload_inputs(w)
        grad = not w.get("infer")
        x = x_cpu.to(dev).requires_grad_(grad)
        h0 = h0_cpu.to(dev).requires_grad_(grad)
        target = target_cpu.to(dev)
        gru = gru.to(dev)
        ours = from_torch_gru(gru)
        t_ours = time_workload(ours, w, x, h0, target, args.steps, args.warmup, sync, mse_loss)
        row = {k: w[k] for k in ("L", "I", "H", "B", "T")}
        row.update({"ms_per_step": t_ours * 1e3, "timesteps_per_s": w["T"] / t_ours,
                    "us_per_timestep": t_ours * 1e6 / w["T"], "tokens_per_s": w["B"] * w["T"] / t_ours})
        if not args.skip_torch_gpu:
            gru.flatten_parameters()
            t_torch = time_workload(gru, w, x, h0, target, max(3, args.steps // 2), 2, sync, F.mse_loss)
            row["torch_gru_gpu_ms_per_step"] = t_torch * 1e3
            row["speedup_of_ours"] = t_torch / t_ours
        rows.append(row)
        del ours, gru, x, h0, target
        torch.cuda.empty_cache()
    first = OTHER_WORKLOADS[name][0]
    kind = "forward only, no autograd" if first.get("infer") else "fwd+bwd, MSE loss, no optimizer"
    if first.get("chunks"):
        kind += f", {first['chunks']} chunks carrying h" + (" (detached)" if first.get("detach") else "")
    result = {
        "metric": f"fp32 GRU {kind}: timesteps/s and µs/timestep, 1 MI355X",
        "workload": name,
        "unit": "timesteps/s",
        "value": rows[0]["timesteps_per_s"] if len(rows) == 1 else None,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "dtype": "fp32",
        "data": "synthetic (seed 42, CPU-generated, PyTorch-uniform init)",
        "results": rows,
    }
    print(json.dumps(result), flush=True)


def cpu_identity():
    """CPU model, logical CPUs and the BLAS / oneDNN builds torch uses."""
    import torch

    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    cfg = torch.__config__.show()
    mkl = next((ln.strip() for ln in cfg.splitlines() if "Math Kernel Library" in ln or "oneMKL" in ln), None)
    onednn = next((ln.strip() for ln in cfg.splitlines() if "oneDNN" in ln or "MKL-DNN" in ln), None)
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "mkl": mkl, "onednn": onednn,
            "torch": torch.__version__}


def torch_cpu_baseline(runs: int = 5):
    """torch.nn.GRU fp32 fwd+bwd (MSE loss) on the host CPU at the full c2
    workload: 1 warm-up + `runs` timed runs with time.perf_counter, median
    (rnn_benchmark.py:674-694)."""
    import torch
    import torch.nn.functional as F

    threads = min(os.cpu_count() or 1, CPU_THREAD_CAP)
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        gru, x, h0, target = make_inputs()
        times = []
        for i in range(runs + 1):
            xs = x.clone().requires_grad_(True)
            hs = h0.clone().requires_grad_(True)
            gru.zero_grad(set_to_none=True)
            t0 = time.perf_counter()
            out, _ = gru(xs, hs)
            F.mse_loss(out, target).backward()
            dt = time.perf_counter() - t0
            if i > 0:
                times.append(dt)
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(times)
    return {
        "value": T / med,
        "unit": "timesteps/s",
        "cores": threads,
        "kind": "reference",
        "ms_per_step": med * 1e3,
        "runs_ms": [round(t * 1e3, 2) for t in times],
        "sample": (f"torch.nn.GRU fp32 fwd+bwd + MSE on the host CPU, full workload B={B} T={T} I={I} H={H}, "
                   f"1 warm-up + {runs} timed runs, median; {threads} threads (the box's CPU share for one GPU "
                   f"is {CPU_THREAD_CAP}, whatever os.cpu_count() reports)"),
        "host": cpu_identity(),
    }


def cpu_oracle_baseline(budget_s: float):
    """C oracle (fp32, single thread) on the c2 shape with fewer timesteps."""
    import numpy as np
    from oracle import gru_oracle

    gru_oracle.build()
    gru, x, h0, target = make_inputs()
    p = {n: getattr(gru, f"{n}_l0").detach().numpy() for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh")}
    t_sample = 8
    while True:
        xs = x[:, :t_sample].numpy()
        t0 = time.perf_counter()
        f = gru_oracle.forward(xs, h0[0].numpy(), p["weight_ih"], p["weight_hh"], p["bias_ih"], p["bias_hh"],
                               dtype=np.float32)
        dy = (2.0 / (B * t_sample * H)) * (f.y - target[:, :t_sample].numpy())
        gru_oracle.backward(xs, h0[0].numpy(), p["weight_ih"], p["weight_hh"], f.y, f.cache, dy, None,
                            dtype=np.float32)
        dt = time.perf_counter() - t0
        # grow the sample (x4 timesteps) while the next one stays within the budget
        if dt * 4 > budget_s or t_sample >= T:
            break
        t_sample = min(T, t_sample * 4)
    return {
        "value": t_sample / dt,
        "unit": "timesteps/s",
        "cores": 1,
        "kind": "port",
        "sample": f"C oracle fp32 fwd+bwd, B={B} I={I} H={H}, T={t_sample} of {T} timesteps, {dt:.2f} s",
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--cpu-budget", type=float, default=20.0,
                        help="upper bound (s) of the C oracle's sample; samples grow x4 in timesteps while "
                             "the next one fits")
    parser.add_argument("--skip-cpu", action="store_true")
    parser.add_argument("--skip-torch-gpu", action="store_true")
    parser.add_argument("--workload", default="c2", choices=["c2"] + sorted(OTHER_WORKLOADS),
                        help="c2 (default): the headline line; the others measure the remaining BASELINE configs "
                             "and the inference path, ours and torch.nn.GRU on the same GPU")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the path is single-GPU "
              "and its data-parallel sharding is a design note, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    if args.workload != "c2":
        run_other_workload(args.workload, args)
        return

    import torch

    from rnn_kernel_amd import _lib, check_recurrences, from_torch_gru, mse_loss

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    sync = torch.cuda.synchronize

    gru, x_cpu, h0_cpu, target_cpu = make_inputs()
    x = x_cpu.to(dev).requires_grad_(True)
    h0 = h0_cpu.to(dev).requires_grad_(True)
    target = target_cpu.to(dev)
    ours = from_torch_gru(gru.to(dev))

    # pass 1: per-stage library events (roofline and stage split)
    _lib.profile_read()  # clear
    time_steps(ours, x, h0, target, args.steps, args.warmup, sync, profile_cb=_lib.profile_enable, loss_fn=mse_loss)
    stages = _lib.profile_read()
    _lib.profile_enable(False)
    # pass 2, the headline: no stage events, one event per step boundary
    t_step, t_event_median = time_steps(ours, x, h0, target, args.steps, 2, sync, loss_fn=mse_loss)
    check_recurrences()  # raises if a recurrence call aborted

    # the exchange the recurrences step with, measured live: 128 workgroup
    # pairs (every CU busy), eight polling wavefronts each
    exch = _lib.measure_exchange_latency(pairs=128, iters=2000)
    # the non-packed fp32 FMA issue rate, measured live on every CU
    fma = _lib.measure_fma_rate()
    valu_peak = fma["tflops"]

    # per-step stage totals; a stage may run as several launches per step
    # (the backward recurrence in time chunks), and side-stream GEMM stages
    # overlap the recurrence, so the stages can sum to more than the step
    flops = stage_flops(B, T, I, H)
    stage_step = {k: ms / args.steps for k, (ms, n) in stages.items()}
    launches = {k: n / args.steps for k, (ms, n) in stages.items()}
    dominant = max(stage_step, key=stage_step.get)
    per_launch = max(launches[dominant], 1.0)
    dom_ms = stage_step[dominant] / per_launch           # mean launch duration
    achieved = flops[dominant] / per_launch / (dom_ms * 1e-3) / 1e12 if dom_ms > 0 else 0.0
    # the step floor of a recurrence: one exchange one way, then the FMAs of
    # the other slices' W_hh columns (H - 64 of the H per gate row and batch
    # row; 64 units per workgroup) at the measured FMA rate over the whole GPU
    remote_flops = 2.0 * B * 3 * H * max(H - 64, 0)
    floor_us = exch["round_trip_ns"] / 2 * 1e-3 + remote_flops / (valu_peak * 1e12) * 1e6
    alg_bytes = stage_bytes(B, T, I, H).get(dominant)
    if alg_bytes:
        alg_bytes /= per_launch

    result = {
        "metric": METRIC,
        "value": T / t_step,
        "unit": "timesteps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_step * 1e3,
        "event_median_ms_per_step": t_event_median * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seed 42, CPU-generated, PyTorch-uniform init)",
        "config": {"workload": "BASELINE config 2: 1-layer GRU fwd+bwd, MSE loss, no optimizer",
                   "batch": B, "seq_len": T, "input_size": I, "hidden_size": H, "layers": L},
        "us_per_timestep": t_step * 1e6 / T,
        "tokens_per_s": B * T / t_step,
        "step_tflops": flops_per_step(B, T, I, H) / t_step / 1e12,
        "stages_ms": {k: round(v, 4) for k, v in stage_step.items()},
        "recurrence_us_per_timestep": {"forward": stage_step.get("forward_recurrence", 0.0) * 1e3 / T,
                                       "backward": stage_step.get("backward_recurrence", 0.0) * 1e3 / T},
        "launches_per_step": {k: round(v, 2) for k, v in launches.items()},
        "roofline": {
            "kernel": dominant,
            "bound": "latency" if dominant in RECURRENCES else "mfma",
            "achieved": achieved,
            "peak": MFMA_FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_FP32_PEAK_TFLOPS,
            "traffic": measured_traffic(dominant),
            "note": ("serial recurrence: VALU FMAs (no MFMA) between one cross-workgroup exchange per timestep, "
                     "latency-bound; achieved = algorithmic FLOPs / mean launch time from hipEvents on the launch "
                     "stream; frac against the published fp32 peak, valu_frac against the non-packed fp32 FMA "
                     "issue rate measured in this run; floor = one exchange (half the measured ping-pong round trip) + the FMAs that need "
                     "the exchanged values (the other slices' share of W_hh h) at that FMA rate, both measured or "
                     "computed in this run; floor_frac = floor / measured step; traffic = copy-calibrated "
                     "FETCH_SIZE+WRITE_SIZE bytes per launch from the committed rocprofv3 summary"),
            "valu_peak": valu_peak,
            "valu_frac": achieved / valu_peak,
            "fma_ns_per_instruction_per_simd": fma["ns_per_instruction"],
            "exchange_round_trip_ns": exch["round_trip_ns"],
            "exchange_pairs_on_one_xcd": exch["same_xcd"],
            "floor_us_per_timestep": floor_us,
            "floor_frac": (floor_us / (stage_step[dominant] * 1e3 / T / per_launch))
            if dominant in RECURRENCES else None,
            "us_per_timestep": stage_step[dominant] * 1e3 / T,
            "launch_ms": dom_ms,
            "launches_per_step": per_launch,
            "alg_bytes": alg_bytes,
            "hbm_frac": (alg_bytes / (dom_ms * 1e-3) / 1e9 / HBM_PEAK_GBS) if (alg_bytes and dom_ms > 0) else None,
        },
    }

    if not args.skip_torch_gpu:
        gru_gpu = gru.to(dev)
        gru_gpu.flatten_parameters()
        x.grad = None
        t_torch, _ = time_steps(gru_gpu, x, h0, target, max(3, args.steps // 2), 2, sync)
        result["torch_gru_gpu"] = {"value": T / t_torch, "unit": "timesteps/s", "ms_per_step": t_torch * 1e3,
                                   "speedup_of_ours": t_torch / t_step}
    if not args.skip_cpu:
        result["cpu_baseline"] = torch_cpu_baseline()
        result["cpu_oracle_port"] = cpu_oracle_baseline(args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
