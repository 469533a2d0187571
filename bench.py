#!/usr/bin/env python3
"""Benchmark of the CompactLogic hot path on one MI355X.

Headline (value): cfg2 training throughput -- 6 x 12000 dense LogicLayers, G = 16, GroupSum
(10, tau 10), batch 1024, fp32, one step = forward + cross-entropy + backward (gradients of
every layer's logits), inputs and parameters resident in HBM.  The step is captured once as
a HIP graph and replayed (``--mode eager`` runs it through Python instead).

Also reported on the same JSON line:
  roofline      the dominant kernel's algorithmic bytes per launch / its average duration,
                timed live with HIP events on the stream it runs on
  cpu_baseline  the pure-PyTorch CPU step (oracle/torch_cpu.py) on a bounded sample
  packed        cfg4: the cfg2 network frozen to argmax gates, 2^24 bit-packed samples,
                layer-by-layer bitwise evaluation + popcount GroupSum, with its own roofline
                and CPU (C oracle) baseline

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
CFG2_BYTES_PER_SAMPLE = 1_398_352
CFG4_BYTES_PER_SAMPLE = 18_138


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--mode", choices=["graph", "eager"], default="graph")
    p.add_argument("--packed-log2-samples", type=int, default=24)
    p.add_argument("--packed-passes", type=int, default=3)
    p.add_argument("--no-packed", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--kernel-reps", type=int, default=20)
    p.add_argument("--kernel-steps", type=int, default=5)
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------------- dense cfg2

def dense_step_fn(model, x, labels, torch):
    def step():
        out = model(x)
        loss = torch.nn.functional.cross_entropy(out, labels)
        loss.backward()
        return loss
    return step


def bench_dense(args, torch):
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    cfg = configs.CONFIGS["cfg2"]
    dev = torch.device("cuda:0")
    model = configs.dense_network(cfg, device=dev)
    x, labels = configs.dense_inputs(cfg, device=dev)
    for m in model:
        if isinstance(m, cl.LogicLayer):
            m.run_plan()
    step = dense_step_fn(model, x, labels, torch)

    if args.mode == "graph":
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                model.zero_grad(set_to_none=True)
                step()
        torch.cuda.current_stream().wait_stream(side)
        model.zero_grad(set_to_none=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    else:
        def run():
            model.zero_grad(set_to_none=True)
            step()
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    grads_run = [p.grad.clone() for p in model.parameters()]
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    samples_s = cfg.batch / dt
    # The timed path must compute what an eager step computes (bitwise: no atomics).
    model.zero_grad(set_to_none=True)
    step()
    torch.cuda.synchronize()
    matches = all(torch.equal(p.grad, g) for p, g in zip(model.parameters(), grads_run))
    kernels = time_dense_kernels(model, step, cfg.batch, args.kernel_steps, torch)
    return cfg, samples_s, dt, kernels, matches


# Algorithmic bytes per launch (activations read once + written once, fp32): forward reads x
# and writes y; the fused backward reads x and grad_y and writes grad_x; the weight gradient
# alone reads x and grad_y.  Parameters, indices and partial moments are not counted.
def algorithmic_bytes(name: str, batch: int) -> int | None:
    import re
    m = re.match(r"(cl_[a-z_]+)\[(\d+)->(\d+)\]", name)
    if not m:
        return None
    kind, i, o = m.group(1), int(m.group(2)), int(m.group(3))
    x, y = 4 * i * batch, 4 * o * batch
    return {"cl_dense_forward_tiled": x + y, "cl_dense_backward_tiled": 2 * x + y,
            "cl_dense_weight_grad": x + y}.get(kind)


def time_dense_kernels(model, step, batch, nsteps, torch):
    """Mean duration of every library call inside `nsteps` real (eager) training steps,
    bracketed with HIP events on the stream each call uses."""
    from compactlogic_amd import timing
    with timing.record() as rec:
        for _ in range(nsteps):
            model.zero_grad(set_to_none=True)
            step()
    out = {}
    for name, v in rec.summary().items():
        sec = v["mean_ms"] * 1e-3
        nbytes = algorithmic_bytes(name, batch)
        out[name] = dict(seconds=sec, calls=v["calls"], algorithmic_bytes=nbytes,
                         achieved_GBs=(nbytes / sec / 1e9) if nbytes else None)
    return out


def cpu_baseline_dense(torch):
    from compactlogic_amd import configs
    from oracle.torch_cpu import CpuDenseNet
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    cfg = configs.CONFIGS["cfg2"]
    batch, warm, steps = 256, 1, 3
    model = configs.dense_network(cfg, device="cpu")
    net = CpuDenseNet.from_model(model)
    x, labels = configs.dense_inputs(cfg, device="cpu", batch=batch)
    for _ in range(warm):
        net.train_step(x, labels)
    t0 = time.perf_counter()
    for _ in range(steps):
        net.train_step(x, labels)
    dt = (time.perf_counter() - t0) / steps
    return {"value": batch / dt, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"cfg2 network (6x12000, G=16, fp32) fwd+bwd in torch CPU autograd "
                      f"(bin_op_s formulation) at batch {batch} of 1024, {warm} warm-up + "
                      f"{steps} timed steps; host {platform.processor() or platform.machine()}, "
                      f"os.cpu_count()={os.cpu_count()}"}


# ---------------------------------------------------------------------------------- packed cfg4

def bench_packed(args, torch):
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    cfg = configs.CONFIGS["cfg2"]
    dev = torch.device("cuda:0")
    model = configs.dense_network(cfg, device=dev)
    configs.freeze_uniform_gates(model)
    n = 1 << args.packed_log2_samples
    words = n // 64
    xw = configs.packed_input_words(cfg.in_dim, words, device=dev)

    def one_pass():
        return model(cl.PackBitsTensor.from_packed(xw))

    counts = one_pass()
    torch.cuda.synchronize()
    times = []
    for _ in range(args.packed_passes):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        counts = one_pass()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    dt = min(times)
    checksum = int(counts.to(torch.int64).sum().item())
    kern = time_packed_kernels(model, xw, args.kernel_reps, torch)
    return dict(n=n, seconds=dt, samples_s=n / dt, checksum=checksum, kernels=kern)


def time_packed_kernels(model, xw, reps, torch):
    import compactlogic_amd as cl
    from compactlogic_amd import _capi
    layers = [m for m in model if isinstance(m, cl.LogicLayer)]
    stream = torch.cuda.current_stream()
    words = xw.shape[1]
    layer = layers[1]
    xin = torch.empty((layer.in_dim, words), dtype=torch.int64, device=xw.device)
    from compactlogic_amd import difflogic_hip as dl
    dl.fill_splitmix64(xin, 77)
    y = torch.empty((layer.out_dim, words), dtype=torch.int64, device=xw.device)
    counts = torch.empty((words * 64, 10), dtype=torch.int32, device=xw.device)
    s = stream.cuda_stream
    ev = lambda: _capi.call("cl_dense_eval_packed", xin.data_ptr(), layer.indices[0].data_ptr(),
                            layer.indices[1].data_ptr(), layer.w.data_ptr(),
                            layer.gate_sequence.data_ptr(), y.data_ptr(), layer.in_dim,
                            layer.out_dim, words * 8, layer.num_gates, s)
    gb = lambda: _capi.call("cl_group_bit_sum", y.data_ptr(), layer.out_dim, words * 8, 0, 10,
                            counts.data_ptr(), s)
    out = {}
    for name, fn, kname, nbytes in (
            ("layer_12000", ev, "k_eval_packed", (layer.in_dim + layer.out_dim) * words * 8),
            ("groupbitsum", gb, "k_group_bit_sum", layer.out_dim * words * 8 + counts.numel() * 4)):
        fn()
        torch.cuda.synchronize()
        r = max(1, reps // 4)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(r):
            fn()
        end.record(stream)
        end.synchronize()
        sec = start.elapsed_time(end) / r * 1e-3
        out[name] = dict(kernel=kname, seconds=sec, algorithmic_bytes=nbytes,
                         achieved_GBs=nbytes / sec / 1e9)
    return out


def cpu_baseline_packed(torch):
    import numpy as np
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    from oracle import packed as P
    cfg = configs.CONFIGS["cfg2"]
    model = configs.dense_network(cfg, device="cpu")
    configs.freeze_uniform_gates(model)
    layers = [P.resolve_slots(m.indices.numpy(), m.gate_sequence.numpy(), m.w.numpy())
              for m in model if isinstance(m, cl.LogicLayer)]
    n = 1 << 16
    words = n // 64
    xw = np.stack([P.fill_splitmix64(words, (1 << 40) + f * words) for f in range(cfg.in_dim)])
    P.network_counts(xw, layers, cfg.k)           # warm
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        P.network_counts(xw, layers, cfg.k)
    dt = (time.perf_counter() - t0) / reps
    return {"value": n / dt / 1e9, "unit": "Gsamples/s", "cores": 1, "kind": "port",
            "sample": f"cfg4 network on 2^16 samples (of 2^24), C oracle oracle/packed_ref.c, "
                      f"single thread, {reps} timed passes"}


def calibration_copy(torch, mib: int = 512):
    """A plain device copy of known size (reads and writes `mib` MiB), run once so that a
    counter profile of this command can scale FETCH_SIZE / WRITE_SIZE against it."""
    src = torch.ones(mib << 18, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


# ---------------------------------------------------------------------------------- main

def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU runs are "
                                   "not part of this build (see DESIGN.md, sharding)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    from compactlogic_amd import _capi
    _capi.load()

    calibration_copy(torch)
    log(f"dense cfg2: mode={args.mode} warmup={args.warmup} steps={args.steps}")
    cfg, samples_s, dt, kernels, matches = bench_dense(args, torch)
    log(f"dense cfg2: {samples_s:,.0f} samples/s, {dt * 1e3:.3f} ms/step")
    # dominant kernel: the library call with the largest total time per step
    dom_name = max((k for k in kernels if kernels[k]["algorithmic_bytes"]),
                   key=lambda k: kernels[k]["seconds"] * kernels[k]["calls"])
    dom = kernels[dom_name]
    roofline = {"bound": "hbm", "achieved": round(dom["achieved_GBs"], 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(dom["achieved_GBs"] / HBM_PEAK_GBS, 4),
                "traffic": None, "kernel": dom_name,
                "per_launch_ms": round(dom["seconds"] * 1e3, 4),
                "algorithmic_bytes_per_launch": dom["algorithmic_bytes"],
                "measured": f"HIP events around each launch inside {args.kernel_steps} eager "
                            "training steps run right after the timed region"}
    step_bytes = CFG2_BYTES_PER_SAMPLE * cfg.batch
    result = {
        "metric": "train samples/s (fwd+bwd) & packed eval Gsamples/s; % of HBM peak",
        "value": round(samples_s, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Bernoulli(0.3) inputs, random-init logits, seeded wiring)",
        "config": {"workload": "cfg2: 6x12000 dense LogicLayer (G=16, one input pair per "
                               "neuron) + GroupSum(10, tau=10), batch 1024, fp32 fwd+CE+bwd",
                   "global_batch": cfg.batch, "mode": args.mode, "parallelism": "none (1 GPU)"},
        "step_hbm_frac": round(step_bytes / dt / 1e9 / HBM_PEAK_GBS, 4),
        "timed_path_matches_eager": matches,
        "roofline": roofline,
        "kernels": {k: {"ms": round(v["seconds"] * 1e3, 4), "calls_per_step": v["calls"] // args.kernel_steps,
                        "GB/s": round(v["achieved_GBs"], 1) if v["achieved_GBs"] else None}
                    for k, v in kernels.items()},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline (dense)")
        result["cpu_baseline"] = cpu_baseline_dense(torch)
    if not args.no_packed:
        log(f"packed cfg4: 2^{args.packed_log2_samples} samples x {args.packed_passes} passes")
        pk = bench_packed(args, torch)
        pk_dom = pk["kernels"]["layer_12000"]
        packed = {
            "workload": f"cfg4: cfg2 network frozen to argmax gates, 2^{args.packed_log2_samples} "
                        "samples bit-packed 64 per word, 6 bitwise layers + popcount GroupSum",
            "value": round(pk["samples_s"] / 1e9, 4), "unit": "Gsamples/s",
            "ms_per_pass": round(pk["seconds"] * 1e3, 3),
            "hbm_frac": round(CFG4_BYTES_PER_SAMPLE * pk["samples_s"] / 1e9 / HBM_PEAK_GBS, 4),
            "counts_checksum": pk["checksum"],
            "roofline": {"bound": "hbm", "achieved": round(pk_dom["achieved_GBs"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pk_dom["achieved_GBs"] / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": pk_dom["kernel"], "per_launch_ms": round(pk_dom["seconds"] * 1e3, 3),
                         "algorithmic_bytes_per_launch": pk_dom["algorithmic_bytes"]},
            "kernels": {k: {"ms": round(v["seconds"] * 1e3, 3), "GB/s": round(v["achieved_GBs"], 1)}
                        for k, v in pk["kernels"].items()},
        }
        log(f"packed cfg4: {packed['value']} Gsamples/s")
        if not args.no_cpu_baseline:
            log("cpu baseline (packed)")
            packed["cpu_baseline"] = cpu_baseline_packed(torch)
        result["packed"] = packed
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
