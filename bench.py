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
  train_full    cfg2 with the optimizer half of the reference's step: clip_grad_norm_(10) and
                Adam fused (FusedAdam), the whole step in one HIP graph
  train_random_wiring  cfg2 with the reference's default connections='random' (a pair per
                slot: the multi-run kernels)
  conv_train    cfg3: conv 9x32x32 -> 256x16x16 -> 512x7x7, flatten, 2 x 16000 dense,
                GroupSum(10, tau 30), batch 256, fp32 fwd + CE + bwd, same measurements
  conv_tree_train  the logic-tree reading of cfg3: two complete ConvLogicLayer blocks (8 taps,
                4 -> 2 -> 1 gates, 2x2 max pool) -> 512x2x2, flatten, 2 x 16000 dense, same step
  packed        cfg4: the cfg2 network frozen to argmax gates, 2^24 bit-packed samples,
                layer-by-layer bitwise evaluation + popcount GroupSum, with its own roofline
                and CPU (C oracle) baseline
  packed_conv   cfg5: the cfg3 network with 4 candidate gates per row, frozen, 2^20
                bit-packed samples; its "fused" member writes conv2's output column-major and
                runs the two dense layers and the counts in one launch
  packed_conv_tree  the cfg3_tree network frozen to argmax gates (pool = OR), 2^20 bit-packed
                samples; its "fused" member runs the two dense layers and the counts in one
                launch after the conv blocks

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
CFG3_BYTES_PER_SAMPLE = 2_462_288
CFG3_TREE_BYTES_PER_SAMPLE = 1_018_448
CFG5_TREE_BYTES_PER_SAMPLE = 13_800
CFG4_BYTES_PER_SAMPLE = 18_138
CFG5_BYTES_PER_SAMPLE = 31_848


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--mode", choices=["graph", "eager"], default="graph")
    p.add_argument("--packed-log2-samples", type=int, default=24)
    p.add_argument("--packed-passes", type=int, default=3)
    p.add_argument("--no-packed", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--kernel-reps", type=int, default=20)
    p.add_argument("--kernel-steps", type=int, default=5)
    p.add_argument("--no-conv", action="store_true")
    p.add_argument("--conv-steps", type=int, default=100)
    p.add_argument("--conv-warmup", type=int, default=50)
    p.add_argument("--conv-packed-log2-samples", type=int, default=20)
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------------- dense cfg2

def dense_step_fn(model, x, labels, torch):
    """One training step: the network, the mean cross-entropy of GroupSum's scores (fused into
    GroupSum's kernels: GroupSum.cross_entropy is cross_entropy(GroupSum(x), labels)), and the
    backward into every layer's logits.  The timed steps are replayed HIP graphs, which take
    this composition (the fused classifier head, sequential_cross_entropy, is not captured),
    so the eager steps timed per kernel take it too."""
    body, head = model[:-1], model[-1]
    one = torch.ones((), dtype=torch.float32, device=x.device)  # d loss / d loss, made once

    def step():
        loss = head.cross_entropy(body(x), labels)
        loss.backward(one)
        return loss
    return step


def bench_train(model, x, labels, steps, warmup, mode, kernel_steps, torch):
    """Time `steps` training steps (forward, cross-entropy, backward into every layer's logits)
    after `warmup`; returns (samples/s, s/step, per-kernel timings, timed == eager)."""
    import compactlogic_amd as cl
    for m in model:
        if isinstance(m, cl.LogicLayer) and not isinstance(m, cl.ConvLayer):
            m.run_plan()
    step = dense_step_fn(model, x, labels, torch)
    if mode == "graph":
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
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    grads_run = [p.grad.clone() for p in model.parameters()]
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    batch = x.shape[0]
    # The timed path must compute what an eager step computes (bitwise: no atomics).
    model.zero_grad(set_to_none=True)
    step()
    torch.cuda.synchronize()
    matches = all(torch.equal(p.grad, g) for p, g in zip(model.parameters(), grads_run))
    kernels = time_train_kernels(model, step, batch, kernel_steps, torch)
    return batch / dt, dt, kernels, matches


def bench_dense(args, torch):
    from compactlogic_amd import configs
    cfg = configs.CONFIGS["cfg2"]
    dev = torch.device("cuda:0")
    model = configs.dense_network(cfg, device=dev)
    x, labels = configs.dense_inputs(cfg, device=dev)
    samples_s, dt, kernels, matches = bench_train(model, x, labels, args.steps, args.warmup,
                                                  args.mode, args.kernel_steps, torch)
    del model
    torch.cuda.empty_cache()
    return cfg, samples_s, dt, kernels, matches


def bench_dense_random(args, torch):
    """cfg2 with the reference's default wiring (connections='random', compactlogic/
    compactlogic.py:160-182): every slot of a neuron reads its own input pair, so a neuron is
    16 runs and the layer takes the multi-run kernels (prep, tiled forward, chunked backward
    with its finalize) instead of the single-run fused forward and row backward."""
    from compactlogic_amd import configs
    cfg = configs.CONFIGS["cfg2"]
    dev = torch.device("cuda:0")
    model = configs.dense_network(cfg, device=dev, wiring="random")
    x, labels = configs.dense_inputs(cfg, device=dev)
    samples_s, dt, kernels, matches = bench_train(model, x, labels, args.steps, args.warmup,
                                                  args.mode, args.kernel_steps, torch)
    del model
    torch.cuda.empty_cache()
    return {"workload": "cfg2 (6x12000, G=16, B=1024, fp32 fwd+CE+bwd) with connections='random': "
                        "16 input pairs per neuron, the multi-run kernels",
            "value": round(samples_s, 1), "unit": "samples/s", "ms_per_step": round(dt * 1e3, 4),
            "steps": args.steps, "timed_path_matches_eager": matches,
            "kernels": kernels_json(kernels, args.kernel_steps)}


# Algorithmic bytes per launch (activations read once + written once, fp32): a forward reads
# its input and writes its output; the dense fused backward and the conv input gradient read
# the input and grad_y and write grad_x; a weight gradient alone reads the input and grad_y.
# Parameters, indices and partial sums are not counted.
def bench_train_full(args, torch):
    """cfg2 with the optimizer half of the reference's training step
    (experiments/experiment_script.py:280-293): forward, the fused GroupSum cross-entropy,
    backward, clip_grad_norm_(10.0) and Adam(lr 0.01) fused (FusedAdam), the whole step
    captured in one HIP graph."""
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    cfg = configs.CONFIGS["cfg2"]
    dev = torch.device("cuda:0")
    model = configs.dense_network(cfg, device=dev)
    x, labels = configs.dense_inputs(cfg, device=dev)
    opt = cl.FusedAdam(model.parameters(), lr=0.01, max_norm=10.0)
    body, head = model[:-1], model[-1]

    def step():
        loss = head.cross_entropy(body(x), labels)
        loss.backward()
        opt.step()

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
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    nparams = sum(p.numel() for p in model.parameters())
    del model, opt, graph
    torch.cuda.empty_cache()
    return {"workload": "cfg2 full training step: fwd + fused CE + bwd + clip_grad_norm_(10) + "
                        "Adam(lr 0.01), one HIP graph",
            "value": round(x.shape[0] / dt, 1), "unit": "samples/s",
            "ms_per_step": round(dt * 1e3, 4), "steps": args.steps, "parameters": nparams}


def train_kernel_bytes(model, batch: int) -> dict:
    import compactlogic_amd as cl
    out = {}
    first = True
    prev_out = 0
    k_out = next((mm.k for mm in model if isinstance(mm, cl.GroupSum)), 0)
    for m in model:
        if isinstance(m, cl.ConvLogicLayer):
            # complete block: forward reads x, writes the pooled y; backward reads x and
            # grad_y and writes grad_x (not for the first module, whose input needs no gradient)
            c, h, w = m._last_shape
            tag = f"[{c}x{h}x{w}->{m.out_channels}]"
            xb = 4 * batch * c * h * w
            ho = (h + 2 * m.padding[0] - m.kernel[0]) // m.stride[0] + 1
            wo = (w + 2 * m.padding[1] - m.kernel[1]) // m.stride[1] + 1
            yb = 4 * batch * m.out_channels * (ho // 2) * (wo // 2)
            out.update({"cl_tree_conv_forward" + tag: xb + yb,
                        "cl_tree_conv_backward" + tag: (xb + yb) if first else (2 * xb + yb)})
        elif isinstance(m, cl.ConvLayer):
            c, h, w = m.in_shape
            tag = f"[{c}x{h}x{w}->{m.c_out}]"
            xb = 4 * batch * c * h * w
            yb = 4 * batch * m.c_out * m.h_out * m.w_out
            out.update({"cl_conv_forward" + tag: xb + yb, "cl_conv_backward_x" + tag: 2 * xb + yb,
                        "cl_conv_backward_w" + tag: xb + yb,
                        "cl_conv_window_forward" + tag: xb + yb,
                        "cl_conv_window_backward_x" + tag: 2 * xb + yb,
                        "cl_conv_window_moments" + tag: xb + yb})
        elif isinstance(m, cl.LogicLayer):
            tag = f"[{m.in_dim}->{m.out_dim}]"
            xb, yb = 4 * batch * m.in_dim, 4 * batch * m.out_dim
            out.update({"cl_dense_forward_tiled" + tag: xb + yb,
                        "cl_dense_forward_fused" + tag: xb + yb,
                        "cl_dense_backward_tiled" + tag: 2 * xb + yb,
                        "cl_dense_backward_rows" + tag: 2 * xb + yb,
                        "cl_dense_backward_part" + tag: 2 * xb + yb,
                        "cl_dense_weight_grad" + tag: xb + yb})
            # as the classifier head with GroupSum's cross-entropy: the forward reads x (and
            # writes scores and softmax, [batch, k] each), the backward reads x, writes grad_x
            out["cl_dense_group_sum_cross_entropy_forward" + tag] = xb + 8 * batch * k_out
            out["cl_dense_group_sum_cross_entropy_backward" + tag] = 2 * xb
            # layout change of a [batch, in_dim] input and of its gradient: read + write
            out[f"cl_transpose[{batch}x{m.in_dim}]"] = 2 * xb
            out[f"cl_transpose[{m.in_dim}x{batch}]"] = 2 * xb
            prev_out = m.out_dim
        elif isinstance(m, cl.GroupSum) and prev_out:
            # unfused cross-entropy: the forward reads the last layer's output, the backward
            # writes its gradient (scores and softmax, [batch, k] each, besides)
            fb = 4 * batch * prev_out
            out["cl_group_sum_cross_entropy_forward"] = fb + 8 * batch * m.k
            out["cl_group_sum_cross_entropy_backward"] = fb
        if not isinstance(m, torch_flatten_types()):
            first = False
    return out


def torch_flatten_types():
    import torch
    return (torch.nn.Flatten,)


def packed_kernel_bytes(model, words: int, k: int) -> dict:
    """Packed eval: read the input rows once, write the output rows once (8 bytes per word);
    GroupSum reads the last rows and writes int32 counts [samples, k]."""
    import compactlogic_amd as cl
    from compactlogic_amd.treelogic import tree_row_bytes
    out = {}
    rows = None
    for m in model:
        if isinstance(m, cl.ConvLogicLayer):
            c, h, w = m._last_shape
            ho = (h + 2 * m.padding[0] - m.kernel[0]) // m.stride[0] + 1
            wo = (w + 2 * m.padding[1] - m.kernel[1]) // m.stride[1] + 1
            fin, fout = c * h * w, m.out_channels * (ho // 2) * (wo // 2)
            out[f"cl_tree_conv_eval_packed[{fin}->{fout}]"] = (fin + fout) * words * 8
            if rows is None and tree_row_bytes(words * 8) != words * 8:
                # the first block widens power-of-two rows once (read + write of its input)
                out[f"widen_rows[{fin}]"] = fin * (words * 8 + tree_row_bytes(words * 8))
            rows = fout
        elif isinstance(m, cl.ConvLayer):
            fin = m.in_shape[0] * m.in_shape[1] * m.in_shape[2]
            out[f"cl_eval_packed_indexed[{fin}->{m.out_dim}]"] = (fin + m.out_dim) * words * 8
            rows = m.out_dim
        elif isinstance(m, cl.LogicLayer):
            out[f"cl_eval_packed_indexed[{m.in_dim}->{m.out_dim}]"] = (m.in_dim + m.out_dim) * words * 8
            rows = m.out_dim
    out[f"cl_group_bit_sum[{rows}]"] = rows * words * 8 + words * 64 * k * 4
    return out


# Entry points whose calls only launch kernels into buffers allocated before the call, so
# that timing.record may issue them several times back to back (the same outputs rewritten).
REPEATABLE = ("cl_dense_backward_rows", "cl_dense_forward_fused", "cl_dense_forward_tiled",
              "cl_dense_backward_tiled", "cl_dense_backward_finalize", "cl_dense_weight_grad",
              "cl_dense_prep", "cl_conv_window_", "cl_tree_conv_backward",
              "cl_tree_conv_forward[")
BACK_TO_BACK = 20   # launches of the dominant kernel between one pair of events


def time_train_kernels(model, step, batch, nsteps, torch):
    """Mean duration of every library call inside `nsteps` real (eager) training steps,
    bracketed with HIP events on the stream each call uses (each call queued behind a spin
    kernel, so the interval holds no host wait; it still holds two event packets, about
    4-5 us).  Then the dominant call again, BACK_TO_BACK launches between one pair of events
    on the operands of two more eager steps: the figure the roofline uses, which a kernel
    trace of the same command reproduces launch by launch."""
    from compactlogic_amd import timing
    with timing.record() as rec:
        for _ in range(nsteps):
            model.zero_grad(set_to_none=True)
            step()
    kernels = kernel_table(rec.summary(), train_kernel_bytes(model, batch))
    dom = dominant_kernel(kernels)
    if dom.startswith(REPEATABLE):
        with timing.record(repeat={dom: BACK_TO_BACK}) as rec2:
            for _ in range(2):
                model.zero_grad(set_to_none=True)
                step()
        kernels[dom]["back_to_back_seconds"] = rec2.summary()[dom]["mean_ms"] * 1e-3
    return kernels


def dominant_kernel(kernels: dict) -> str:
    """The kernel with the largest total time per step among those with a byte count."""
    return max((k for k in kernels if kernels[k]["algorithmic_bytes"]),
               key=lambda k: kernels[k]["seconds"] * kernels[k]["calls"])


def kernel_table(summary: dict, nbytes_of: dict) -> dict:
    out = {}
    for name, v in summary.items():
        sec = v["mean_ms"] * 1e-3
        nbytes = nbytes_of.get(name)
        out[name] = dict(seconds=sec, calls=v["calls"], algorithmic_bytes=nbytes,
                         achieved_GBs=(nbytes / sec / 1e9) if nbytes else None)
    return out


def measured_traffic() -> dict:
    """HBM-side bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated) of the dominant kernels,
    from the committed counter profile; a kernel that is not listed reports null."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "traffic_per_launch.json")
    try:
        with open(path) as f:
            return json.load(f)["bytes"]
    except (OSError, ValueError, KeyError):
        return {}


def roofline_of(kernels: dict, how: str) -> dict:
    """The dominant kernel (largest total time per step among those with a byte count): its
    algorithmic bytes per launch over its launch duration, from the back-to-back launches
    when they were timed (time_train_kernels), else from the single-launch events."""
    name = dominant_kernel(kernels)
    d = kernels[name]
    b2b = d.get("back_to_back_seconds")
    sec = b2b if b2b else d["seconds"]
    achieved = d["algorithmic_bytes"] / sec / 1e9
    out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
           "traffic": measured_traffic().get(name), "kernel": name,
           "per_launch_ms": round(sec * 1e3, 4),
           "algorithmic_bytes_per_launch": d["algorithmic_bytes"],
           "measured": (f"HIP events around {BACK_TO_BACK} back-to-back launches of the kernel "
                        "on the operands of an eager training step" if b2b else how),
           "traffic_source": "profiles/traffic_per_launch.json (rocprofv3 --pmc FETCH_SIZE / "
                             "WRITE_SIZE of this command, calibrated by a 512 MiB copy)"}
    if b2b:
        out["in_step_event_ms"] = round(d["seconds"] * 1e3, 4)
        out["in_step_note"] = ("events around each single launch inside the eager steps; "
                               "they include the two event packets")
    # the same launch against the VALU, where the counter profile has it (the conv and tree
    # kernels are VALU-bound, not HBM-bound): frac is the counters' VALU busy (issue cycles
    # over elapsed cycles); the instruction rate over the nominal four-cycles-per-instruction
    # peak is beside it, and it can pass 1 where instructions take fewer cycles
    prof = valu_profile().get(name)
    if prof:
        valu = prof["valu_wave_instructions"] / sec / 1e9
        out["valu"] = {"frac": prof.get("valu_busy"), "achieved": round(valu, 1),
                       "peak": VALU_PEAK_G, "unit": "G wave64 VALU instructions/s",
                       "issue_frac": round(valu / VALU_PEAK_G, 4),
                       "valu_wave_instructions_per_launch": prof["valu_wave_instructions"],
                       "kernels": prof["kernel"],
                       "source": "profiles/valu_per_launch.json (rocprofv3 --pmc SQ_INSTS_VALU "
                                 "SQ_ACTIVE_INST_VALU GRBM_GUI_ACTIVE of this command)"}
    return out


def valu_profile() -> dict:
    """VALU wave64 instructions per launch and VALU busy of the fused packed kernels, from
    the committed counter profile (SQ_INSTS_VALU, SQ_ACTIVE_INST_VALU, GRBM_GUI_ACTIVE)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "valu_per_launch.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"]
    except (OSError, ValueError, KeyError):
        return {}


# VALU issue peak: one wave64 instruction per CU per cycle (four SIMD16 units, four cycles
# per wave64 instruction), 256 CUs at the 2.4 GHz peak engine clock.
VALU_PEAK_G = 256 * 2.4


def valu_roofline(key: str, seconds: float) -> dict | None:
    """Roofline of a VALU-bound fused pass: its profiled VALU instruction count per launch
    over the live launch duration, against VALU_PEAK_G; the counter profile's VALU busy
    (issue cycles over elapsed cycles, which also counts the launch's ramp) beside it."""
    prof = valu_profile().get(key)
    if not prof:
        return None
    achieved = prof["valu_wave_instructions"] / seconds / 1e9
    return {"bound": "valu", "achieved": round(achieved, 1), "peak": VALU_PEAK_G,
            "unit": "G wave64 VALU instructions/s", "frac": round(achieved / VALU_PEAK_G, 4),
            "traffic": None, "kernel": prof["kernel"], "per_launch_ms": round(seconds * 1e3, 3),
            "valu_wave_instructions_per_launch": prof["valu_wave_instructions"],
            "valu_busy_counter": prof.get("valu_busy"),
            "lds_bank_conflict_share": prof.get("lds_bank_conflict"),
            "source": "profiles/valu_per_launch.json (rocprofv3 --pmc SQ_INSTS_VALU "
                      "SQ_ACTIVE_INST_VALU GRBM_GUI_ACTIVE of this command)"}


def kernels_json(kernels: dict, steps: int) -> dict:
    return {k: {"ms": round(v["seconds"] * 1e3, 4), "calls_per_step": v["calls"] // steps,
                "GB/s": round(v["achieved_GBs"], 1) if v["achieved_GBs"] else None}
            for k, v in kernels.items()}


def cpu_baseline_train(torch, which: str):
    from compactlogic_amd import configs
    from oracle.torch_cpu import CpuDenseNet
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    if which == "cfg2":
        cfg = configs.CONFIGS["cfg2"]
        batch, warm, steps = 256, 1, 3
        model = configs.dense_network(cfg, device="cpu")
        x, labels = configs.dense_inputs(cfg, device="cpu", batch=batch)
        what = "cfg2 network (6x12000, G=16, fp32)"
    elif which == "cfg3_tree":
        cfg = configs.TREE_CONFIGS["cfg3_tree"]
        batch, warm, steps = 32, 1, 3
        # the blocks are built on the device (their constructor requires one), then copied
        model = configs.tree_network(cfg, device=torch.device("cuda:0"))
        x, labels = configs.conv_inputs(cfg, device="cpu", batch=batch)
        what = ("cfg3_tree network (2 logic-tree conv blocks, the python-path block of "
                "oracle/torch_cpu.py, + 2x16000 dense, fp32)")
    else:
        cfg = configs.CONV_CONFIGS["cfg3"]
        batch, warm, steps = 64, 1, 3
        model = configs.conv_network(cfg, device="cpu")
        x, labels = configs.conv_inputs(cfg, device="cpu", batch=batch)
        what = "cfg3 network (2 conv + 2x16000 dense, G=16, fp32)"
    net = CpuDenseNet.from_model(model)
    for _ in range(warm):
        net.train_step(x, labels)
    t0 = time.perf_counter()
    for _ in range(steps):
        net.train_step(x, labels)
    dt = (time.perf_counter() - t0) / steps
    return {"value": batch / dt, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"{what} fwd+bwd in torch CPU autograd (oracle/torch_cpu.py) at batch "
                      f"{batch} of {cfg.batch}, {warm} warm-up + {steps} timed steps; host "
                      f"{platform.processor() or platform.machine()}, "
                      f"os.cpu_count()={os.cpu_count()}"}


def bench_conv(args, torch):
    from compactlogic_amd import configs
    cfg = configs.CONV_CONFIGS["cfg3"]
    dev = torch.device("cuda:0")
    model = configs.conv_network(cfg, device=dev)
    x, labels = configs.conv_inputs(cfg, device=dev)
    samples_s, dt, kernels, matches = bench_train(model, x, labels, args.conv_steps,
                                                  args.conv_warmup, args.mode, args.kernel_steps,
                                                  torch)
    out = {
        "workload": "cfg3: ConvLayer 9x32x32 -> 256x16x16 (ks 3, stride 2, pad 1) -> 512x7x7 "
                    "(ks 3, stride 2, pad 0), flatten, LogicLayer 25088->16000->16000, "
                    "GroupSum(10, tau=30), G=16, batch 256, fp32 fwd+CE+bwd",
        "value": round(samples_s, 1), "unit": "samples/s", "steps": args.conv_steps,
        "warmup": args.conv_warmup, "ms_per_step": round(dt * 1e3, 4),
        "step_hbm_frac": round(CFG3_BYTES_PER_SAMPLE * samples_s / 1e9 / HBM_PEAK_GBS, 4),
        "timed_path_matches_eager": matches,
        "roofline": roofline_of(kernels, f"HIP events around each launch inside "
                                         f"{args.kernel_steps} eager training steps"),
        "kernels": kernels_json(kernels, args.kernel_steps),
    }
    del model
    torch.cuda.empty_cache()
    return out


def annotate_block_shapes(model, in_shape):
    """Record each ConvLogicLayer's input shape (for the byte accounting)."""
    shape = tuple(in_shape)
    for m in model:
        if hasattr(m, "complete"):
            m._last_shape = shape
            ho = (shape[1] + 2 * m.padding[0] - m.kernel[0]) // m.stride[0] + 1
            wo = (shape[2] + 2 * m.padding[1] - m.kernel[1]) // m.stride[1] + 1
            shape = (m.out_channels, ho // 2, wo // 2)


def bench_tree(args, torch):
    """The logic-tree reading of cfg3: two complete ConvLogicLayer blocks, the dense layers and
    GroupSum, trained like cfg3."""
    from compactlogic_amd import configs
    cfg = configs.TREE_CONFIGS["cfg3_tree"]
    dev = torch.device("cuda:0")
    model = configs.tree_network(cfg, device=dev)
    x, labels = configs.conv_inputs(cfg, device=dev)
    annotate_block_shapes(model, cfg.in_shape)
    samples_s, dt, kernels, matches = bench_train(model, x, labels, args.conv_steps,
                                                  args.conv_warmup, args.mode, args.kernel_steps,
                                                  torch)
    out = {
        "workload": "cfg3_tree: ConvLogicLayer(9->256, ks 3, stride 2, pad 1, complete: 8 taps, "
                    "4->2->1 gates, 2x2 max pool) -> 256x8x8 -> ConvLogicLayer(256->512) -> "
                    "512x2x2, flatten, LogicLayer 2048->16000->16000, GroupSum(10, tau=30), "
                    "batch 256, fp32 fwd+CE+bwd",
        "value": round(samples_s, 1), "unit": "samples/s", "steps": args.conv_steps,
        "warmup": args.conv_warmup, "ms_per_step": round(dt * 1e3, 4),
        "step_hbm_frac": round(CFG3_TREE_BYTES_PER_SAMPLE * samples_s / 1e9 / HBM_PEAK_GBS, 4),
        "timed_path_matches_eager": matches,
        "roofline": roofline_of(kernels, f"HIP events around each launch inside "
                                         f"{args.kernel_steps} eager training steps"),
        "kernels": kernels_json(kernels, args.kernel_steps),
    }
    del model
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------------- packed cfg4 / cfg5

def bench_packed_net(model, in_features: int, log2n: int, passes: int, k: int, torch):
    """Whole packed passes over 2^log2n resident samples (min over `passes`), then one more
    pass with every library call bracketed by HIP events."""
    import compactlogic_amd as cl
    from compactlogic_amd import configs, timing
    n = 1 << log2n
    words = n // 64
    xw = configs.packed_input_words(in_features, words, device=torch.device("cuda:0"))

    def one_pass():
        return model(cl.PackBitsTensor.from_packed(xw))

    counts = one_pass()
    torch.cuda.synchronize()
    times = []
    for _ in range(passes):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        counts = one_pass()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    dt = min(times)
    checksum = int(counts.to(torch.int64).sum().item())
    with timing.record() as rec:
        one_pass()
    kernels = kernel_table(rec.summary(), packed_kernel_bytes(model, words, k))
    del xw, counts
    torch.cuda.empty_cache()
    return dict(n=n, seconds=dt, samples_s=n / dt, checksum=checksum, kernels=kernels)


def bench_packed_fused(model, in_features: int, log2n: int, passes: int, checksum: int, torch,
                       key: str = ""):
    """The same network through PackedNetwork: its dense tail and the popcount GroupSum in one
    launch (activations in LDS), after the modules before the tail (conv blocks) layer by layer
    on the packed kernels.  Compulsory HBM bytes of a pass with no such prefix: the packed
    input and the int32 counts."""
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    n = 1 << log2n
    xw = configs.packed_input_words(in_features, n // 64, device=torch.device("cuda:0"))
    net = cl.PackedNetwork(model)
    x = cl.PackBitsTensor.from_packed(xw)
    counts = net(x)
    torch.cuda.synchronize()
    times = []
    for _ in range(passes):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        counts = net(x)
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) * 1e-3)
    dt = min(times)
    same = int(counts.to(torch.int64).sum().item()) == checksum
    from compactlogic_amd import timing
    with timing.record() as rec:
        net(x)
    calls = rec.summary()
    fused_call = next((v for k, v in calls.items() if k.startswith("cl_packed_network")), None)
    fused_rows = net.rows or []
    prefix = len(net.prefix)
    producer = net.producer is not None
    del xw, counts, net
    torch.cuda.empty_cache()
    out = {"workload": ("the same network and inputs through PackedNetwork: "
                        + (f"{prefix} modules layer by layer, then " if prefix else "")
                        + ("the layer before the dense tail written column-major, then "
                           if producer else "")
                        + f"the dense layers {fused_rows} and the class counts in one launch, "
                          "32-sample columns held in LDS through all fused layers"),
           "value": round(n / dt / 1e9, 4), "unit": "Gsamples/s", "ms_per_pass": round(dt * 1e3, 3),
           "counts_match_layerwise": same, "speedup_vs_layerwise": None,
           "kernels": {k: {"ms": round(v["mean_ms"], 4), "calls_per_step": v["calls"]}
                       for k, v in calls.items()}}
    if not prefix:
        fused_bytes = in_features // 8 + 4 * model[-1].k
        out["fused_compulsory_bytes_per_sample"] = fused_bytes
        out["hbm_frac_of_fused_bytes"] = round(fused_bytes * n / dt / 1e9 / HBM_PEAK_GBS, 4)
    if fused_call is not None:
        # the fused kernel keeps its activations in LDS and is bound by VALU issue
        roof = valu_roofline(key, fused_call["mean_ms"] * 1e-3)
        if roof is not None:
            out["roofline"] = roof
    return out


def packed_json(pk: dict, workload: str, bytes_per_sample: int) -> dict:
    return {
        "workload": workload,
        "value": round(pk["samples_s"] / 1e9, 4), "unit": "Gsamples/s",
        "ms_per_pass": round(pk["seconds"] * 1e3, 3),
        "hbm_frac": round(bytes_per_sample * pk["samples_s"] / 1e9 / HBM_PEAK_GBS, 4),
        "counts_checksum": pk["checksum"],
        "roofline": roofline_of(pk["kernels"], "HIP events around each launch inside one "
                                               "extra whole pass"),
        "kernels": kernels_json(pk["kernels"], 1),
    }


def cpu_baseline_packed(torch, which: str):
    import numpy as np
    import compactlogic_amd as cl
    from compactlogic_amd import configs
    from oracle import packed as P
    if which == "cfg4":
        cfg = configs.CONFIGS["cfg2"]
        model = configs.dense_network(cfg, device="cpu")
        configs.freeze_uniform_gates(model)
        in_features, log2n = cfg.in_dim, 16
    elif which == "cfg3_tree":
        cfg = configs.TREE_CONFIGS["cfg3_tree"]
        model = configs.tree_network(cfg, device=torch.device("cuda:0"))
        configs.freeze_argmax(model)
        in_features, log2n = cfg.in_shape[0] * cfg.in_shape[1] * cfg.in_shape[2], 16
    else:
        cfg = configs.CONV_CONFIGS["cfg5"]
        model = configs.conv_network(cfg, device="cpu")
        configs.freeze_argmax(model)
        in_features, log2n = cfg.in_shape[0] * cfg.in_shape[1] * cfg.in_shape[2], 15
    layers, blocks = [], []
    shape = getattr(cfg, "in_shape", None)
    for m in model:
        if isinstance(m, cl.ConvLogicLayer):
            gates = m.weights.argmax(-1).to(torch.uint8).cpu().numpy()
            sel = m.selection.to(torch.int32).cpu().numpy()
            blocks.append((gates, sel, shape, m.stride, m.padding, m.kernel))
            ho = (shape[1] + 2 * m.padding[0] - m.kernel[0]) // m.stride[0] + 1
            wo = (shape[2] + 2 * m.padding[1] - m.kernel[1]) // m.stride[1] + 1
            shape = (m.out_channels, ho // 2, wo // 2)
        elif isinstance(m, cl.ConvLayer):
            layers.append(P.resolve_conv_slots(m.offsets_ch.numpy(), m.offsets_h.numpy(),
                                               m.offsets_w.numpy(), m.gate_sequence.numpy(),
                                               m.w.numpy(), m.in_shape, m.stride, m.out_shape[1:]))
        elif isinstance(m, cl.LogicLayer):
            layers.append(P.resolve_slots(m.indices.cpu().numpy(), m.gate_sequence.cpu().numpy(),
                                          m.w.cpu().numpy()))
    # the samples (64 per word) split into one contiguous word range per host thread; the C
    # oracle releases the interpreter lock while it runs, so the threads run in parallel
    threads = min(16, os.cpu_count() or 1)
    log2n += 2 if threads >= 8 else 0
    n = 1 << log2n
    words = n // 64
    xw = np.stack([P.fill_splitmix64(words, (1 << 40) + f * words) for f in range(in_features)])
    bounds = np.linspace(0, words, threads + 1).astype(int)
    chunks = [np.ascontiguousarray(xw[:, lo:hi]) for lo, hi in zip(bounds[:-1], bounds[1:])
              if hi > lo]

    def counts_of(h):
        for gates, sel, shp, stride, pad, kernel in blocks:
            h = P.tree_block_bits(h, gates, sel, shp, stride, pad, kernel)
        return P.network_counts(h, layers, cfg.k)

    def one_pass():
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(len(chunks)) as ex:
            return np.concatenate(list(ex.map(counts_of, chunks)))

    one_pass()                                    # warm
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        one_pass()
    dt = (time.perf_counter() - t0) / reps
    return {"value": n / dt / 1e9, "unit": "Gsamples/s", "cores": len(chunks), "kind": "port",
            "sample": f"{which} network on 2^{log2n} samples, C oracle oracle/packed_ref.c, "
                      f"{len(chunks)} host threads (one word range each; "
                      f"os.cpu_count()={os.cpu_count()}), {reps} timed passes"}


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
                                   "not part of this build",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    from compactlogic_amd import _capi, configs
    _capi.load()

    calibration_copy(torch)
    log(f"dense cfg2: mode={args.mode} warmup={args.warmup} steps={args.steps}")
    cfg, samples_s, dt, kernels, matches = bench_dense(args, torch)
    log(f"dense cfg2: {samples_s:,.0f} samples/s, {dt * 1e3:.3f} ms/step")
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
        "roofline": roofline_of(kernels, f"HIP events around each launch inside "
                                         f"{args.kernel_steps} eager training steps run right "
                                         "after the timed region"),
        "kernels": kernels_json(kernels, args.kernel_steps),
    }
    log("dense cfg2 full step (with clip + Adam)")
    result["train_full"] = bench_train_full(args, torch)
    log(f"dense cfg2 full step: {result['train_full']['ms_per_step']:.3f} ms/step")
    log("dense cfg2 with the reference's default wiring (connections='random')")
    result["train_random_wiring"] = bench_dense_random(args, torch)
    log(f"dense cfg2 random wiring: {result['train_random_wiring']['ms_per_step']:.3f} ms/step")
    if not args.no_cpu_baseline:
        log("cpu baseline (cfg2)")
        result["cpu_baseline"] = cpu_baseline_train(torch, "cfg2")
    if not args.no_conv:
        log(f"conv cfg3: warmup={args.conv_warmup} steps={args.conv_steps}")
        conv = bench_conv(args, torch)
        log(f"conv cfg3: {conv['value']:,.0f} samples/s, {conv['ms_per_step']:.3f} ms/step")
        if not args.no_cpu_baseline:
            log("cpu baseline (cfg3)")
            conv["cpu_baseline"] = cpu_baseline_train(torch, "cfg3")
        result["conv_train"] = conv
        log(f"tree conv cfg3_tree: warmup={args.conv_warmup} steps={args.conv_steps}")
        tree = bench_tree(args, torch)
        log(f"tree conv cfg3_tree: {tree['value']:,.0f} samples/s, {tree['ms_per_step']:.3f} ms/step")
        if not args.no_cpu_baseline:
            log("cpu baseline (cfg3_tree)")
            tree["cpu_baseline"] = cpu_baseline_train(torch, "cfg3_tree")
        result["conv_tree_train"] = tree
    if not args.no_packed:
        log(f"packed cfg4: 2^{args.packed_log2_samples} samples x {args.packed_passes} passes")
        c2 = configs.CONFIGS["cfg2"]
        model = configs.dense_network(c2, device=torch.device("cuda:0"))
        configs.freeze_uniform_gates(model)
        pk = bench_packed_net(model, c2.in_dim, args.packed_log2_samples, args.packed_passes,
                              c2.k, torch)
        fused = bench_packed_fused(model, c2.in_dim, args.packed_log2_samples,
                                   args.packed_passes, pk["checksum"], torch, key="cfg4")
        del model
        packed = packed_json(pk, f"cfg4: cfg2 network frozen to argmax gates, "
                                 f"2^{args.packed_log2_samples} samples bit-packed 64 per word, "
                                 "6 bitwise layers + popcount GroupSum", CFG4_BYTES_PER_SAMPLE)
        fused["speedup_vs_layerwise"] = round(fused["value"] / packed["value"], 2)
        # The layer path's algorithmic bytes at the full 8 TB/s set a floor no unfused
        # implementation can beat; the fused pass removes those bytes instead.
        floor_ms = CFG4_BYTES_PER_SAMPLE * (1 << args.packed_log2_samples) / (HBM_PEAK_GBS * 1e6)
        fused["layerwise_hbm_floor_ms"] = round(floor_ms, 3)
        fused["speedup_vs_layerwise_hbm_floor"] = round(floor_ms / fused["ms_per_pass"], 2)
        packed["fused"] = fused
        log(f"packed cfg4: {packed['value']} Gsamples/s layer by layer, "
            f"{fused['value']} Gsamples/s fused")
        if not args.no_cpu_baseline:
            log("cpu baseline (cfg4)")
            packed["cpu_baseline"] = cpu_baseline_packed(torch, "cfg4")
        result["packed"] = packed
        if not args.no_conv:
            log(f"packed cfg5: 2^{args.conv_packed_log2_samples} samples")
            c5 = configs.CONV_CONFIGS["cfg5"]
            model = configs.conv_network(c5, device=torch.device("cuda:0"))
            configs.freeze_argmax(model)
            feats5 = c5.in_shape[0] * c5.in_shape[1] * c5.in_shape[2]
            pk = bench_packed_net(model, feats5, args.conv_packed_log2_samples,
                                  args.packed_passes, c5.k, torch)
            del model
            pc = packed_json(pk, f"cfg5: cfg3 network with 4 candidate gates per row, frozen "
                                 f"to argmax, 2^{args.conv_packed_log2_samples} samples bit-packed "
                                 "64 per word, 2 packed conv + 2 dense layers + popcount GroupSum",
                             CFG5_BYTES_PER_SAMPLE)
            model = configs.conv_network(c5, device=torch.device("cuda:0"))
            configs.freeze_argmax(model)
            fc = bench_packed_fused(model, feats5, args.conv_packed_log2_samples,
                                    args.packed_passes, pc["counts_checksum"], torch, key="cfg5")
            del model
            fc["speedup_vs_layerwise"] = round(fc["value"] / pc["value"], 2)
            pc["fused"] = fc
            log(f"packed cfg5: {pc['value']} Gsamples/s layer by layer, "
                f"{fc['value']} Gsamples/s with the dense tail fused")
            if not args.no_cpu_baseline:
                log("cpu baseline (cfg5)")
                pc["cpu_baseline"] = cpu_baseline_packed(torch, "cfg5")
            result["packed_conv"] = pc
            log(f"packed cfg3_tree: 2^{args.conv_packed_log2_samples} samples")
            ct = configs.TREE_CONFIGS["cfg3_tree"]
            model = configs.tree_network(ct, device=torch.device("cuda:0"))
            configs.freeze_argmax(model)
            annotate_block_shapes(model, ct.in_shape)
            pk = bench_packed_net(model, ct.in_shape[0] * ct.in_shape[1] * ct.in_shape[2],
                                  args.conv_packed_log2_samples, args.packed_passes, ct.k, torch)
            del model
            pt = packed_json(pk, f"cfg3_tree frozen to argmax gates (pool = OR), "
                                 f"2^{args.conv_packed_log2_samples} samples bit-packed 64 per "
                                 "word, 2 packed ConvLogic blocks + 2 dense layers + popcount "
                                 "GroupSum", CFG5_TREE_BYTES_PER_SAMPLE)
            model = configs.tree_network(ct, device=torch.device("cuda:0"))
            configs.freeze_argmax(model)
            ft = bench_packed_fused(model, ct.in_shape[0] * ct.in_shape[1] * ct.in_shape[2],
                                    args.conv_packed_log2_samples, args.packed_passes,
                                    pt["counts_checksum"], torch, key="cfg3_tree")
            del model
            ft["speedup_vs_layerwise"] = round(ft["value"] / pt["value"], 2)
            pt["fused"] = ft
            log(f"packed cfg3_tree: {pt['value']} Gsamples/s layer by layer, "
                f"{ft['value']} Gsamples/s with the dense tail fused")
            if not args.no_cpu_baseline:
                log("cpu baseline (packed cfg3_tree)")
                pt["cpu_baseline"] = cpu_baseline_packed(torch, "cfg3_tree")
            result["packed_conv_tree"] = pt
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
