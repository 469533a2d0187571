"""Experiment checkpoints in the reference's format, and the networks they describe.

A checkpoint (experiments/experiment_script.py:520-541) is a ``torch.save`` dict
``{"step", "model_state", "optim_state", "rng_state", "freezer_info"}`` whose model_state is
the network's state dict without the frozen layers' ``.w`` buffers; its experiment directory
holds ``meta_data.json`` (experiments/results_json.py:21-44) whose ``args`` name the topology.
`build_model` restates the compiler's model builder (compiler/model_builder.py:55-114) with this
package's modules, so a reference checkpoint loads into a network that runs on the HIP
kernels, and `load_checkpoint` reads one without executing anything stored in it
(``torch.load(weights_only=True)``).
"""
from __future__ import annotations

import json
import os
from pathlib import Path

import torch

from .layers import ConvLayer, GroupSum, LogicLayer


def input_shape_of_dataset(dataset: str) -> tuple:
    """compiler/model_builder.py:26-37."""
    if dataset == "mnist":
        return (1, 28, 28)
    if "cifar-10" in dataset:
        return (3 * int(dataset.split("-")[2]), 32, 32)
    if "tiny-imagenet" in dataset:
        return (3 * int(dataset.split("-")[2]), 64, 64)
    if "ECG2D" in dataset:
        return (1, int(dataset.split("-")[1]), 187)
    raise ValueError(f"unsupported dataset {dataset!r}")


def input_dim_of_dataset(dataset: str) -> int:
    """compiler/model_builder.py:10-23."""
    if "ECG" in dataset:
        return int(dataset.split("-")[1]) * 187
    c, h, w = input_shape_of_dataset(dataset)
    return c * h * w


def num_classes_of_dataset(dataset: str) -> int:
    """compiler/model_builder.py:40-49."""
    if dataset == "mnist" or "cifar-10" in dataset:
        return 10
    if "tiny-imagenet" in dataset:
        return 200
    if "ECG" in dataset:
        return 5
    raise ValueError(f"unsupported dataset {dataset!r}")


def build_model(args: dict) -> torch.nn.Sequential:
    """The network of an experiment's args (compiler/model_builder.py:55-114): 'regular'
    (Flatten, model_scale-wide LogicLayers, GroupSum) or 'conv_spm' / 'conv_chm' (four
    ConvLayers, Flatten, two LogicLayers, GroupSum), on the CPU."""
    dataset, struct = str(args.get("dataset")), str(args.get("struct"))
    kw = dict(num_gates=int(args["num_gates"]), residual_init=bool(args.get("residual_init", False)))
    tau = float(args["tau"])
    k_cls = num_classes_of_dataset(dataset)
    if struct == "regular":
        width, depth = int(args["model_scale"]), int(args["num_layers"])
        mods = [torch.nn.Flatten(), LogicLayer(input_dim_of_dataset(dataset), width, **kw)]
        mods += [LogicLayer(width, width, **kw) for _ in range(depth - 1)]
        return torch.nn.Sequential(*mods, GroupSum(k_cls, tau, device="cpu"))
    if struct in ("conv_spm", "conv_chm"):
        k = int(args["model_scale"])
        neurons = 1250 * k if "tiny-imagenet" in dataset else 625 * k
        chn = int(args.get("num_chn", 1))
        c1 = ConvLayer(input_shape_of_dataset(dataset), padding=1, c_out=k, ks=3, stride=2,
                       num_chn=chn, **kw)
        if struct == "conv_chm":
            c2 = ConvLayer(c1.out_shape, padding=0, c_out=k, ks=1, stride=1, num_chn=0, **kw)
            c3 = ConvLayer(c2.out_shape, padding=1, c_out=4 * k, ks=3, stride=2, num_chn=chn, **kw)
            c4 = ConvLayer(c3.out_shape, padding=0, c_out=4 * k, ks=1, stride=1, num_chn=0, **kw)
        else:
            c2 = ConvLayer(c1.out_shape, padding=1, c_out=k, ks=3, stride=1, num_chn=chn, **kw)
            c3 = ConvLayer(c2.out_shape, padding=1, c_out=4 * k, ks=3, stride=2, num_chn=chn, **kw)
            c4 = ConvLayer(c3.out_shape, padding=1, c_out=4 * k, ks=3, stride=1, num_chn=chn, **kw)
        r1 = LogicLayer(c4.out_dim, int(neurons), **kw)
        r2 = LogicLayer(r1.out_dim, int(neurons), **kw)
        return torch.nn.Sequential(c1, c2, c3, c4, torch.nn.Flatten(), r1, r2,
                                   GroupSum(k_cls, tau, device="cpu"))
    raise ValueError(f"unsupported structure {struct!r}")


def filtered_model_state_dict(model: torch.nn.Module) -> dict:
    """The state dict without the frozen layers' ``.w`` buffers
    (experiments/experiment_script.py:520-525)."""
    return {k: v for k, v in model.state_dict().items() if not k.endswith(".w")}


def save_checkpoint(path, step, model, optimizer, freezer_info=None) -> None:
    """A checkpoint in the reference's layout (experiments/experiment_script.py:527-541): the
    optimizer is required, as there, since the reference's loader restores it; the host RNG
    and, with a GPU, every device's RNG state are saved."""
    if optimizer is None or not hasattr(optimizer, "state_dict"):
        raise TypeError("save_checkpoint needs the optimizer (its state is part of the layout)")
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    torch.save({
        "step": step,
        "model_state": {k: v.detach().cpu() for k, v in filtered_model_state_dict(model).items()},
        "optim_state": optimizer.state_dict(),
        "rng_state": {
            "torch": torch.get_rng_state(),
            "cuda": torch.cuda.get_rng_state_all() if torch.cuda.is_available() else None,
        },
        "freezer_info": freezer_info if freezer_info is not None else "",
    }, path)


def resume_checkpoint(path, model, optimizer, map_location="cpu", strict=False):
    """Restore a training run from a checkpoint, as the reference's training loader does
    (experiments/experiment_script.py:543-569): the model state (non-strict: frozen layers'
    ``.w`` buffers are not saved), layers that hold a ``w`` buffer marked frozen, the
    optimizer state moved to the parameters' device, and the RNG states.  Loads with
    ``weights_only=True``.  Returns (step, freezer_info)."""
    ckpt = torch.load(path, map_location=map_location, weights_only=True)
    model.load_state_dict(ckpt["model_state"], strict=strict)
    for layer in model:
        if getattr(layer, "w", None) is not None:
            layer.is_frozen = True
    optimizer.load_state_dict(ckpt["optim_state"])
    params = list(model.parameters())
    if params:
        device = params[0].device
        for state in optimizer.state.values():
            for key, v in state.items():
                if torch.is_tensor(v) and key != "step":
                    state[key] = v.to(device)
    rng = ckpt.get("rng_state")
    if rng is not None:
        if rng.get("torch") is not None:
            torch.set_rng_state(rng["torch"])
        if torch.cuda.is_available() and rng.get("cuda") is not None:
            torch.cuda.set_rng_state_all(rng["cuda"])
    return ckpt.get("step"), ckpt.get("freezer_info")


def save_meta_data(directory, args: dict) -> None:
    """meta_data.json with the experiment's args (experiments/results_json.py:21-35)."""
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "meta_data.json"), "w") as f:
        json.dump({"args": args}, f)


def load_checkpoint(path, meta_path=None, device="cuda"):
    """(model, args, step) of a checkpoint and its experiment's meta_data.json (by default the
    checkpoint's sibling, compiler/extract.py:22-38).  The model is built from the args, its
    state loaded non-strictly as the reference does (experiments/experiment_script.py:543-
    547), moved to `device` and put in eval mode: every layer evaluates its argmax slot."""
    path = Path(path)
    meta_path = Path(meta_path) if meta_path is not None else path.with_name("meta_data.json")
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    with open(meta_path) as f:
        args = json.load(f).get("args", {})
    model = build_model(args)
    model.load_state_dict(ckpt["model_state"], strict=False)
    model = model.to(device)
    for m in model:
        if isinstance(m, GroupSum):
            m.device = device
    model.eval()
    return model, args, ckpt.get("step")
