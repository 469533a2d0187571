"""The optimizer half of a CompactLogic training step on the HIP kernels.

The reference trains with (experiments/experiment_script.py:280-293, :362)::

    loss.backward()
    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm=grad_clip_norm)   # 10.0
    optimizer.step()                                                              # torch.optim.Adam

`FusedAdam` does both in two launches over all parameters (cl_adam_clip_step): the global
gradient norm, the clipped gradients written back into ``p.grad`` as clip_grad_norm_ leaves
them, and the Adam update of every parameter.  The step count is a device tensor, so a step
captured in a HIP graph replays with correct bias corrections.  Sums have a fixed order: the
update is bitwise reproducible.

Differences from torch.optim.Adam: every parameter of the optimizer shares one step count,
which advances on every call (torch advances a parameter's count only when it has a
gradient); weight decay, amsgrad and maximize are not supported.  State dicts interchange
with torch.optim.Adam's: ``state_dict()`` gives each parameter its step as a float32 host
scalar, as Adam keeps it, and after ``load_state_dict`` the shared count resumes from the
loaded steps (which must agree), so the bias corrections continue where they stopped.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi
from . import difflogic_hip as _dl
from . import timing


class FusedAdam(torch.optim.Optimizer):
    """clip_grad_norm_(params, max_norm) followed by Adam(lr, betas, eps), fused.

    ``max_norm=None`` (or <= 0) skips the clipping.  All parameters must be HIP tensors of one
    dtype (float32 or float64) on one device."""

    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 max_norm: float | None = 10.0):
        if lr < 0 or eps < 0 or not (0 <= betas[0] < 1 and 0 <= betas[1] < 1):
            raise ValueError(f"invalid Adam hyper-parameters lr={lr} betas={betas} eps={eps}")
        defaults = dict(lr=lr, betas=tuple(betas), eps=eps)
        super().__init__(params, defaults)
        self.max_norm = max_norm
        self._step_t = None     # shared device step count
        self._workspace = None

    def _loaded_step(self) -> float:
        """The step count held in the state (after load_state_dict, a torch.optim.Adam or a
        FusedAdam state dict): equal for every parameter that has one, else an error; 0 when
        no parameter has one yet."""
        steps = set()
        for p, _ in self._params():
            st = self.state.get(p, {})
            if "step" in st:
                v = st["step"]
                steps.add(float(v.item() if torch.is_tensor(v) else v))
        if len(steps) > 1:
            raise RuntimeError(f"FusedAdam shares one step count, but the loaded state holds "
                               f"several: {sorted(steps)}")
        return steps.pop() if steps else 0.0

    def load_state_dict(self, state_dict):
        super().load_state_dict(state_dict)
        # the shared count is taken from the loaded per-parameter steps at the next step()
        self._step_t = None

    def state_dict(self):
        """torch.optim.Adam's layout: per-parameter step as a float32 host scalar."""
        sd = super().state_dict()
        state = {}
        for k, st in sd["state"].items():
            st = dict(st)
            if "step" in st and torch.is_tensor(st["step"]):
                st["step"] = torch.tensor(float(st["step"].item()), dtype=torch.float32)
            state[k] = st
        sd["state"] = state
        return sd

    def _params(self):
        out = []
        for group in self.param_groups:
            for p in group["params"]:
                out.append((p, group))
        return out

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        items = [(p, g) for p, g in self._params() if p.grad is not None]
        if not items:
            return loss
        p0 = items[0][0]
        dev, dtype = p0.device, p0.dtype
        code = _dl.dtype_code(p0)
        for p, _ in items:
            _dl._check(p, "parameter")
            if p.device != dev or p.dtype != dtype:
                raise RuntimeError("FusedAdam needs all parameters on one device in one dtype")
            if p.grad.dtype != dtype or not p.grad.is_contiguous():
                raise RuntimeError("FusedAdam needs contiguous gradients of the parameter dtype")
            if p.grad.is_sparse:
                raise RuntimeError("FusedAdam does not support sparse gradients")
        groups = {id(g): g for _, g in items}
        hp = {(g["lr"], g["betas"], g["eps"]) for g in groups.values()}
        if len(hp) != 1:
            raise RuntimeError("FusedAdam applies one set of hyper-parameters per call; "
                               "use one optimizer per parameter group setting")
        lr, (beta1, beta2), eps = next(iter(hp))
        if self._step_t is None or self._step_t.device != dev or self._step_t.dtype != dtype:
            start = self._loaded_step() if self._step_t is None else float(self._step_t)
            self._step_t = torch.full((), start, dtype=dtype, device=dev)
        for p, _ in items:
            st = self.state[p]
            if "exp_avg" not in st:
                st["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            for key in ("exp_avg", "exp_avg_sq"):   # loaded moments: the kernel's layout
                t = st[key]
                if t.shape != p.shape:
                    raise RuntimeError(f"FusedAdam state {key} has shape {tuple(t.shape)}, "
                                       f"the parameter {tuple(p.shape)}")
                if not t.is_contiguous() or t.device != dev or t.dtype != dtype:
                    st[key] = t.to(device=dev, dtype=dtype).contiguous()
            st["step"] = self._step_t
        max_t = ctypes.c_int64()
        _capi.call("cl_adam_clip_max_tensors", ctypes.byref(max_t))
        if len(items) > max_t.value:
            raise RuntimeError(f"FusedAdam updates at most {max_t.value} parameter tensors "
                               f"per optimizer, got {len(items)}")
        max_norm = float(self.max_norm) if self.max_norm is not None else 0.0
        ps = [p for p, _ in items]
        n = len(ps)
        arr = ctypes.c_void_p * n
        numels = (ctypes.c_int64 * n)(*[p.numel() for p in ps])
        nparts = ctypes.c_int64()
        _capi.call("cl_adam_clip_workspace", n, numels, ctypes.byref(nparts))
        if self._workspace is None or self._workspace.numel() < max(nparts.value, 1) \
                or self._workspace.device != dev or self._workspace.dtype != dtype:
            self._workspace = torch.empty(max(nparts.value, 1), dtype=dtype, device=dev)
        ptrs = [arr(*[t.data_ptr() for t in ts]) for ts in
                (ps, [p.grad for p in ps], [self.state[p]["exp_avg"] for p in ps],
                 [self.state[p]["exp_avg_sq"] for p in ps])]
        with torch.cuda.device(dev):
            timing.timed(f"cl_adam_clip_step[{sum(numels)}]", lambda: _capi.call(
                "cl_adam_clip_step", code, n, *ptrs, numels, self._step_t.data_ptr(),
                float(lr), float(beta1), float(beta2), float(eps), max_norm,
                self._workspace.data_ptr(), self._workspace.numel(), _dl.stream_of(p0)))
        return loss
