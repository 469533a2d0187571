"""LogicLayer / GroupSum / PackBitsTensor and their autograd Functions on gfx950.

The constructors, buffers, forward dispatch and autograd signatures follow the reference
modules in compactlogic/compactlogic.py (LogicLayer :10-444, GroupSum :450-468,
LogicLayerCudaFunction :474-508) and the packed-bit API of the difflogic lineage
(third_party/convlogic_source_code/src/difflogic/packbitstensor.py:11-43,
difflogic.py:92-106,149-164,203-205).  Every numeric path runs on the HIP library; a tensor
that is not on a HIP device is rejected, never computed on the CPU.
"""
from __future__ import annotations

import ctypes
import weakref

import numpy as np
import torch

from . import _capi
from . import convlogic_hip as _cl
from . import difflogic_hip as _dl
from . import timing
from .plan import PART_SLOTS, REORDER_FRACTION, RunPlan, build_run_plan, locality_order


########################################################################################################################
# Packed bits


class PackBitsTensor:
    """Bit-packed batch: `t` is [features, ceil(batch / bit_count)] integer words, bit i of word
    w holds sample bit_count * w + i (packbitstensor.py:11-21); the last pad_len bits of a row
    are padding (layers may widen the rows and pad_len with them)."""

    def __init__(self, t: torch.Tensor, bit_count: int = 32):
        assert len(t.shape) == 2, t.shape
        self.bit_count = bit_count
        if t.device.type != "cuda":
            raise NotImplementedError(
                f"PackBitsTensor only supports device tensors, but got {t.device}.")
        t = t.T.contiguous()
        self.t, self.pad_len = _dl.tensor_packbits_cuda(t, self.bit_count)

    @classmethod
    def from_packed(cls, words: torch.Tensor, pad_len: int = 0, bit_count: int | None = None):
        """Wrap already packed rows [features, words] (no copy)."""
        obj = cls.__new__(cls)
        obj.t = words
        obj.pad_len = int(pad_len)
        obj.bit_count = bit_count or words.element_size() * 8
        return obj

    @property
    def is_cuda(self) -> bool:
        return self.t.is_cuda

    @property
    def device(self):
        return self.t.device

    @property
    def num_samples(self) -> int:
        return self.t.shape[1] * self.t.element_size() * 8 - self.pad_len

    def group_sum(self, k):
        return timing.timed(f"cl_group_bit_sum[{self.t.shape[0]}]",
                            lambda: _dl.groupbitsum(self.t, self.pad_len, k))

    def flatten(self, start_dim=0, end_dim=-1, **kwargs):
        """Returns the PackBitsTensor itself (its feature axis is already flat)."""
        return self

    def _member_repr(self, member):
        bits = self.bit_count
        if len(member) <= 4:
            return " ".join(np.binary_repr(int(v), width=bits)[::-1] for v in member)
        head = " ".join(np.binary_repr(int(v), width=bits)[::-1] for v in member[:3])
        return f"{head} ... {np.binary_repr(int(member[-1]), width=bits)[::-1]}"

    def __repr__(self):
        return "\n".join(self._member_repr(row.tolist()) for row in self.t.cpu())


########################################################################################################################
# Autograd functions


class LogicLayerCudaFunction(torch.autograd.Function):
    """Reference autograd bridge (compactlogic/compactlogic.py:474-508) over the drop-in
    kernels: same inputs, same saved tensors, same (grad_x, grad_w) outputs."""

    @staticmethod
    def forward(ctx, x, a, b, w, gate_sequence, given_x_indices_of_y_start, given_x_indices_of_y,
                given_x_indices_of_gate):
        ctx.save_for_backward(x, a, b, w, gate_sequence, given_x_indices_of_y_start,
                              given_x_indices_of_y, given_x_indices_of_gate)
        return _dl.forward(x, a, b, w, gate_sequence)

    @staticmethod
    def backward(ctx, grad_y):
        (x, a, b, w, gate_sequence, given_x_indices_of_y_start, given_x_indices_of_y,
         given_x_indices_of_gate) = ctx.saved_tensors
        grad_y = grad_y.contiguous()
        grad_w = grad_x = None
        if ctx.needs_input_grad[0]:
            grad_x = _dl.backward_x(x, a, b, w, gate_sequence, grad_y, given_x_indices_of_y_start,
                                    given_x_indices_of_y, given_x_indices_of_gate)
        if ctx.needs_input_grad[3]:
            grad_w = _dl.backward_w(x, a, b, gate_sequence, grad_y)
        return grad_x, None, None, grad_w, None, None, None, None


def _chunks(x: torch.Tensor, in_dim: int, out_dim: int) -> int:
    n = ctypes.c_int64(0)
    _capi.call("cl_dense_tiled_chunks", _dl.dtype_code(x), x.shape[1], in_dim, out_dim,
               ctypes.byref(n))
    return n.value


class LogicLayerRunsFunction(torch.autograd.Function):
    """Dense layer through the connection-run plan (same math as LogicLayerCudaFunction).

    ``w`` holds logits when ``softmax`` is true (the softmax and its backward run inside the
    HIP kernels and the gradient returned is that of the logits), else probabilities.  Slots
    sharing an input pair are collapsed, the batch is tiled in XCD-pinned chunks, and both
    gradients come from one pass over the inverse index plus a per-neuron finalize (a single
    whole-batch pass when the input needs no gradient).  When every neuron is one run of at
    most 16 slots, the softmax and the collapse happen inside the forward kernel
    (cl_dense_forward_fused); `fused_forward = False` selects the separate prep launch.
    `partitioned_backward = True` takes the input gradient through the plan's tiles
    (cl_dense_backward_part: runs with both inputs in one tile read grad_y once and their
    inputs from LDS).  It reads a third fewer row bytes but its barrier-separated phases keep
    fewer loads in flight, and it measures slower than cl_dense_backward_tiled at cfg2, so it
    is off by default.  Layers of single-run neurons with batches of up to 2048 (fp32) take
    both gradients from cl_dense_backward_rows (one wave per input row over the whole batch,
    finalize inside); `row_backward = False` selects the chunked passes."""

    fused_forward = True
    partitioned_backward = False
    row_backward = True

    @staticmethod
    def forward(ctx, x, w, gate_sequence, plan: RunPlan, softmax: bool = False,
                side: dict | None = None):
        _dl._check(x, "x")
        if w.dtype != x.dtype:
            raise RuntimeError("w must have the dtype of x")
        if x.shape[0] != plan.in_dim:
            raise RuntimeError(f"x has {x.shape[0]} rows, the layer expects {plan.in_dim}")
        batch = x.shape[1]
        w = w.contiguous()
        dev = x.device
        code = _dl.dtype_code(x)
        probs = torch.empty_like(w) if softmax else None
        inv_coef = torch.empty((2 * plan.num_runs, 2), dtype=x.dtype, device=dev)
        y = torch.empty((plan.out_dim, batch), dtype=x.dtype, device=dev)
        stream = _dl.stream_of(x)
        if (LogicLayerRunsFunction.fused_forward and plan.single_run and plan.num_gates <= 16
                and batch > 0):
            with torch.cuda.device(dev):
                timing.timed(f"cl_dense_forward_fused[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                    "cl_dense_forward_fused", code, x.data_ptr(), w.data_ptr(), int(softmax),
                    gate_sequence.data_ptr(), plan.nab.data_ptr(), plan.inv_pos.data_ptr(),
                    _dl.ptr(probs), inv_coef.data_ptr(), y.data_ptr(), plan.in_dim, plan.out_dim,
                    plan.num_runs, batch, plan.num_gates, stream))
            ctx.save_for_backward(x, inv_coef, gate_sequence, probs)
            ctx.plan = plan
            if side is not None:
                side["probs"] = probs
            return y
        coef = torch.empty((plan.num_runs, 4), dtype=x.dtype, device=dev)
        with torch.cuda.device(dev):
            timing.timed(f"cl_dense_prep[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                "cl_dense_prep", code, w.data_ptr(), int(softmax), gate_sequence.data_ptr(),
                plan.run_ptr.data_ptr(), plan.run_gl.data_ptr(), plan.inv_pos.data_ptr(),
                _dl.ptr(probs), coef.data_ptr(), inv_coef.data_ptr(), plan.out_dim,
                plan.num_runs, plan.num_gates, stream))
            timing.timed(f"cl_dense_forward_tiled[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                "cl_dense_forward_tiled", code, x.data_ptr(), coef.data_ptr(), plan.nab.data_ptr(),
                plan.run_ab.data_ptr(), y.data_ptr(), plan.in_dim, plan.out_dim, plan.num_runs,
                batch, stream))
        ctx.save_for_backward(x, inv_coef, gate_sequence, probs)
        ctx.plan = plan
        if side is not None:
            side["probs"] = probs
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, inv_coef, gate_sequence, probs = ctx.saved_tensors
        plan: RunPlan = ctx.plan
        grad_y = grad_y.contiguous()
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grad_x = torch.empty_like(x) if need_x else None
        grad_w = (torch.empty((plan.out_dim, plan.num_gates), dtype=x.dtype, device=x.device)
                  if need_w else None)
        code = _dl.dtype_code(x)
        stream = _dl.stream_of(x)
        batch = x.shape[1]
        with torch.cuda.device(x.device):
            wide = 16 // x.element_size()
            if (need_x and LogicLayerRunsFunction.row_backward and plan.single_run
                    and plan.num_gates <= 64 and 0 < batch <= 64 * wide * 8
                    and batch % wide == 0):
                timing.timed(f"cl_dense_backward_rows[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                    "cl_dense_backward_rows", code, x.data_ptr(), grad_y.data_ptr(),
                    plan.slot_rec.data_ptr(), plan.inv_rec.data_ptr(), inv_coef.data_ptr(),
                    gate_sequence.data_ptr(), _dl.ptr(probs), plan.run_ptr.data_ptr(),
                    _dl.ptr(grad_w), grad_x.data_ptr(), plan.in_dim, plan.out_dim,
                    plan.num_runs, batch, plan.num_gates, stream))
            elif need_x:
                moments, nchunks = None, 1
                if need_w:
                    nchunks = _chunks(x, plan.in_dim, plan.out_dim)
                    moments = torch.empty((plan.num_runs, nchunks, 4), dtype=x.dtype,
                                          device=x.device)
                if LogicLayerRunsFunction.partitioned_backward and plan.tile_ptr is not None:
                    timing.timed(f"cl_dense_backward_part[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                        "cl_dense_backward_part", code, x.data_ptr(), grad_y.data_ptr(),
                        plan.slot_rec.data_ptr(), plan.inv_rec.data_ptr(), inv_coef.data_ptr(),
                        plan.inv_slot.data_ptr(), plan.tile_ptr.data_ptr(),
                        plan.tile_run.data_ptr(), plan.tile_loc.data_ptr(),
                        plan.tile_loc.numel(), PART_SLOTS,
                        grad_x.data_ptr(), _dl.ptr(moments), nchunks, plan.in_dim, plan.out_dim,
                        plan.num_runs, batch, stream))
                else:
                    timing.timed(f"cl_dense_backward_tiled[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                        "cl_dense_backward_tiled", code, x.data_ptr(), grad_y.data_ptr(),
                        plan.run_ptr.data_ptr(), plan.run_ab.data_ptr(), plan.slot_rec.data_ptr(),
                        plan.inv_rec.data_ptr(), inv_coef.data_ptr(), grad_x.data_ptr(),
                        _dl.ptr(moments), nchunks, plan.in_dim, plan.out_dim, plan.num_runs,
                        batch, stream))
                if need_w:
                    timing.timed(f"cl_dense_backward_finalize[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                        "cl_dense_backward_finalize", code, moments.data_ptr(), nchunks,
                        gate_sequence.data_ptr(), _dl.ptr(probs), plan.run_ptr.data_ptr(),
                        plan.run_gl.data_ptr(), grad_w.data_ptr(), plan.out_dim, plan.num_runs,
                        plan.num_gates, stream))
            elif need_w:
                timing.timed(f"cl_dense_weight_grad[{plan.in_dim}->{plan.out_dim}]", lambda: _capi.call(
                    "cl_dense_weight_grad", code, x.data_ptr(), grad_y.data_ptr(),
                    gate_sequence.data_ptr(), _dl.ptr(probs), plan.run_ptr.data_ptr(),
                    plan.run_ab.data_ptr(), plan.run_gl.data_ptr(), grad_w.data_ptr(),
                    plan.in_dim, plan.out_dim, plan.num_runs, batch, plan.num_gates, stream))
        return grad_x, grad_w, None, None, None, None


# Entries per input row (2 * num_runs / in_dim, rounded down) from which
# cl_dense_backward_rows shares a row among several waves (CL_BWD_ROWS_S2 in
# dense_tiled.hip); its first-layer mode keeps one wave per row.
_ROWS_SHARED_FROM = 6


def _row_backward_fits(plan: RunPlan, x: torch.Tensor) -> bool:
    """Whether cl_dense_backward_rows takes this layer at this batch (x: [in_dim, batch])."""
    wide = 16 // x.element_size()
    batch = x.shape[1]
    return (plan.single_run and plan.num_gates <= 64 and 0 < batch <= 64 * wide * 8
            and batch % wide == 0)


class LogicLayerFirstPairFunction(torch.autograd.Function):
    """The second dense layer of a network together with the logits gradient of the first,
    whose input needs no gradient (compactlogic/compactlogic.py:83-118 applied to two layers in
    turn).  The forward is the second layer's (its input, the first layer's output y1, is
    taken as data); the backward is the second layer's row backward, which also finishes the
    first layer's logits gradient from the gradient of y1 as it computes it
    (cl_dense_backward_rows_first), so that gradient [out_dim1, batch] is never stored and
    the first layer's weight-gradient pass never runs.  Gradients are bitwise those of the two
    layers' own autograd steps.  No counterpart in the reference."""

    @staticmethod
    def forward(ctx, y1, w2, gate_sequence2, plan2: RunPlan, w1, x0, probs1, gate_sequence1,
                plan1: RunPlan):
        y = torch.empty((plan2.out_dim, y1.shape[1]), dtype=y1.dtype, device=y1.device)
        inv_coef = torch.empty((2 * plan2.num_runs, 2), dtype=y1.dtype, device=y1.device)
        probs2 = torch.empty_like(w2)
        w2 = w2.contiguous()
        with torch.cuda.device(y1.device):
            timing.timed(f"cl_dense_forward_fused[{plan2.in_dim}->{plan2.out_dim}]", lambda: _capi.call(
                "cl_dense_forward_fused", _dl.dtype_code(y1), y1.data_ptr(), w2.data_ptr(), 1,
                gate_sequence2.data_ptr(), plan2.nab.data_ptr(), plan2.inv_pos.data_ptr(),
                probs2.data_ptr(), inv_coef.data_ptr(), y.data_ptr(), plan2.in_dim,
                plan2.out_dim, plan2.num_runs, y1.shape[1], plan2.num_gates, _dl.stream_of(y1)))
        ctx.save_for_backward(y1, inv_coef, gate_sequence2, probs2, x0, probs1, gate_sequence1)
        ctx.plan2, ctx.plan1 = plan2, plan1
        return y

    @staticmethod
    def backward(ctx, grad_y):
        y1, inv_coef, gs2, probs2, x0, probs1, gs1 = ctx.saved_tensors
        plan2, plan1 = ctx.plan2, ctx.plan1
        grad_y = grad_y.contiguous()
        dev = y1.device
        grad_w2 = torch.empty((plan2.out_dim, plan2.num_gates), dtype=y1.dtype, device=dev)
        grad_w1 = torch.empty((plan1.out_dim, plan1.num_gates), dtype=y1.dtype, device=dev)
        with torch.cuda.device(dev):
            timing.timed(f"cl_dense_backward_rows_first[{plan2.in_dim}->{plan2.out_dim}]", lambda: _capi.call(
                "cl_dense_backward_rows_first", _dl.dtype_code(y1), y1.data_ptr(),
                grad_y.data_ptr(), plan2.slot_rec.data_ptr(), plan2.inv_rec.data_ptr(),
                inv_coef.data_ptr(), gs2.data_ptr(), probs2.data_ptr(), plan2.run_ptr.data_ptr(),
                grad_w2.data_ptr(), plan2.in_dim, plan2.out_dim, plan2.num_runs, y1.shape[1],
                plan2.num_gates, x0.data_ptr(), plan1.in_dim, plan1.nab.data_ptr(),
                plan1.num_runs, gs1.data_ptr(), probs1.data_ptr(), grad_w1.data_ptr(),
                plan1.num_gates, _dl.stream_of(y1)))
        return None, grad_w2, None, None, grad_w1, None, None, None, None


def _transpose_rows(x: torch.Tensor) -> torch.Tensor:
    """Contiguous [cols, rows] transpose of a contiguous 2-D device tensor [rows, cols]."""
    out = torch.empty((x.shape[1], x.shape[0]), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        timing.timed(f"cl_transpose[{x.shape[0]}x{x.shape[1]}]", lambda: _capi.call(
            "cl_transpose", _dl.dtype_code(x), x.data_ptr(), out.data_ptr(), x.shape[0],
            x.shape[1], _dl.stream_of(x)))
    return out


class TransposeFunction(torch.autograd.Function):
    """x [batch, features] -> contiguous [features, batch] rows, and the gradient back, through
    the HIP transpose kernel: the layout change of compactlogic/compactlogic.py:100-101."""

    @staticmethod
    def forward(ctx, x):
        return _transpose_rows(x.contiguous())

    @staticmethod
    def backward(ctx, grad):
        return _transpose_rows(grad.contiguous())


def to_rows(x: torch.Tensor) -> torch.Tensor:
    """[batch, features] -> contiguous [features, batch]; a view when x already is the
    transpose of a contiguous tensor (the output of a previous LogicLayer)."""
    t = x.transpose(0, 1)
    if t.is_contiguous():
        return t
    if x.device.type == "cuda" and x.dtype in (torch.float32, torch.float64):
        return TransposeFunction.apply(x)
    return t.contiguous()


class GroupSumFunction(torch.autograd.Function):
    """GroupSum (compactlogic/compactlogic.py:460-465) on the HIP kernels.  Reads the input
    through its strides, so the transposed view a LogicLayer returns costs no copy, and
    returns the input gradient in the same memory layout as the input."""

    @staticmethod
    def forward(ctx, x, k, tau):
        if x.device.type != "cuda":
            raise RuntimeError("GroupSum input must be a HIP device tensor")
        if x.dim() != 2:
            raise RuntimeError("GroupSum expects a 2-D [batch, features] input")
        batch, feats = x.shape
        sb, sf = x.stride()
        if sb < 0 or sf < 0 or (batch > 1 and feats > 1 and (sb == 0 or sf == 0)):
            x = x.contiguous()
            sb, sf = x.stride()
        out = torch.empty((batch, k), dtype=x.dtype, device=x.device)
        need = ctypes.c_int64(0)
        _capi.call("cl_group_sum_workspace_size", _dl.dtype_code(x), batch, feats, sb, sf, k,
                   ctypes.byref(need))
        ws = torch.empty(need.value, dtype=torch.uint8, device=x.device) if need.value else None
        with torch.cuda.device(x.device):
            timing.timed("cl_group_sum_forward", lambda: _capi.call(
                "cl_group_sum_forward", _dl.dtype_code(x), x.data_ptr(), batch, feats, sb, sf, k,
                float(tau), out.data_ptr(), _dl.ptr(ws), need.value, _dl.stream_of(x)))
        ctx.k, ctx.tau = k, tau
        ctx.shape = (batch, feats)
        ctx.batch_major = sb == 1 and sf != 1
        return out

    @staticmethod
    def backward(ctx, grad_out):
        grad_out = grad_out.contiguous()
        batch, feats = ctx.shape
        if ctx.batch_major:
            grad_x = torch.empty((feats, batch), dtype=grad_out.dtype, device=grad_out.device).t()
        else:
            grad_x = torch.empty((batch, feats), dtype=grad_out.dtype, device=grad_out.device)
        sb, sf = grad_x.stride()
        with torch.cuda.device(grad_out.device):
            timing.timed("cl_group_sum_backward", lambda: _capi.call(
                "cl_group_sum_backward", _dl.dtype_code(grad_out), grad_out.data_ptr(), batch,
                feats, ctx.k, float(ctx.tau), grad_x.data_ptr(), sb, sf, _dl.stream_of(grad_out)))
        return grad_x, None, None


########################################################################################################################
# Modules


# Average reads per input row up to which a frozen layer's packed evaluation follows the
# chain order (above it, many consecutive neurons would read the same input row at once).
_PACKED_CHAIN_MAX_DEGREE = 8


class LogicLayer(torch.nn.Module):
    """Differentiable logic-gate layer (compactlogic/compactlogic.py:10-130).

    Parameters
    ----------
    in_dim, out_dim : int
    connections : {'random', 'original'}
        'random' draws an independent input pair for every gate slot; 'original' draws one
        pair per neuron shared by all its slots.
    num_gates : int, default 16
        Candidate gate slots per neuron (opcode of slot g defaults to g & 15).
    residual_init : bool
        Bias every neuron towards the pass-through gate (slot 3) instead of N(0, 1) logits.

    Buffers: ``gate_sequence`` uint8 [out, G], ``indices`` int64 [2, out, G] and the inverse
    index ``given_x_indices_of_y_start`` / ``given_x_indices_of_y`` /
    ``given_x_indices_of_gate`` (state-dict compatible with the reference); ``w`` (uint8 argmax
    slots) after ``freeze()``.  The connection-run plan used by the kernels is derived state
    and is not saved.
    """

    def __init__(self, in_dim: int, out_dim: int, connections: str = 'random', num_gates=16,
                 residual_init: bool = False):
        super().__init__()
        self.in_dim = in_dim
        self.out_dim = out_dim
        self.connections = connections
        self.num_gates = num_gates
        self.log_k = torch.log(torch.tensor(self.num_gates)).item()
        self.init_weights(residual_init)
        self.init_gate_sequence()
        self.get_connections(device=self.weights.device)
        self._plan = None
        self._plan_key = None
        self.refresh_backward_index()
        self.num_neurons = out_dim
        self.num_weights = out_dim
        self.is_frozen = False

    # caches keyed by weak references, which do not pickle; they rebuild on the next call
    _weak_caches = ("_argmax_cache", "_plan_key", "_plan", "_packed_key", "_packed_tables")

    def __getstate__(self):
        state = super().__getstate__()
        for name in self._weak_caches:
            if name in state:
                state[name] = None
        return state

    # -- forward ------------------------------------------------------------------------------------------------------

    def forward(self, x):
        if getattr(self, "is_frozen", False) or not self.training or isinstance(x, PackBitsTensor):
            with torch.no_grad():
                return self.forward_cuda_eval(x)
        return self.forward_cuda(x)

    def forward_cuda(self, x):
        """Training forward: x [batch, in_dim] -> [batch, out_dim] (a transposed view of the
        kernel's [out_dim, batch] output, as in the reference, :83-118)."""
        assert x.ndim == 2, x.ndim
        x_in = x
        x = to_rows(x)
        assert x.shape[0] == self.in_dim, (x.shape, self.in_dim)
        if x.dtype == torch.float16:
            # half: the reference-interface kernels (half storage, fp32 sums) with the
            # reference's own argument list and inverse index
            w = torch.nn.functional.softmax(self.weights, dim=-1).to(x.dtype)
            return LogicLayerCudaFunction.apply(
                x, self.indices[0], self.indices[1], w, self.gate_sequence,
                self.given_x_indices_of_y_start, self.given_x_indices_of_y,
                self.given_x_indices_of_gate).transpose(0, 1)
        plan = self.run_plan()
        if self.weights.dtype == x.dtype:
            # softmax(weights) and its backward run inside the kernels
            pair = self._first_pair(x_in, x, plan)
            if pair is not None:
                return pair.transpose(0, 1)
            side = {} if self._may_lead_pair(x, plan) else None
            y = LogicLayerRunsFunction.apply(x, self.weights, self.gate_sequence, plan, True, side)
            out = y.transpose(0, 1)
            if side is not None and side.get("probs") is not None:
                # the next dense layer may finish this layer's logits gradient
                out._cl_first = (self, x, side["probs"], plan, out._version)
            return out
        else:
            w = torch.nn.functional.softmax(self.weights, dim=-1).to(x.dtype)
            y = LogicLayerRunsFunction.apply(x, w, self.gate_sequence, plan, False)
        return y.transpose(0, 1)

    # Whether the first-layer pairing applies (LogicLayerFirstPairFunction); a class switch.
    first_pair = True

    def _may_lead_pair(self, x: torch.Tensor, plan: RunPlan) -> bool:
        """This layer's output may feed the next layer's pair step: its input needs no
        gradient, its logits do, and its neurons are single runs of at most 64 slots."""
        return (LogicLayer.first_pair and type(self) is LogicLayer and torch.is_grad_enabled()
                and not x.requires_grad and self.weights.requires_grad
                and x.dtype in (torch.float32, torch.float64) and _row_backward_fits(plan, x))

    def _first_pair(self, x_in: torch.Tensor, x: torch.Tensor, plan: RunPlan):
        """This layer's output through LogicLayerFirstPairFunction when x_in is the output of
        a first layer (tagged by its forward, unmodified since) and this layer's row backward
        applies; else None."""
        tag = getattr(x_in, "_cl_first", None)
        if tag is None or not LogicLayer.first_pair or type(self) is not LogicLayer:
            return None
        first, x0, probs1, plan1, version = tag
        # the pair gives y1 no gradient of its own: not when the caller retains or hooks it
        if x_in.retains_grad or getattr(x_in, "_backward_hooks", None):
            return None
        if (x_in._version != version or not torch.is_grad_enabled()
                or not self.weights.requires_grad or not first.weights.requires_grad
                or first.weights.dtype != x.dtype or x.data_ptr() != x_in.data_ptr()
                or plan1.out_dim != plan.in_dim or not _row_backward_fits(plan, x)):
            return None
        # bitwise equal to the unpaired steps only where those take one wave per input row
        if 2 * plan.num_runs // max(plan.in_dim, 1) >= _ROWS_SHARED_FROM:
            return None
        return LogicLayerFirstPairFunction.apply(
            x.detach(), self.weights, self.gate_sequence, plan, first.weights, x0, probs1,
            first.gate_sequence, plan1)

    @torch.no_grad()
    def forward_cuda_eval(self, x):
        """Discrete forward with the argmax slot per neuron (:120-130).  A PackBitsTensor is
        evaluated bitwise and updated in place, as in difflogic.py:149-164."""
        assert self.is_frozen or not self.training
        w = getattr(self, "w", None)
        if w is None:
            w = self._argmax_slots()
        a, b = self.indices[0], self.indices[1]
        if isinstance(x, PackBitsTensor):
            assert x.t.shape[0] == self.in_dim, (x.t.shape, self.in_dim)
            ia, ib, gate, order = self.packed_tables(w)
            x.t = timing.timed(f"cl_eval_packed_indexed[{self.in_dim}->{self.out_dim}]",
                               lambda: _cl.eval_packed_indexed(x.t, ia, ib, gate, order))
            return x
        assert x.shape[-1] == self.in_dim, (x.shape, self.in_dim)
        return _dl.eval(to_rows(x), a, b, w, self.gate_sequence).transpose(0, 1)

    @torch.no_grad()
    def _argmax_slots(self) -> torch.Tensor:
        """Winner slots of an unfrozen layer (argmax of the logits, uint8), recomputed on every
        call: the logits change without a version bump when an optimizer writes them through
        raw pointers (FusedAdam) or a captured training step is replayed.  When the winners
        equal the previous call's, that tensor object is returned, so the packed tables keyed
        on it stay cached across eval calls (one device comparison, which synchronises; under
        graph capture the fresh winners are returned as they are)."""
        src = self.weights
        w = src.argmax(-1).to(dtype=torch.uint8, device=src.device)
        if src.device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            return w
        prev = getattr(self, "_argmax_cache", None)
        if prev is not None and prev.shape == w.shape and prev.device == w.device \
                and torch.equal(prev, w):
            return prev
        self._argmax_cache = w
        return w

    @torch.no_grad()
    def packed_tables(self, w: torch.Tensor):
        """(ia, ib, gate, order) of the packed layer for the winner slots ``w``: the two input
        rows and the opcode of every neuron's winner slot (int32, int32, uint8; a winner slot
        outside [0, num_gates) or an input outside [0, in_dim) gets row in_dim, which the kernel
        evaluates as zero words, as the slot-indirect evaluation does), and the order in which
        the kernel evaluates the neurons: sorted by the later of their two inputs in the
        depth-first order of the input rows (plan.locality_order over the edges (ia, ib)), so
        that neurons adjacent in the order mostly share an input row; None (neuron order)
        when the input rows are read more than _PACKED_CHAIN_MAX_DEGREE times on average.  Cached until the
        winners, the wiring or the opcodes change (weak references and versions)."""
        srcs = (w, self.indices, self.gate_sequence)
        key = tuple((t._version, t.device) for t in srcs)
        hit = getattr(self, "_packed_key", None)
        if hit is not None and hit[1] == key and all(r() is t for r, t in zip(hit[0], srcs)):
            return self._packed_tables
        rows = torch.arange(self.out_dim, device=w.device)
        s = w.to(torch.long)
        ok_s = s < self.num_gates
        sc = torch.where(ok_s, s, torch.zeros_like(s))
        a = self.indices[0, rows, sc]
        b = self.indices[1, rows, sc]
        ok = ok_s & (a >= 0) & (a < self.in_dim) & (b >= 0) & (b < self.in_dim)
        bad = torch.full_like(a, self.in_dim)
        ia = torch.where(ok, a, bad).to(torch.int32).contiguous()
        ib = torch.where(ok, b, bad).to(torch.int32).contiguous()
        gate = self.gate_sequence[rows, sc].contiguous()
        order = None
        if 2 * self.out_dim <= _PACKED_CHAIN_MAX_DEGREE * self.in_dim:
            ga = torch.where(ok, a, torch.zeros_like(a))
            gb = torch.where(ok, b, torch.zeros_like(b))
            pos = torch.empty(self.in_dim, dtype=torch.long, device=w.device)
            pos[locality_order(ga, gb, self.in_dim)] = torch.arange(self.in_dim, device=w.device)
            later = torch.maximum(pos[ga], pos[gb])
            order = torch.sort(later * self.out_dim + rows).indices.to(torch.int32).contiguous()
        self._packed_tables = (ia, ib, gate, order)
        self._packed_key = (tuple(weakref.ref(t) for t in srcs), key)
        return self._packed_tables

    def extra_repr(self):
        return '{}, {}, {}'.format(self.in_dim, self.out_dim, 'train' if self.training else 'eval')

    # -- parameters and wiring (same draws, in the same order, as the reference) ----------------------------------------

    def init_weights(self, residual_init: bool = False):
        """N(0, 1) logits, or the residual init: log(9 (G - 1)) on slot 3, zeros elsewhere
        (:135-147)."""
        rows = getattr(self, 'c_out', self.out_dim)
        if residual_init:
            logits = torch.zeros((rows, self.num_gates))
            logits[:, 3] = float(np.log(9 * (self.num_gates - 1)))
        else:
            logits = torch.randn([rows, self.num_gates])
        self.weights = torch.nn.parameter.Parameter(logits)

    def init_gate_sequence(self):
        """gate_sequence[row, g] = g & 15 (:149-158)."""
        rows = self.c_out if hasattr(self, "c_out") else self.out_dim
        seq = torch.arange(self.num_gates, device=self.weights.device, dtype=torch.int64) & 15
        self.register_buffer('gate_sequence', seq.unsqueeze(0).repeat(rows, 1).to(torch.uint8))

    def get_connections(self, device='cuda'):
        """Input pairs per neuron and slot (:160-182).  'random' gives every slot column its
        own pair of random permutations over 2*out_dim targets folded onto the inputs;
        'original' draws one pair per neuron and repeats it over the slots."""
        assert self.out_dim * 2 >= self.in_dim, (
            'The number of neurons ({}) must not be smaller than half of the number of inputs '
            '({}) because otherwise not all inputs could be used or considered.'.format(
                self.out_dim, self.in_dim))
        g = self.num_gates
        if self.connections == 'random':
            targets = torch.argsort(torch.rand(2 * self.out_dim, g, device=device), dim=0) % self.in_dim
            relabel = torch.argsort(torch.rand(self.in_dim, g, device=device), dim=0)
            pairs = torch.gather(relabel, 0, targets).view(2, self.out_dim, g)
        elif self.connections == 'original':
            flat = torch.randperm(2 * self.out_dim) % self.in_dim
            flat = torch.randperm(self.in_dim)[flat]
            pairs = flat.unsqueeze(-1).expand(*flat.shape, g).reshape(2, self.out_dim, g)
        else:
            raise NotImplementedError(f'self.connections: "{self.connections}" not implemented.')
        self.register_buffer('indices', pairs.to(torch.int64).to(device).contiguous())

    def _set_or_register_buffer(self, name: str, tensor: torch.Tensor) -> None:
        if name in self._buffers:
            self._buffers[name] = tensor
        else:
            self.register_buffer(name, tensor)

    def refresh_backward_index(self, changed_rows: torch.Tensor | None = None) -> None:
        """Rebuild the inverse index (:184-274): for every input, the (neuron, code) uses of
        it, with code g for operand a of slot g and -(g+1) for operand b, grouped by input in
        CSR form.  Rows are rebuilt in full (a stable sort, so the order inside a row is
        canonical); an empty `changed_rows` leaves the index as it is, as in the reference."""
        if not hasattr(self, "indices") or self.indices.ndim != 3:
            return
        if changed_rows is not None and "given_x_indices_of_y_start" in self._buffers:
            if torch.as_tensor(changed_rows).numel() == 0:
                return
        starts, ys, codes = _dl.inverse_index(self.indices[0], self.indices[1], self.in_dim)
        self._set_or_register_buffer("given_x_indices_of_y_start", starts)
        self._set_or_register_buffer("given_x_indices_of_y", ys)
        self._set_or_register_buffer("given_x_indices_of_gate", codes)
        self._plan = None

    def run_plan(self) -> RunPlan:
        """The connection-run plan for the current `indices`, rebuilt after any change: the
        cache holds a weak reference to the indices tensor and its version, so an in-place
        rewiring or a new tensor (even one at a recycled address) rebuilds it.  An in-place
        rewiring of few neurons (plan.REORDER_FRACTION of them since the last full build)
        keeps the previous processing order of the inputs, which skips the plan's host round
        trip; the rest of the plan is rebuilt from the new wiring."""
        ind = self.indices
        hit = self._plan_key
        if (self._plan is None or hit is None or hit[0]() is not ind
                or hit[1] != (ind._version, ind.device)):
            old, order, stale = self._plan, None, 0
            if (old is not None and hit is not None and hit[0]() is ind
                    and old.src_indices is not None and old.src_indices.shape == ind.shape
                    and old.src_indices.device == ind.device):
                changed = int((old.src_indices != ind).any(0).any(-1).sum())
                if old.stale + changed <= REORDER_FRACTION * ind.shape[1]:
                    order, stale = old.row_order, old.stale + changed
            self._plan = build_run_plan(ind, self.in_dim, row_order=order)
            self._plan.stale = stale
            self._plan_key = (weakref.ref(ind), (ind._version, ind.device))
        return self._plan

    # -- rewiring, entropy, freezing ----------------------------------------------------------------------------------

    @torch.no_grad()
    def resample_connections(self, converged_rows, threshold_high: float = 0.95,
                             threshold_low: float = 0.0, update_gate=True,
                             keep_strong_weights=True):
        """Re-draw logits, opcodes and wiring of the selected rows (:282-348): rows whose top
        probability is below `threshold_low` are re-drawn in full; rows above
        `threshold_high` keep their winning slot and re-draw the others."""
        device = self.weights.device
        num_rows = self.weights.shape[0]
        assert len(converged_rows.shape) == 1
        selected = torch.zeros(num_rows, device=device, dtype=torch.bool)
        selected[converged_rows.detach().clone().to(device)] = True
        probs = torch.nn.functional.softmax(self.weights, dim=-1)
        row_max, row_argmax = probs.max(dim=1)
        strong_mask = (row_max > threshold_high) & selected
        weak_mask = (row_max < threshold_low) & selected
        n_strong = int(strong_mask.sum().item())
        n_weak = int(weak_mask.sum().item())
        gate_pool = torch.arange(16, device=device, dtype=torch.uint8)
        if n_weak:
            self.weights[weak_mask] = torch.randn((n_weak, self.num_gates), device=device)
            if update_gate:
                pick = torch.randint(0, len(gate_pool), (n_weak, self.num_gates), device=device)
                self.gate_sequence[weak_mask] = gate_pool[pick]
            self.update_indices_weak(n_weak, weak_mask)
        if n_strong:
            refill = torch.zeros_like(self.weights, dtype=torch.bool, device=device)
            refill[strong_mask] = True
            strong_rows = strong_mask.nonzero(as_tuple=False).squeeze(-1)
            keep = row_argmax[strong_rows]
            refill[strong_rows, keep] = False
            kept_p = row_max[strong_mask].clamp(min=1e-6, max=1 - 1e-6)
            self.weights[strong_mask] = 0.0
            if keep_strong_weights:
                self.weights[strong_rows, keep] = torch.log(kept_p * (self.num_gates - 1) / (1 - kept_p))
            else:
                self.weights[strong_rows, keep] = float(np.log(9 * (self.num_gates - 1)))
            n_fill = int(refill.sum().item())
            if update_gate and n_fill > 0:
                pick = torch.randint(0, len(gate_pool), (n_fill,), device=device)
                self.gate_sequence[refill] = gate_pool[pick]
            self.update_indices_strong(refill, n_fill)
        if n_weak or n_strong:
            changed = torch.nonzero(weak_mask | strong_mask, as_tuple=False).flatten()
            self.refresh_backward_index(changed)
        return weak_mask, strong_mask

    @torch.no_grad()
    def update_indices_weak(self, n_weak, weak_mask):
        """New uniform input pairs for every slot of the weak rows (:350-359)."""
        device = self.weights.device
        self.indices[0][weak_mask] = torch.randint(0, self.in_dim, (n_weak, self.num_gates),
                                                   device=device, dtype=torch.int64)
        self.indices[1][weak_mask] = torch.randint(0, self.in_dim, (n_weak, self.num_gates),
                                                   device=device, dtype=torch.int64)

    @torch.no_grad()
    def update_indices_strong(self, mask2d, num_to_fill):
        """New uniform input pairs for the refilled slots of the strong rows (:361-368)."""
        device = self.weights.device
        self.indices[0][mask2d] = torch.randint(0, self.in_dim, (num_to_fill,), device=device,
                                                dtype=torch.int64)
        self.indices[1][mask2d] = torch.randint(0, self.in_dim, (num_to_fill,), device=device,
                                                dtype=torch.int64)

    @torch.no_grad()
    def weights_entropy(self, dim: int = -1) -> torch.Tensor:
        """Entropy of the gate distribution per row divided by log(G) (:370-385)."""
        log_p = torch.log_softmax(self.weights, dim=dim)
        return -(log_p.exp() * log_p).sum(dim=dim) / self.log_k

    def freeze(self):
        """Fix every neuron to its argmax slot (:387-394)."""
        self.weights.requires_grad = False
        self.register_buffer("w", self.weights.argmax(-1).to(dtype=torch.uint8,
                                                              device=self.weights.device))
        self.is_frozen = True

    def unfreeze(self):
        self.weights.requires_grad = True
        self.is_frozen = False

    @torch.no_grad()
    def connected_neurons(self, y_flag: torch.Tensor, const_gates=None, trivial_gates_a=None,
                          trivial_gates_b=None, device=None):
        """Inputs feeding the active, non-trivial outputs (:400-444).  Returns (x_flag,
        y_flag); y_flag is updated in place as in the reference."""
        assert y_flag.shape == (self.out_dim,), \
            f'y_flag shape mismatch: {y_flag.shape}, should be {self.out_dim}'
        device = device if device is not None else y_flag.device
        const_gates = torch.tensor([0, 15], device=device) if const_gates is None else const_gates
        trivial_gates_a = torch.tensor([3, 12], device=device) if trivial_gates_a is None else trivial_gates_a
        trivial_gates_b = torch.tensor([5, 10], device=device) if trivial_gates_b is None else trivial_gates_b
        x_flag = torch.zeros(self.in_dim, dtype=torch.bool, device=device)
        w = getattr(self, 'w', None)
        w = (self.weights.argmax(-1) if w is None else w).to(torch.long)
        pair = torch.gather(self.indices, 2, w.view(1, -1, 1).expand(2, -1, 1)).squeeze(-1)
        g = torch.gather(self.gate_sequence, 1, w.unsqueeze(-1)).squeeze(-1)
        is_const = torch.isin(g, const_gates.to(g.device))
        only_a = torch.isin(g, trivial_gates_a.to(g.device))
        only_b = torch.isin(g, trivial_gates_b.to(g.device))
        uses_a = ~is_const & ~only_b
        uses_b = ~is_const & ~only_a
        y_flag[is_const] = False
        used = torch.unique(torch.cat((pair[0][y_flag & uses_a], pair[1][y_flag & uses_b])))
        x_flag[used] = True
        y_flag[only_a | only_b] = False
        return x_flag, y_flag


class ConvLayerCudaFunction(torch.autograd.Function):
    """Autograd bridge for the conv kernels, argument list as in
    compactlogic/compactlogic.py:838-867: (x, offsets_ch, offsets_h, offsets_w, w,
    gate_sequence, stride, pad, ks) with ``w`` the gate probabilities."""

    @staticmethod
    def forward(ctx, x, offsets_ch, offsets_h, offsets_w, w, gate_sequence, stride, pad, ks):
        y = timing.timed(_conv_name("cl_conv_forward", x, w), lambda: _cl.forward(
            x, offsets_ch, offsets_h, offsets_w, w, gate_sequence, stride, pad, ks))
        ctx.save_for_backward(x, offsets_ch, offsets_h, offsets_w, w, gate_sequence)
        ctx.stride = stride
        ctx.pad = pad
        ctx.index = (_cl.inverse_index(offsets_ch, offsets_h, offsets_w, x.shape[1], stride)
                     if ctx.needs_input_grad[0] else None)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, offsets_ch, offsets_h, offsets_w, w, gate_sequence = ctx.saved_tensors
        grad_y = grad_y.contiguous()
        grad_x = grad_w = None
        if ctx.needs_input_grad[0]:
            grad_x = timing.timed(_conv_name("cl_conv_backward_x", x, w), lambda: _cl.backward_x(
                x, offsets_ch, offsets_h, offsets_w, w, gate_sequence, grad_y, ctx.stride, ctx.pad,
                ctx.index))
        if ctx.needs_input_grad[4]:
            grad_w = timing.timed(_conv_name("cl_conv_backward_w", x, w), lambda: _cl.backward_w(
                x, offsets_ch, offsets_h, offsets_w, gate_sequence, grad_y, ctx.stride))
        return grad_x, None, None, None, grad_w, None, None, None, None


class ConvLayerSoftmaxFunction(torch.autograd.Function):
    """ConvLayerCudaFunction with the softmax over the gate logits folded in: the forward
    computes the probabilities once, and the weight-gradient kernel applies the softmax
    backward in its final reduction, returning the gradient of the logits."""

    @staticmethod
    def forward(ctx, x, offsets_ch, offsets_h, offsets_w, logits, gate_sequence, stride, pad, ks):
        probs = torch.softmax(logits, dim=-1).contiguous()
        y = timing.timed(_conv_name("cl_conv_forward", x, probs), lambda: _cl.forward(
            x, offsets_ch, offsets_h, offsets_w, probs, gate_sequence, stride, pad, ks))
        ctx.save_for_backward(x, offsets_ch, offsets_h, offsets_w, probs, gate_sequence)
        ctx.stride = stride
        ctx.pad = pad
        ctx.index = (_cl.inverse_index(offsets_ch, offsets_h, offsets_w, x.shape[1], stride)
                     if ctx.needs_input_grad[0] else None)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, offsets_ch, offsets_h, offsets_w, probs, gate_sequence = ctx.saved_tensors
        grad_y = grad_y.contiguous()
        grad_x = grad_w = None
        if ctx.needs_input_grad[0]:
            grad_x = timing.timed(_conv_name("cl_conv_backward_x", x, probs), lambda: _cl.backward_x(
                x, offsets_ch, offsets_h, offsets_w, probs, gate_sequence, grad_y, ctx.stride,
                ctx.pad, ctx.index))
        if ctx.needs_input_grad[4]:
            grad_w = timing.timed(_conv_name("cl_conv_backward_w", x, probs), lambda: _cl.backward_w(
                x, offsets_ch, offsets_h, offsets_w, gate_sequence, grad_y, ctx.stride, probs))
        return grad_x, None, None, None, grad_w, None, None, None, None


class ConvLayerWindowFunction(torch.autograd.Function):
    """ConvLayer training step through the window path (every output channel reads one input
    channel): the softmax and the collapse of all slots into per-channel window coefficients
    run in one prep kernel; the forward evaluates every output channel of an input channel
    from one load of each window; the backward gives the input gradient per (sample, input
    channel) plane and the gradient of the logits from per-chunk window moments."""

    @staticmethod
    def forward(ctx, x, logits, gate_sequence, plan, stride: int, out_hw: tuple):
        for t, nm in ((x, "x"), (gate_sequence, "gate_sequence"), (plan.slot_win, "slot_win")):
            _dl._check(t, nm)
        _dl._same_device(x, logits, gate_sequence, plan.slot_win, plan.grp_ptr, plan.chan_order)
        if logits.dtype != x.dtype:
            raise RuntimeError("logits must have the dtype of x")
        n, cin, h, w = x.shape
        cout, g = logits.shape
        if (plan.grp_ptr.numel() != cin + 1 or plan.chan_order.numel() != cout
                or tuple(plan.slot_win.shape) != (cout, g)
                or tuple(gate_sequence.shape) != (cout, g)):
            raise RuntimeError("window plan, gate_sequence and logits do not match the input")
        ho, wo = out_hw
        code = _dl.dtype_code(x)
        stream = _dl.stream_of(x)
        logits = logits.contiguous()
        probs = torch.empty_like(logits)
        coef = torch.empty((cout, plan.width), dtype=x.dtype, device=x.device)
        y = torch.empty((n, cout, ho, wo), dtype=x.dtype, device=x.device)
        tag = f"[{cin}x{h}x{w}->{cout}]"
        geo = (stride, ho, wo, plan.oy0, plan.ox0, plan.kw)
        with torch.cuda.device(x.device):
            timing.timed("cl_conv_window_prep" + tag, lambda: _capi.call(
                "cl_conv_window_prep", code, logits.data_ptr(), 1, gate_sequence.data_ptr(),
                plan.slot_win.data_ptr(), probs.data_ptr(), coef.data_ptr(), cout, g, plan.kw,
                stream))
            timing.timed("cl_conv_window_forward" + tag, lambda: _capi.call(
                "cl_conv_window_forward", code, x.data_ptr(), coef.data_ptr(),
                plan.grp_ptr.data_ptr(), plan.chan_order.data_ptr(), y.data_ptr(), n, cin, h, w,
                cout, *geo, stream))
        ctx.save_for_backward(x, coef, probs, gate_sequence)
        ctx.plan, ctx.geo, ctx.tag = plan, geo, tag
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, coef, probs, gate_sequence = ctx.saved_tensors
        plan, geo, tag = ctx.plan, ctx.geo, ctx.tag
        grad_y = grad_y.contiguous()
        n, cin, h, w = x.shape
        cout, g = probs.shape
        code = _dl.dtype_code(x)
        stream = _dl.stream_of(x)
        grad_x = grad_w = None
        with torch.cuda.device(x.device):
            if ctx.needs_input_grad[0]:
                grad_x = torch.empty_like(x)
                timing.timed("cl_conv_window_backward_x" + tag, lambda: _capi.call(
                    "cl_conv_window_backward_x", code, x.data_ptr(), grad_y.data_ptr(),
                    coef.data_ptr(), plan.grp_ptr.data_ptr(), plan.chan_order.data_ptr(),
                    grad_x.data_ptr(), n, cin, h, w, cout, *geo, stream))
            if ctx.needs_input_grad[1]:
                nq = ctypes.c_int64(0)
                _capi.call("cl_conv_window_chunks", n, cin, plan.max_group, geo[1] * geo[2],
                           ctypes.byref(nq))
                moments = torch.empty((nq.value, cout, plan.width), dtype=x.dtype, device=x.device)
                grad_w = torch.empty_like(probs)
                timing.timed("cl_conv_window_moments" + tag, lambda: _capi.call(
                    "cl_conv_window_moments", code, x.data_ptr(), grad_y.data_ptr(),
                    plan.grp_ptr.data_ptr(), plan.chan_order.data_ptr(), moments.data_ptr(),
                    nq.value, plan.max_group, n, cin, h, w, cout, *geo, stream))
                timing.timed("cl_conv_window_finalize" + tag, lambda: _capi.call(
                    "cl_conv_window_finalize", code, moments.data_ptr(), nq.value,
                    gate_sequence.data_ptr(), plan.slot_win.data_ptr(), probs.data_ptr(),
                    grad_w.data_ptr(), cout, g, plan.kw, stream))
        return grad_x, grad_w, None, None, None, None


def _conv_name(entry: str, x: torch.Tensor, w: torch.Tensor) -> str:
    return f"{entry}[{x.shape[1]}x{x.shape[2]}x{x.shape[3]}->{w.shape[0]}]"


class ConvLayer(LogicLayer):
    """Convolutional logic layer (compactlogic/compactlogic.py:514-835).

    ``in_shape`` = (c_in, h, w) of the unpadded input; every output channel has ``num_gates``
    candidate slots, each reading two taps (channel, dh, dw) of the receptive field of size
    ``ks``; taps outside the input plane read 0.  ``num_chn`` selects the channel sampling:
    0 uniform, 1 channel c mod c_in for output channel c, > 1 groups of ``num_chn`` input
    channels.  Buffers ``offsets_ch`` int32, ``offsets_h`` / ``offsets_w`` int8, all
    [2, c_out, G], hold the spatial offsets already shifted by ``-padding``; ``in_dim`` counts
    the padded plane and ``out_dim`` = c_out * h_out * w_out, as in the reference.
    """

    def __init__(self, in_shape, padding: int, c_out: int, ks: int, stride: int,
                 num_chn: int = 1, **kwargs):
        self.padding = padding
        self.c_in = in_shape[0]
        self.h_in = in_shape[1] + 2 * padding
        self.w_in = in_shape[2] + 2 * padding
        self.in_dim = int(np.prod((self.c_in, self.h_in, self.w_in)))
        self.in_shape = tuple(in_shape)
        self.c_out = c_out
        self.ks = ks
        self.stride = stride
        self.h_out = (self.h_in - self.ks) // self.stride + 1
        self.w_out = (self.w_in - self.ks) // self.stride + 1
        self.out_shape = (self.c_out, self.h_out, self.w_out)
        self.out_dim = int(np.prod(self.out_shape))
        self.chn_grp = num_chn if num_chn <= 1 else (self.c_in // num_chn)
        super().__init__(self.in_dim, self.out_dim, **kwargs)
        self._packed_key = None
        self._packed_tables = None
        self._packed_order = None

    _weak_caches = LogicLayer._weak_caches + ("_packed_order",)

    def forward_cuda(self, x):
        """x [N, c_in, h, w] -> [N, c_out, h_out, w_out] (:598-626)."""
        assert tuple(x.shape[1:]) == self.in_shape, f'input shape mismatch {x.shape}, {self.in_shape}'
        assert x.ndim == 4, x.ndim
        x = x.contiguous()
        if self.weights.dtype == x.dtype and self.num_gates <= 64:
            plan = self.window_plan(x)
            if plan is not None:
                return ConvLayerWindowFunction.apply(x, self.weights, self.gate_sequence, plan,
                                                     self.stride, (self.h_out, self.w_out))
            return ConvLayerSoftmaxFunction.apply(
                x, self.offsets_ch, self.offsets_h, self.offsets_w, self.weights,
                self.gate_sequence, self.stride, self.padding, self.ks)
        w = torch.nn.functional.softmax(self.weights, dim=-1).to(x.dtype)
        return ConvLayerCudaFunction.apply(
            x, self.offsets_ch, self.offsets_h, self.offsets_w, w, self.gate_sequence,
            self.stride, self.padding, self.ks)

    def window_plan(self, x: torch.Tensor):
        """The window-path tables when this layer qualifies (each output channel reads one
        input channel, taps within 3 x 3, at most 1024 output positions and an input plane of
        at most 64 KiB), else None."""
        c_in, h, w = self.in_shape
        if self.h_out * self.w_out > 1024 or h * w * x.element_size() > 65536:
            return None
        return _cl.window_plan(self.offsets_ch, self.offsets_h, self.offsets_w, c_in)

    @torch.no_grad()
    def forward_cuda_eval(self, x):
        """Discrete conv with the argmax slot per output channel (:628-640).  A
        PackBitsTensor (rows = the c_in * h * w input features in NCHW order) is evaluated
        bitwise and updated in place; its rows become the c_out * h_out * w_out outputs."""
        assert self.is_frozen or not self.training
        w = getattr(self, "w", None)
        if w is None:
            w = self._argmax_slots()
        if isinstance(x, PackBitsTensor):
            ia, ib, gate = self.packed_tables(w)
            order = self.packed_order(w)
            assert x.t.shape[0] == int(np.prod(self.in_shape)), (x.t.shape, self.in_shape)
            x.t = timing.timed(f"cl_eval_packed_indexed[{x.t.shape[0]}->{ia.numel()}]",
                               lambda: _cl.eval_packed_indexed(x.t, ia, ib, gate, order))
            return x
        return _cl.eval(x.contiguous(), self.offsets_ch, self.offsets_h, self.offsets_w, w,
                        self.gate_sequence, self.stride, self.padding, self.ks)

    @torch.no_grad()
    def packed_tables(self, w: torch.Tensor):
        """(ia, ib, gate) per output feature (c, oy, ox) for the winner slots ``w``: the
        flattened NCHW input feature of each tap, -1 outside the plane (compiler/extract.py:
        101-174), and the opcode.  Cached until the offsets, opcodes or winners change: the
        cache holds weak references to those tensors and their versions, so a new tensor at a
        recycled address never hits it."""
        srcs = (w, self.offsets_ch, self.offsets_h, self.offsets_w, self.gate_sequence)
        key = tuple(t._version for t in srcs)
        hit = self._packed_key
        if hit is not None and hit[1] == key and all(r() is t for r, t in zip(hit[0], srcs)):
            return self._packed_tables
        dev = w.device
        c_in, h, wd = self.in_shape
        rows = torch.arange(self.c_out, device=dev)
        slot = w.to(torch.long)
        oy = torch.arange(self.h_out, device=dev).view(1, -1, 1) * self.stride
        ox = torch.arange(self.w_out, device=dev).view(1, 1, -1) * self.stride
        tables = []
        for side in (0, 1):
            ch = self.offsets_ch[side, rows, slot].to(torch.long).view(-1, 1, 1)
            iy = oy + self.offsets_h[side, rows, slot].to(torch.long).view(-1, 1, 1)
            ix = ox + self.offsets_w[side, rows, slot].to(torch.long).view(-1, 1, 1)
            inside = (iy >= 0) & (iy < h) & (ix >= 0) & (ix < wd)
            feat = (ch * h + iy) * wd + ix
            tables.append(torch.where(inside, feat, torch.full_like(feat, -1))
                          .reshape(-1).to(torch.int32).contiguous())
        gate = (self.gate_sequence[rows, slot].view(-1, 1)
                .expand(self.c_out, self.h_out * self.w_out).reshape(-1).contiguous())
        self._packed_tables = (tables[0], tables[1], gate)
        self._packed_order = None
        self._packed_key = (tuple(weakref.ref(t) for t in srcs), key)
        return self._packed_tables

    def packed_order(self, w: torch.Tensor) -> torch.Tensor:
        """Order in which the packed kernel evaluates the output features (int32): the output
        channels sorted by the input channel of their winner slot's first tap, each channel's
        positions in order.  The channels reading one input channel then run together, and
        the rows of that channel they all gather stay cache resident.  Cached with the
        tables."""
        self.packed_tables(w)
        if self._packed_order is None:
            dev = w.device
            rows = torch.arange(self.c_out, device=dev)
            ch = self.offsets_ch[0, rows, w.to(torch.long)].to(torch.long)
            chans = torch.sort(ch * self.c_out + rows).values % self.c_out
            hw = self.h_out * self.w_out
            pos = torch.arange(hw, device=dev)
            self._packed_order = (chans.view(-1, 1) * hw + pos.view(1, -1)).reshape(-1) \
                .to(torch.int32).contiguous()
        return self._packed_order

    def get_connections(self, device='cuda'):
        """Sample the two taps of every slot (:642-699), in the reference's draw order."""
        shape = (2, self.c_out, self.num_gates)
        if self.chn_grp > 1:
            assert self.chn_grp <= self.c_in and self.chn_grp <= self.c_out
            offsets_h = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
            offsets_w = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
            per_group = self.c_in // self.chn_grp
            sizes = torch.full((self.chn_grp,), per_group, device=device)
            sizes[:self.c_in % self.chn_grp] += 1
            starts = torch.cat([torch.zeros(1, device=device), sizes.cumsum(0)]).to(torch.int32)
            channels = torch.arange(self.c_in, device=device, dtype=torch.int32)
            out_per_group = self.c_out // self.chn_grp
            group_of = torch.clamp(torch.arange(self.c_out, device=device, dtype=torch.int32)
                                   // out_per_group, 0, self.chn_grp - 1)
            offsets_ch = torch.empty(shape, device=device, dtype=torch.int32)
            for gid in range(self.chn_grp):
                members = channels[starts[gid]:starts[gid + 1]]
                rows = (group_of == gid).nonzero(as_tuple=True)[0]
                if rows.numel() > 0:
                    k = members.numel()
                    offsets_ch[0, rows] = members[torch.randint(0, k, (rows.numel(), self.num_gates), device=device)]
                    offsets_ch[1, rows] = members[torch.randint(0, k, (rows.numel(), self.num_gates), device=device)]
        elif self.chn_grp == 1:
            assert self.ks > 1
            offsets_ch = torch.arange(0, self.c_out, device=device, dtype=torch.int32) % self.c_in
            offsets_ch = offsets_ch.unsqueeze(-1).expand(2, -1, self.num_gates)
            offsets_h = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
            offsets_w = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
        else:
            offsets_ch = torch.randint(0, self.c_in, size=shape, device=device, dtype=torch.int32)
            offsets_h = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
            offsets_w = torch.randint(0, self.ks, size=shape, device=device, dtype=torch.int8)
        offsets_ch, offsets_h, offsets_w = self.resolve_conflicts(
            offsets_ch, offsets_h, offsets_w, self.ks, self.c_in)
        offsets_h -= self.padding
        offsets_w -= self.padding
        self.register_buffer("offsets_ch", offsets_ch.contiguous().to(device))
        self.register_buffer("offsets_h", offsets_h.contiguous().to(device))
        self.register_buffer("offsets_w", offsets_w.contiguous().to(device))

    @staticmethod
    def resolve_conflicts(offsets_ch, offsets_h, offsets_w, ks, c_in):
        """Re-draw operand b of every slot whose two taps coincide until none do (:700-743):
        its spatial offsets when ks > 1, its channel when ks == 1."""
        def clash():
            return ((offsets_ch[0] == offsets_ch[1]) & (offsets_h[0] == offsets_h[1])
                    & (offsets_w[0] == offsets_w[1]))
        conflict = clash()
        while conflict.any():
            num = conflict.sum()
            if ks > 1:
                offsets_h[1][conflict] = torch.randint(0, ks, size=(num,), device=offsets_h.device,
                                                       dtype=torch.int8)
                offsets_w[1][conflict] = torch.randint(0, ks, size=(num,), device=offsets_w.device,
                                                       dtype=torch.int8)
            elif ks == 1:
                offsets_ch[1][conflict] = torch.randint(0, c_in, size=(num,), device=offsets_ch.device,
                                                        dtype=torch.int32)
            conflict = clash()
        return offsets_ch, offsets_h, offsets_w

    @torch.no_grad()
    def update_indices_weak(self, n_weak, weak_mask):
        """New taps for every slot of the weak rows (:745-764): channels when ks == 1, else
        spatial offsets (shifted by -padding)."""
        device = self.weights.device
        size = (n_weak, self.num_gates)
        if self.ks == 1:
            self.offsets_ch[0][weak_mask] = torch.randint(0, self.c_in, size=size, device=device, dtype=torch.int32)
            self.offsets_ch[1][weak_mask] = torch.randint(0, self.c_in, size=size, device=device, dtype=torch.int32)
        else:
            for t in (self.offsets_h[0], self.offsets_h[1], self.offsets_w[0], self.offsets_w[1]):
                t[weak_mask] = torch.randint(0, self.ks, size=size, device=device,
                                             dtype=torch.int8) - self.padding

    @torch.no_grad()
    def update_indices_strong(self, mask2d, num_to_fill):
        """New taps for the refilled slots of the strong rows (:766-778)."""
        device = self.weights.device
        if self.ks == 1:
            self.offsets_ch[0][mask2d] = torch.randint(0, self.c_in, size=(num_to_fill,), device=device, dtype=torch.int32)
            self.offsets_ch[1][mask2d] = torch.randint(0, self.c_in, size=(num_to_fill,), device=device, dtype=torch.int32)
        else:
            for t in (self.offsets_h[0], self.offsets_h[1], self.offsets_w[0], self.offsets_w[1]):
                t[mask2d] = torch.randint(0, self.ks, size=(num_to_fill,), device=device,
                                          dtype=torch.int8) - self.padding

    def extra_repr(self):
        return 'in_shape={}, out_shape={}, pad={}, kernel_size={}, stride={}, num_chn={}, {}'.format(
            self.in_shape, self.out_shape, self.padding, self.ks, self.stride,
            self.chn_grp if self.chn_grp <= 1 else (self.c_in // self.chn_grp),
            'train' if self.training else 'eval')

    @torch.no_grad()
    def connected_neurons(self, y_flag: torch.Tensor, const_gates=None, trivial_gates=None,
                          device=None):
        """Input pixels feeding the active, non-trivial outputs (:793-835).  Returns (x_flag
        [c_in, h, w], y_flag [c_out, h_out, w_out]); y_flag is updated in place."""
        assert tuple(y_flag.shape) == self.out_shape, \
            f'y_flag shape mismatch: {y_flag.shape}, should be {self.out_shape}'
        device = device if device is not None else y_flag.device
        const_gates = torch.tensor([0, 15], device=device) if const_gates is None else const_gates
        trivial_gates = (torch.tensor([3, 5, 10, 12], device=device) if trivial_gates is None
                         else trivial_gates)
        x_flag = torch.zeros(self.in_shape, dtype=torch.bool, device=device)
        w = getattr(self, 'w', None)
        w = (self.weights.argmax(-1) if w is None else w).to(torch.long)
        idx = w.view(1, -1, 1).expand(2, -1, 1)
        och = torch.gather(self.offsets_ch, 2, idx).squeeze(-1).to(torch.long)
        oh = torch.gather(self.offsets_h, 2, idx).squeeze(-1).to(torch.long)
        ow = torch.gather(self.offsets_w, 2, idx).squeeze(-1).to(torch.long)
        g = torch.gather(self.gate_sequence, 1, w.unsqueeze(-1)).squeeze(-1)
        is_const = torch.isin(g, const_gates.to(g.device))
        is_trivial = torch.isin(g, trivial_gates.to(g.device))
        y_flag[is_const] = False
        uses = (~is_const & (g != 5) & (g != 10), ~is_const & (g != 3) & (g != 12))
        c, oy, ox = torch.nonzero(y_flag, as_tuple=True)
        _, h, wd = self.in_shape
        for side in (0, 1):
            keep = uses[side][c]
            cc, yy, xx = c[keep], oy[keep], ox[keep]
            iy = yy * self.stride + oh[side][cc]
            ix = xx * self.stride + ow[side][cc]
            inside = (iy >= 0) & (iy < h) & (ix >= 0) & (ix < wd)
            x_flag[och[side][cc][inside], iy[inside], ix[inside]] = True
        y_flag[is_trivial] = False
        return x_flag, y_flag


class GroupSumCrossEntropyFunction(torch.autograd.Function):
    """cross_entropy(GroupSum(k, tau)(x), labels) with the mean over counted samples, fused:
    the group sums, the softmax and the loss in three launches and the input gradient in one,
    instead of GroupSum's two plus torch's log-softmax / NLL kernels each way.  No counterpart
    in the reference (its training loops call torch's cross_entropy on GroupSum's output,
    compactlogic/compactlogic.py:450-468); the result is the same function.  Returns
    (loss, scores); the scores are not differentiable through this function."""

    @staticmethod
    def forward(ctx, x, labels, k, tau, ignore_index):
        if x.device.type != "cuda" or labels.device != x.device:
            raise RuntimeError("GroupSum cross-entropy needs x and labels on the same HIP device")
        if x.dim() != 2:
            raise RuntimeError("GroupSum expects a 2-D [batch, features] input")
        batch, feats = x.shape
        if labels.dtype != torch.int64 or labels.shape != (batch,):
            raise RuntimeError(f"labels must be int64 of shape ({batch},)")
        labels = labels.contiguous()
        sb, sf = x.stride()
        if sb < 0 or sf < 0 or (batch > 1 and feats > 1 and (sb == 0 or sf == 0)):
            x = x.contiguous()
            sb, sf = x.stride()
        out = torch.empty((batch, k), dtype=x.dtype, device=x.device)
        probs = torch.empty((batch, k), dtype=x.dtype, device=x.device)
        loss = torch.empty((), dtype=x.dtype, device=x.device)
        count = torch.empty((), dtype=x.dtype, device=x.device)  # samples in the mean
        need = ctypes.c_int64(0)
        _capi.call("cl_group_sum_cross_entropy_workspace_size", _dl.dtype_code(x), batch, feats,
                   k, ctypes.byref(need))
        ws = torch.empty(need.value, dtype=torch.uint8, device=x.device) if need.value else None
        with torch.cuda.device(x.device):
            timing.timed("cl_group_sum_cross_entropy_forward", lambda: _capi.call(
                "cl_group_sum_cross_entropy_forward", _dl.dtype_code(x), x.data_ptr(), batch,
                feats, sb, sf, k, float(tau), labels.data_ptr(), int(ignore_index),
                out.data_ptr(), probs.data_ptr(), loss.data_ptr(), count.data_ptr(),
                _dl.ptr(ws), need.value, _dl.stream_of(x)))
        ctx.save_for_backward(probs, labels, count)
        ctx.k, ctx.tau, ctx.ignore_index = k, tau, int(ignore_index)
        ctx.shape = (batch, feats)
        ctx.batch_major = sb == 1 and sf != 1
        ctx.mark_non_differentiable(out)
        ctx.set_materialize_grads(False)  # the scores' gradient is never used: no zero fill
        return loss, out

    @staticmethod
    def backward(ctx, grad_loss, _grad_out):
        if grad_loss is None:
            return None, None, None, None, None
        probs, labels, count = ctx.saved_tensors
        grad_loss = grad_loss.to(probs.dtype).contiguous()
        batch, feats = ctx.shape
        if ctx.batch_major:
            grad_x = torch.empty((feats, batch), dtype=probs.dtype, device=probs.device).t()
        else:
            grad_x = torch.empty((batch, feats), dtype=probs.dtype, device=probs.device)
        sb, sf = grad_x.stride()
        with torch.cuda.device(probs.device):
            timing.timed("cl_group_sum_cross_entropy_backward", lambda: _capi.call(
                "cl_group_sum_cross_entropy_backward", _dl.dtype_code(probs), probs.data_ptr(),
                labels.data_ptr(), ctx.ignore_index, grad_loss.data_ptr(), count.data_ptr(),
                batch, feats, ctx.k, float(ctx.tau),
                grad_x.data_ptr(), sb, sf, _dl.stream_of(probs)))
        return grad_x, None, None, None, None


class GroupSum(torch.nn.Module):
    """k class scores from the summed outputs of k equal feature groups, divided by tau
    (compactlogic/compactlogic.py:450-468).  A PackBitsTensor gives int32 per-class counts
    (difflogic.py:203-205)."""

    def __init__(self, k: int, tau: float = 1., device='cuda'):
        super().__init__()
        self.k = k
        self.tau = tau
        self.device = device

    def forward(self, x):
        """[..., features] -> [..., k] (any leading dims, as the reference's reshape-and-sum);
        features not divisible by k are summed as if zero-padded to the next multiple."""
        if isinstance(x, PackBitsTensor):
            return x.group_sum(self.k)
        if x.dtype == torch.float16:
            # half scores from fp32 sums (torch's half sum in the reference accumulates in
            # fp32 as well); the gradient is cast back by autograd
            return self(x.float()).to(torch.float16)
        if x.dim() == 2:
            return GroupSumFunction.apply(x, self.k, self.tau)
        if x.dim() == 0:
            raise RuntimeError("GroupSum needs an input with a feature dimension")
        lead = x.shape[:-1]
        out = GroupSumFunction.apply(x.reshape(-1, x.shape[-1]), self.k, self.tau)
        return out.reshape(*lead, self.k)

    def cross_entropy(self, x, labels, ignore_index: int = -100, return_scores: bool = False):
        """torch.nn.functional.cross_entropy(self(x), labels, ignore_index=ignore_index) in one
        fused op (mean over the samples whose label is not ignore_index); with return_scores,
        also the scores self(x) (not differentiable through this call)."""
        if isinstance(x, torch.Tensor) and x.dtype == torch.float16:
            loss, out = GroupSumCrossEntropyFunction.apply(x.float(), labels, self.k, self.tau,
                                                           ignore_index)
            loss, out = loss.to(torch.float16), out.to(torch.float16)
        else:
            loss, out = GroupSumCrossEntropyFunction.apply(x, labels, self.k, self.tau,
                                                           ignore_index)
        return (loss, out) if return_scores else loss

    def extra_repr(self):
        return 'k={}, tau={}'.format(self.k, self.tau)


class LogicGroupSumCrossEntropyFunction(torch.autograd.Function):
    """The classifier head of a training step, fused: a dense LogicLayer's training forward,
    GroupSum(k, tau) and the mean cross-entropy (cl_dense_group_sum_cross_entropy_forward /
    _backward).  The same function as GroupSumCrossEntropyFunction applied to
    LogicLayerRunsFunction's output, but the layer's output [out_dim, batch] and its gradient
    are never stored: the forward sums each tile of outputs by class, the backward reads one
    gradient row per class.  No counterpart in the reference (its training loops run the layer,
    GroupSum and torch's cross_entropy in turn: compactlogic/compactlogic.py:83-118, :450-468).
    Returns (loss, scores); the scores are not differentiable through this function."""

    @staticmethod
    def forward(ctx, x, w, gate_sequence, plan: RunPlan, softmax, labels, k, tau, ignore_index,
                forward_bytes, backward_bytes):
        _dl._check(x, "x")
        batch = x.shape[1]
        dev, code = x.device, _dl.dtype_code(x)
        w = w.contiguous()
        labels = labels.contiguous()
        probs = torch.empty_like(w) if softmax else None
        inv_coef = torch.empty((2 * plan.num_runs, 2), dtype=x.dtype, device=dev)
        scores = torch.empty((batch, k), dtype=x.dtype, device=dev)
        ce_probs = torch.empty((batch, k), dtype=x.dtype, device=dev)
        loss = torch.empty((), dtype=x.dtype, device=dev)
        count = torch.empty((), dtype=x.dtype, device=dev)
        ws = torch.empty(forward_bytes, dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            timing.timed(f"cl_dense_group_sum_cross_entropy_forward[{plan.in_dim}->{plan.out_dim}]",
                         lambda: _capi.call(
                "cl_dense_group_sum_cross_entropy_forward", code, x.data_ptr(), w.data_ptr(),
                int(softmax), gate_sequence.data_ptr(), plan.nab.data_ptr(),
                plan.inv_pos.data_ptr(), _dl.ptr(probs), inv_coef.data_ptr(), plan.in_dim,
                plan.out_dim, plan.num_runs, batch, plan.num_gates, k, float(tau),
                labels.data_ptr(), int(ignore_index), scores.data_ptr(), ce_probs.data_ptr(),
                loss.data_ptr(), count.data_ptr(), ws.data_ptr(), forward_bytes,
                _dl.stream_of(x)))
        ctx.save_for_backward(x, inv_coef, gate_sequence, probs, ce_probs, labels, count)
        ctx.plan, ctx.k, ctx.tau, ctx.ignore_index = plan, k, tau, int(ignore_index)
        ctx.backward_bytes = backward_bytes
        ctx.mark_non_differentiable(scores)
        ctx.set_materialize_grads(False)
        return loss, scores

    @staticmethod
    def backward(ctx, grad_loss, _grad_scores):
        if grad_loss is None:
            return (None,) * 11
        x, inv_coef, gate_sequence, probs, ce_probs, labels, count = ctx.saved_tensors
        plan: RunPlan = ctx.plan
        grad_loss = grad_loss.to(x.dtype).contiguous()
        batch = x.shape[1]
        grad_x = torch.empty_like(x)  # the row backward always writes it
        grad_w = (torch.empty((plan.out_dim, plan.num_gates), dtype=x.dtype, device=x.device)
                  if ctx.needs_input_grad[1] else None)
        ws = torch.empty(ctx.backward_bytes, dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            timing.timed(f"cl_dense_group_sum_cross_entropy_backward[{plan.in_dim}->{plan.out_dim}]",
                         lambda: _capi.call(
                "cl_dense_group_sum_cross_entropy_backward", _dl.dtype_code(x), x.data_ptr(),
                ce_probs.data_ptr(), labels.data_ptr(), ctx.ignore_index, grad_loss.data_ptr(),
                count.data_ptr(), ctx.k, float(ctx.tau), plan.slot_rec.data_ptr(),
                plan.inv_rec.data_ptr(), inv_coef.data_ptr(), gate_sequence.data_ptr(),
                _dl.ptr(probs), plan.run_ptr.data_ptr(), _dl.ptr(grad_w), grad_x.data_ptr(),
                plan.in_dim, plan.out_dim, plan.num_runs, batch, plan.num_gates, ws.data_ptr(),
                ctx.backward_bytes, _dl.stream_of(x)))
        return (grad_x if ctx.needs_input_grad[0] else None, grad_w) + (None,) * 9


def _head_workspace(layer: LogicLayer, x: torch.Tensor, k: int):
    """(forward, backward) workspace bytes of the fused classifier head for layer on x
    ([batch, in_dim]), or None when it does not apply."""
    if (type(layer) is not LogicLayer or not layer.training or getattr(layer, "is_frozen", False)
            or isinstance(x, PackBitsTensor) or x.device.type != "cuda" or x.dim() != 2
            or x.dtype not in (torch.float32, torch.float64) or layer.weights.dtype != x.dtype):
        return None
    # Not under HIP graph capture: a capture of the fused head ended the process in
    # torch's capture_end (cause not established); captured steps take the composition.
    if torch.cuda.is_current_stream_capturing():
        return None
    batch = x.shape[0]
    wide = 16 // x.element_size()
    if batch == 0 or batch % wide or batch > 64 * wide * 8:
        return None
    plan = layer.run_plan()
    if not plan.single_run or plan.num_gates > 16:
        return None
    fb, bb = ctypes.c_int64(), ctypes.c_int64()
    _capi.call("cl_dense_group_sum_cross_entropy_workspace_size", _dl.dtype_code(x),
               layer.out_dim, batch, int(k), ctypes.byref(fb), ctypes.byref(bb))
    return None if fb.value < 0 else (fb.value, bb.value)


def logic_group_sum_cross_entropy(layer: LogicLayer, group_sum: GroupSum, x, labels,
                                  ignore_index: int = -100, return_scores: bool = False):
    """group_sum.cross_entropy(layer(x), labels, ignore_index): the loss of a classifier whose
    last dense layer is `layer`, with the layer's output never stored (the fused head,
    LogicGroupSumCrossEntropyFunction).  Gradients flow to x and the layer's logits exactly as
    through the composition (equal up to the rounding of the class sums).  Where the fused
    head does not apply (a conv or frozen layer, eval mode, classes narrower than a forward
    tile, batches outside the row backward's range, or under HIP graph capture) this is the
    composition itself."""
    ws = _head_workspace(layer, x, group_sum.k) if isinstance(x, torch.Tensor) else None
    if ws is None:
        return group_sum.cross_entropy(layer(x), labels, ignore_index, return_scores)
    if labels.device != x.device or labels.dtype != torch.int64 or labels.shape != (x.shape[0],):
        raise RuntimeError(f"labels must be int64 of shape ({x.shape[0]},) on {x.device}")
    xr = to_rows(x)
    assert xr.shape[0] == layer.in_dim, (xr.shape, layer.in_dim)
    loss, scores = LogicGroupSumCrossEntropyFunction.apply(
        xr, layer.weights, layer.gate_sequence, layer.run_plan(), True, labels, group_sum.k,
        group_sum.tau, ignore_index, ws[0], ws[1])
    return (loss, scores) if return_scores else loss


def sequential_cross_entropy(model, x, labels, ignore_index: int = -100,
                             return_scores: bool = False):
    """cross_entropy(model(x), labels) for a Sequential ending in GroupSum, the training loss of
    experiments/experiment_script.py:280-284; when the module before the GroupSum is a dense
    LogicLayer, through the fused head (logic_group_sum_cross_entropy)."""
    mods = list(model)
    if not mods or not isinstance(mods[-1], GroupSum):
        raise ValueError("the model must end with a GroupSum")
    h = x
    if len(mods) >= 2 and type(mods[-2]) is LogicLayer:
        for m in mods[:-2]:
            h = m(h)
        return logic_group_sum_cross_entropy(mods[-2], mods[-1], h, labels, ignore_index,
                                             return_scores)
    for m in mods[:-1]:
        h = m(h)
    return mods[-1].cross_entropy(h, labels, ignore_index, return_scores)
