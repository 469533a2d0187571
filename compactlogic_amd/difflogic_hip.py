"""Tensor-level mirror of the reference's ``difflogic_cuda`` extension
(compactlogic/cuda/difflogic.cpp:60-105), backed by libcompactlogic_hip.so.

Same function names, argument order, dtypes and output shapes as the reference binding:
inputs are borrowed (must be contiguous device tensors), outputs are allocated here on the
input's device and returned.  Work is enqueued on the current stream of that device.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi

_DTYPES = {torch.float32: _capi.CL_DTYPE_F32, torch.float64: _capi.CL_DTYPE_F64}


def _check(t: torch.Tensor, name: str) -> None:
    # CHECK_INPUT of compactlogic/cuda/utils.cuh:9-37: device tensor and contiguous.
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a CUDA (HIP) tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check_dtype(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}, got {t.dtype}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported floating dtype {t.dtype}; the kernels take float32 "
                           "and float64") from None


def dense_dtype_code(t: torch.Tensor) -> int:
    """dtype code for the four reference-interface dense kernels, which also take float16
    (half storage, fp32 sums), as the reference dispatches them over half
    (compactlogic/cuda/difflogic_kernel.cu:222,267,315,397)."""
    if t.dtype == torch.float16:
        return _capi.CL_DTYPE_F16
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported floating dtype {t.dtype}; the dense kernels take "
                           "float16, float32 and float64") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _same_device(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on {dev}, got {t.device}")


def forward(x, a, b, w, gate_seq):
    """y[out, batch] = sum_g w * op_g(x[a], x[b]) (compactlogic/cuda/difflogic_kernel.cu:197-236)."""
    for t, n in ((x, "x"), (a, "a"), (b, "b"), (w, "w"), (gate_seq, "gate_seq")):
        _check(t, n)
    _same_device(x, a, b, w, gate_seq)
    _check_dtype(a, torch.int64, "a")
    _check_dtype(b, torch.int64, "b")
    _check_dtype(gate_seq, torch.uint8, "gate_seq")
    if w.dtype != x.dtype:
        raise RuntimeError("w must have the dtype of x")
    in_dim, batch = x.shape
    out_dim, g = w.shape
    if a.shape != (out_dim, g) or b.shape != (out_dim, g) or gate_seq.shape != (out_dim, g):
        raise RuntimeError("a, b, w and gate_seq must all be [out_dim, num_gates]")
    y = torch.empty((out_dim, batch), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_dense_forward", dense_dtype_code(x), ptr(x), ptr(a), ptr(b), ptr(w),
                   ptr(gate_seq), ptr(y), in_dim, out_dim, batch, g, stream_of(x))
    return y


def backward_w(x, a, b, gate_seq, grad_y):
    """grad_w[out, G] = sum_n grad_y * op_g(x[a], x[b]) (difflogic_kernel.cu:239-282)."""
    for t, n in ((x, "x"), (a, "a"), (b, "b"), (gate_seq, "gate_seq"), (grad_y, "grad_y")):
        _check(t, n)
    _same_device(x, a, b, gate_seq, grad_y)
    in_dim, batch = x.shape
    out_dim, g = a.shape
    if grad_y.shape != (out_dim, batch) or grad_y.dtype != x.dtype:
        raise RuntimeError("grad_y must be [out_dim, batch] with the dtype of x")
    grad_w = torch.empty((out_dim, g), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_dense_backward_w", dense_dtype_code(x), ptr(x), ptr(a), ptr(b), ptr(gate_seq),
                   ptr(grad_y), ptr(grad_w), in_dim, out_dim, batch, g, stream_of(x))
    return grad_w


def backward_x(x, a, b, w, gate_seq, grad_y, given_x_indices_of_y_start, given_x_indices_of_y,
               given_x_indices_of_gate):
    """grad_x[in, batch] through the inverse index, no atomics (difflogic_kernel.cu:285-333)."""
    named = ((x, "x"), (a, "a"), (b, "b"), (w, "w"), (gate_seq, "gate_seq"), (grad_y, "grad_y"),
             (given_x_indices_of_y_start, "given_x_indices_of_y_start"),
             (given_x_indices_of_y, "given_x_indices_of_y"),
             (given_x_indices_of_gate, "given_x_indices_of_gate"))
    for t, n in named:
        _check(t, n)
    _same_device(*(t for t, _ in named))
    _check_dtype(given_x_indices_of_y_start, torch.int64, "given_x_indices_of_y_start")
    _check_dtype(given_x_indices_of_y, torch.int64, "given_x_indices_of_y")
    _check_dtype(given_x_indices_of_gate, torch.int8, "given_x_indices_of_gate")
    in_dim, batch = x.shape
    out_dim, g = w.shape
    if given_x_indices_of_y_start.numel() != in_dim + 1:
        raise RuntimeError("given_x_indices_of_y_start must have in_dim + 1 entries")
    if given_x_indices_of_y.numel() != given_x_indices_of_gate.numel():
        raise RuntimeError("given_x_indices_of_y and given_x_indices_of_gate differ in length")
    grad_x = torch.empty_like(x)
    with torch.cuda.device(x.device):
        _capi.call("cl_dense_backward_x", dense_dtype_code(x), ptr(x), ptr(a), ptr(b), ptr(w),
                   ptr(gate_seq), ptr(grad_y), ptr(given_x_indices_of_y_start),
                   ptr(given_x_indices_of_y), ptr(given_x_indices_of_gate),
                   given_x_indices_of_y.numel(), ptr(grad_x), in_dim, out_dim, batch, g,
                   stream_of(x))
    return grad_x


def inverse_index(a, b, in_dim: int):
    """The inverse connection index of compactlogic/compactlogic.py:184-274 for pairs a, b
    [out, G] (int64): per input i, entries start[i] .. start[i+1]-1 of (neuron, code) with
    code g when i is operand a of slot g, -(g+1) when it is operand b.  Built on the tensors'
    device; the order inside a row is ascending by (side, neuron, slot) (a stable sort)."""
    dev = a.device
    out, g = a.shape
    rows = torch.arange(out, device=dev, dtype=torch.int64).unsqueeze(1).expand(out, g).reshape(-1)
    slots = torch.arange(g, device=dev, dtype=torch.int64).unsqueeze(0).expand(out, g).reshape(-1)
    inputs = torch.cat((a.reshape(-1), b.reshape(-1))).to(torch.int64)
    ys = torch.cat((rows, rows))
    codes = torch.cat((slots, -(slots + 1))).to(torch.int8)
    order = torch.sort(inputs, stable=True).indices
    counts = torch.bincount(inputs, minlength=in_dim)
    starts = torch.zeros(in_dim + 1, dtype=torch.int64, device=dev)
    starts[1:] = torch.cumsum(counts, 0)
    return starts, ys[order].contiguous(), codes[order].contiguous()


def backward_x_atomicAdd(x, a, b, w, gate_seq, grad_y):  # noqa: N802 - reference name
    """difflogic_cuda.backward_x_atomicAdd (compactlogic/cuda/difflogic.cpp:99-104,
    difflogic_kernel.cu:613-653): the same input gradient without a caller-supplied index.
    The reference scatters with float atomics; here the index is built on the device and the
    gradient gathered through it, so the result is deterministic."""
    for t, n in ((x, "x"), (a, "a"), (b, "b"), (w, "w"), (gate_seq, "gate_seq"), (grad_y, "grad_y")):
        _check(t, n)
    _check_dtype(a, torch.int64, "a")
    _check_dtype(b, torch.int64, "b")
    start, ys, codes = inverse_index(a, b, x.shape[0])
    return backward_x(x, a, b, w, gate_seq, grad_y, start, ys, codes)


def eval(x, a, b, w, gate_seq):  # noqa: A001 - mirrors difflogic_cuda.eval
    """Discrete forward with argmax slots w (uint8 slot ids) (difflogic_kernel.cu:341-411)."""
    for t, n in ((x, "x"), (a, "a"), (b, "b"), (w, "w"), (gate_seq, "gate_seq")):
        _check(t, n)
    _same_device(x, a, b, w, gate_seq)
    _check_dtype(w, torch.uint8, "w")
    in_dim, batch = x.shape
    out_dim, g = a.shape
    if w.numel() != out_dim:
        raise RuntimeError("w must hold one slot per neuron")
    y = torch.empty((out_dim, batch), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_dense_eval", dense_dtype_code(x), ptr(x), ptr(a), ptr(b), ptr(w),
                   ptr(gate_seq), ptr(y), in_dim, out_dim, batch, g, stream_of(x))
    return y


_PACK_DTYPES = {8: torch.int8, 16: torch.int16, 32: torch.int32, 64: torch.int64}


def tensor_packbits_cuda(t, bit_count):
    """bool [rows, n] -> (packed [rows, ceil(n / bit_count)], pad_len)
    (compactlogic/cuda/difflogic_kernel.cu:453-494)."""
    _check(t, "t")
    if t.dtype != torch.bool:
        raise RuntimeError("t must be a bool tensor")
    if bit_count not in _PACK_DTYPES:
        raise ValueError("`bit_count` has to be in { 8, 16, 32, 64 }")
    rows, n = t.shape
    words = -(-n // bit_count)
    packed = torch.empty((rows, words), dtype=_PACK_DTYPES[bit_count], device=t.device)
    pad = ctypes.c_int64(0)
    with torch.cuda.device(t.device):
        _capi.call("cl_pack_bits", ptr(t), rows, n, bit_count, ptr(packed), ctypes.byref(pad),
                   stream_of(t))
    return packed, int(pad.value)


def groupbitsum(b, pad_len, k):
    """packed [rows, words] -> int32 [N, k] per-class set-bit counts
    (compactlogic/cuda/difflogic.cpp:90-98, difflogic_kernel.cu:500-568)."""
    _check(b, "b")
    if b.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8):
        raise RuntimeError("packed tensor must have an integer dtype")
    rows = b.shape[0]
    if rows % k != 0:
        raise ValueError(f"in_dim ({rows}) has to be divisible by k ({k}) but it is not")
    row_bytes = b.shape[1] * b.element_size()
    n = row_bytes * 8 - pad_len
    counts = torch.empty((n, k), dtype=torch.int32, device=b.device)
    with torch.cuda.device(b.device):
        _capi.call("cl_group_bit_sum", ptr(b), rows, row_bytes, pad_len, k, ptr(counts),
                   stream_of(b))
    return counts


def eval_packed(x, a, b, w, gate_seq):
    """Bitwise layer on packed rows (integer difflogic_cuda.eval,
    third_party/convlogic_source_code/src/difflogic/cuda/difflogic_kernel.cu:271-330) with
    compactlogic's argmax-slot indirection.  x: [in_dim, words] of any integer width."""
    for t, n in ((x, "x"), (a, "a"), (b, "b"), (w, "w"), (gate_seq, "gate_seq")):
        _check(t, n)
    _same_device(x, a, b, w, gate_seq)
    _check_dtype(w, torch.uint8, "w")
    in_dim = x.shape[0]
    out_dim, g = a.shape
    row_bytes = x.shape[1] * x.element_size()
    y = torch.empty((out_dim, x.shape[1]), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_dense_eval_packed", ptr(x), ptr(a), ptr(b), ptr(w), ptr(gate_seq), ptr(y),
                   in_dim, out_dim, row_bytes, g, stream_of(x))
    return y


def fill_splitmix64(out: torch.Tensor, base: int) -> torch.Tensor:
    """out.view(-1)[i] = splitmix64(base + i) for a contiguous int64 tensor."""
    _check(out, "out")
    if out.dtype != torch.int64:
        raise RuntimeError("out must be int64")
    with torch.cuda.device(out.device):
        _capi.call("cl_fill_splitmix64", ptr(out), out.numel(), base & 0xFFFFFFFFFFFFFFFF,
                   stream_of(out))
    return out
