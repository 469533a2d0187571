"""Logic-tree convolution blocks of the third-party ConvLogic package on the HIP kernels of
csrc/tree_conv.hip: ConvLogicLayer (third_party/convlogic_source_code/src/convlogic/
convlogic_layer.py:85-470), TreeLogicLayer (treelogic_layer.py:33-130), PoolLogicLayer
(convlogic_layer.py:473-500) and the autograd bridges ConvLogicFunction, FullConvLogicFunction
and TreeLogicFunction with the reference's argument lists.

Differences from the reference, all on purpose:
- the complete block does not keep its node outputs for the backward pass: the backward
  recomputes the winner position of each pooling window from x (eight taps), so the forward
  writes only y and the pooling indices unless the caller asks for the intermediates;
- the input gradient is a deterministic gather (no float atomics), reproducible bit for bit;
- implementation='python' (the reference's CPU restatement) is not shipped: the modules run the
  HIP kernels only and fail loudly without them;
- a PackBitsTensor input (frozen block, eval mode) is evaluated bitwise with argmax gates and
  the pool as the OR of the window, the discrete reading of the block in
  third_party/convlogic/extract.py:177-214.
"""
from __future__ import annotations

import ctypes
import math
import weakref

import torch
from torch import nn
from torch.autograd import Function

from . import _capi, timing
from . import difflogic_hip as _dl
from .layers import PackBitsTensor

__all__ = [
    "ConvLogicLayer", "TreeLogicLayer", "PoolLogicLayer", "ConvLogicFunction",
    "FullConvLogicFunction", "TreeLogicFunction", "GradFactor", "generate_selection",
    "unpack_selection", "convlogic_forward", "full_convlogic_forward", "tree_conv_backward",
    "treelogic_forward", "treelogic_backward", "tree_conv_eval_packed", "channel_uses",
]


class GradFactor(Function):
    """Identity forward, gradient scaled by `f` (third_party/convlogic_source_code/src/difflogic/
    functional.py GradFactor)."""

    @staticmethod
    def forward(ctx, x, f):
        ctx.f = f
        return x.view_as(x)

    @staticmethod
    def backward(ctx, grad_y):
        return grad_y * ctx.f, None


def unpack_selection(selection: torch.Tensor):
    """(channel, row, col) of packed taps ch << 16 | row << 8 | col (convlogic_layer.py:182-186)."""
    return (selection >> 16) & 0xFFFF, (selection >> 8) & 0xFF, selection & 0xFF


def channel_uses(selection: torch.Tensor, c_in: int):
    """(ent_ptr int32 [c_in + 1], ent int32 [8 * c_out]): the taps c * 8 + k reading each input
    channel, in ascending order -- the gather order of the input gradient.  Raises ValueError
    for a tap channel outside [0, c_in)."""
    ch = unpack_selection(selection.reshape(-1).to(torch.int64))[0]
    if ch.numel() and int(ch.max()) >= c_in:
        raise ValueError(f"selection names input channel {int(ch.max())} of {c_in}")
    ent = torch.argsort(ch, stable=True).to(torch.int32)
    ptr = torch.zeros(c_in + 1, dtype=torch.int64, device=selection.device)
    ptr[1:] = torch.cumsum(torch.bincount(ch, minlength=c_in), 0)
    return ptr.to(torch.int32).contiguous(), ent.contiguous()


def _pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def _out_hw(h, w, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w):
    return (h + 2 * pad_h - kernel_h) // stride_h + 1, (w + 2 * pad_w - kernel_w) // stride_w + 1


def _check_block(x, w_prob, selection, nodes):
    _dl._check(x, "x")
    _dl._check(w_prob, "w_prob")
    _dl._check_dtype(selection, torch.int32, "selection")
    _dl._same_device(x, w_prob, selection)
    if x.dim() != 4:
        raise RuntimeError(f"x must be [N, C, H, W], got {tuple(x.shape)}")
    if w_prob.dtype != x.dtype:
        raise RuntimeError("w_prob must have the dtype of x")
    c_out = selection.shape[0]
    if selection.dim() != 2 or selection.shape[1] != 8:
        raise RuntimeError(f"selection must be [C_out, 8], got {tuple(selection.shape)}")
    if tuple(w_prob.shape) != (c_out, nodes, 16):
        raise RuntimeError(f"w_prob must be [{c_out}, {nodes}, 16], got {tuple(w_prob.shape)}")
    return c_out


def _forward_call(softmax: bool, regular: bool, y_rows: bool = False):
    if (regular or y_rows) and not softmax:
        raise ValueError("the regular-taps guarantee and the feature-major output are taken by "
                         "the logits forward only")
    return ("cl_tree_conv_forward_softmax",) if softmax else ("cl_tree_conv_forward",)


def _forward_tail(softmax: bool, regular: bool, y_rows: bool = False):
    return (int(regular), int(y_rows)) if softmax else ()


def full_convlogic_forward(x, w_prob, selection, stride_h, stride_w, pad_h, pad_w, kernel_h,
                           kernel_w, intermediate: bool = True, softmax: bool = False,
                           regular: bool = False, y_rows: bool = False, coefs=None):
    """Complete block forward (replaces convlogic_cuda.full_convlogic_forward,
    full_convlogic_kernel.cu:156-231): (y [N, C, Ho/2, Wo/2], x2 [N, C, Ho, Wo, 4],
    x3 [N, C, Ho, Wo, 2], indices int32 [N, C, Ho/2 * Wo/2]); x2 and x3 are None unless
    `intermediate`.  With `softmax`, w_prob holds the node logits and the kernels take their
    softmax (cl_tree_conv_forward_softmax); `regular` then passes that call the guarantee that
    every tap lies in the kernel window and reads an input channel, and `y_rows` has it write y
    feature-major: y is then the [N, C, Ho/2, Wo/2] view of a contiguous [C*Ho/2*Wo/2, N]
    buffer, which flattens to the transpose a following dense layer reads as its rows.
    `coefs` (logits only): a [C, 7, 4] tensor the call fills with the collapsed node
    coefficients for tree_conv_backward(..., coefs=) on the same logits
    (cl_tree_conv_forward_softmax_coefs)."""
    c_out = _check_block(x, w_prob, selection, 7)
    if coefs is not None:
        if not softmax:
            raise ValueError("the coefficient hand-over is for the logits forward")
        _dl._check(coefs, "coefs")
        if tuple(coefs.shape) != (c_out, 7, 4) or coefs.dtype != x.dtype:
            raise RuntimeError(f"coefs must be [{c_out}, 7, 4] of the dtype of x")
    n, c_in, h, w = x.shape
    ho, wo = _out_hw(h, w, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
    if ho <= 0 or wo <= 0:
        raise RuntimeError(f"Invalid output shape: H_out={ho}, W_out={wo}")
    if ho % 2 or wo % 2:
        raise RuntimeError("Output height and width after convolution must be divisible by 2 for "
                           f"2x2 max pooling, but got H_out={ho}, W_out={wo}")
    if y_rows:
        y = torch.empty((c_out, ho // 2, wo // 2, n), dtype=x.dtype,
                        device=x.device).permute(3, 0, 1, 2)
    else:
        y = torch.empty((n, c_out, ho // 2, wo // 2), dtype=x.dtype, device=x.device)
    idx = torch.empty((n, c_out, (ho // 2) * (wo // 2)), dtype=torch.int32, device=x.device)
    x2 = x3 = None
    if intermediate:
        x2 = torch.empty((n, c_out, ho, wo, 4), dtype=x.dtype, device=x.device)
        x3 = torch.empty((n, c_out, ho, wo, 2), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        if coefs is not None:
            timing.timed(f"cl_tree_conv_forward[{c_in}x{h}x{w}->{c_out}]", lambda: _capi.call(
                "cl_tree_conv_forward_softmax_coefs", _dl.dtype_code(x), x.data_ptr(),
                w_prob.data_ptr(), selection.data_ptr(), n, c_in, h, w, c_out, stride_h,
                stride_w, pad_h, pad_w, kernel_h, kernel_w, y.data_ptr(), _dl.ptr(x2),
                _dl.ptr(x3), idx.data_ptr(), int(regular), int(y_rows), coefs.data_ptr(),
                _dl.stream_of(x)))
        else:
            timing.timed(f"cl_tree_conv_forward[{c_in}x{h}x{w}->{c_out}]", lambda: _capi.call(
                *_forward_call(softmax, regular, y_rows), _dl.dtype_code(x), x.data_ptr(),
                w_prob.data_ptr(), selection.data_ptr(), n, c_in, h, w, c_out, stride_h,
                stride_w, pad_h, pad_w, kernel_h, kernel_w, 1, y.data_ptr(), _dl.ptr(x2),
                _dl.ptr(x3), idx.data_ptr(), *_forward_tail(softmax, regular, y_rows),
                _dl.stream_of(x)))
    return y, x2, x3, idx


def convlogic_forward(x, w_prob, selection, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w,
                      softmax: bool = False, regular: bool = False):
    """Conv gates only (replaces convlogic_cuda.convlogic_forward, convlogic_kernel.cu:67-107):
    y [N, C, Ho, Wo, 4].  With `softmax`, w_prob holds the node logits."""
    c_out = _check_block(x, w_prob, selection, 4)
    n, c_in, h, w = x.shape
    ho, wo = _out_hw(h, w, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
    if ho <= 0 or wo <= 0:
        raise RuntimeError(f"Invalid output shape: H_out={ho}, W_out={wo}")
    y = torch.empty((n, c_out, ho, wo, 4), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call(*_forward_call(softmax, regular), _dl.dtype_code(x), x.data_ptr(),
                   w_prob.data_ptr(), selection.data_ptr(), n, c_in, h, w, c_out, stride_h,
                   stride_w, pad_h, pad_w, kernel_h, kernel_w, 0, y.data_ptr(), None, None, None,
                   *_forward_tail(softmax, regular), _dl.stream_of(x))
    return y


def tree_conv_backward(grad_y, x, w_prob, selection, indices, stride_h, stride_w, pad_h, pad_w,
                       kernel_h, kernel_w, complete: bool, need_x: bool = True,
                       need_w: bool = True, uses=None, softmax: bool = False, coefs=None):
    """(grad_x or None, grad_w_prob or None) of the complete block or of the conv gates
    (replaces full_convlogic_backward_x / _weight and convlogic_backward_x / _weight).  `uses`
    is channel_uses(selection, C_in), computed when not given.  With `softmax`, w_prob holds
    the node logits and the second result is the gradient of the logits; `coefs` (complete
    block, logits) are those full_convlogic_forward(..., coefs=) filled for these logits
    (cl_tree_conv_backward_softmax_coefs)."""
    if coefs is not None and not (softmax and complete):
        raise ValueError("the coefficient hand-over is for the complete block's logits")
    nodes = 7 if complete else 4
    c_out = _check_block(x, w_prob, selection, nodes)
    n, c_in, h, w = x.shape
    # the logits path reads a complete block's grad_y feature-major as it comes from a
    # flattened dense layer (the transpose of a contiguous [C*Hp*Wp, N]), NCHW otherwise
    y_rows = (softmax and complete and grad_y.dim() == 4 and not grad_y.is_contiguous()
              and grad_y.permute(1, 2, 3, 0).is_contiguous())
    if not y_rows:
        grad_y = grad_y.contiguous()
    _dl._check(grad_y.permute(1, 2, 3, 0) if y_rows else grad_y, "grad_y")
    if complete:
        _dl._check_dtype(indices, torch.int32, "indices")
    gx = torch.empty_like(x) if need_x else None
    gw = torch.empty((c_out, nodes, 16), dtype=x.dtype, device=x.device) if need_w else None
    if gx is None and gw is None:
        return None, None
    if need_x and uses is None:
        uses = channel_uses(selection, c_in)
    ptr, ent = uses if need_x else (None, None)
    code = _dl.dtype_code(x)
    need = ctypes.c_int64(0)
    _capi.call("cl_tree_conv_workspace", code, n, c_in, h, w, c_out, stride_h, stride_w, pad_h,
               pad_w, kernel_h, kernel_w, int(complete), int(gx is not None), ctypes.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        if coefs is not None:
            _dl._check(coefs, "coefs")
            if tuple(coefs.shape) != (c_out, 7, 4) or coefs.dtype != x.dtype:
                raise RuntimeError(f"coefs must be [{c_out}, 7, 4] of the dtype of x")
            timing.timed(f"cl_tree_conv_backward[{c_in}x{h}x{w}->{c_out}]", lambda: _capi.call(
                "cl_tree_conv_backward_softmax_coefs", code, grad_y.data_ptr(), x.data_ptr(),
                w_prob.data_ptr(), selection.data_ptr(), indices.data_ptr(), _dl.ptr(ptr),
                _dl.ptr(ent), n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w,
                kernel_h, kernel_w, _dl.ptr(gx), _dl.ptr(gw), ws.data_ptr(), need.value,
                int(y_rows), coefs.data_ptr(), _dl.stream_of(x)))
        else:
            timing.timed(f"cl_tree_conv_backward[{c_in}x{h}x{w}->{c_out}]", lambda: _capi.call(
                "cl_tree_conv_backward_softmax" if softmax else "cl_tree_conv_backward", code,
                grad_y.data_ptr(), x.data_ptr(), w_prob.data_ptr(),
                selection.data_ptr(), indices.data_ptr() if complete else None, _dl.ptr(ptr),
                _dl.ptr(ent), n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w,
                kernel_h, kernel_w, int(complete), _dl.ptr(gx), _dl.ptr(gw), ws.data_ptr(),
                need.value, *((int(y_rows),) if softmax else ()), _dl.stream_of(x)))
    return gx, gw


def _level_shape(x, w_prob):
    _dl._check(x, "x")
    _dl._check(w_prob, "w_prob")
    _dl._same_device(x, w_prob)
    if x.dim() != 5:
        raise RuntimeError(f"Expected input tensor x to be 5D (N, C, H, W, 2*Xout), but got {x.dim()}")
    n, c, hh, ww, xin = x.shape
    xout = xin // 2
    if xin != 2 * xout:
        raise RuntimeError(f"Expected input x.size(4) (Xin) to equal 2*Xout ({2 * xout}), but got {xin}")
    if xout > 4:
        raise RuntimeError("Xout > 4 is not supported")
    if tuple(w_prob.shape) != (c, xout, 16) or w_prob.dtype != x.dtype:
        raise RuntimeError(f"w_prob must be [{c}, {xout}, 16] of the dtype of x")
    return n, c, hh * ww, xout


def treelogic_forward(x, w_prob):
    """One tree level (replaces convlogic_cuda.treelogic_forward, treelogic_kernel.cu:46-86)."""
    n, c, s, xout = _level_shape(x, w_prob)
    y = torch.empty(x.shape[:4] + (xout,), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_tree_level_forward", _dl.dtype_code(x), x.data_ptr(), w_prob.data_ptr(),
                   n, c, s, xout, y.data_ptr(), _dl.stream_of(x))
    return y


def treelogic_backward(grad_y, x, w_prob, need_x: bool = True, need_w: bool = True):
    """(grad_x, grad_w_prob) of one tree level (replaces treelogic_backward_x and
    treelogic_backward_weight, treelogic_kernel.cu:160-290)."""
    n, c, s, xout = _level_shape(x, w_prob)
    grad_y = grad_y.contiguous()
    _dl._check(grad_y, "grad_y")
    if tuple(grad_y.shape) != tuple(x.shape[:4]) + (xout,):
        raise RuntimeError(f"grad_y must be {tuple(x.shape[:4]) + (xout,)}")
    gx = torch.empty_like(x) if need_x else None
    gw = torch.empty((c, xout, 16), dtype=x.dtype, device=x.device) if need_w else None
    code = _dl.dtype_code(x)
    need = ctypes.c_int64(0)
    _capi.call("cl_tree_level_workspace", code, n, c, s, xout, ctypes.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_tree_level_backward", code, grad_y.data_ptr(), x.data_ptr(),
                   w_prob.data_ptr(), n, c, s, xout, _dl.ptr(gx), _dl.ptr(gw), ws.data_ptr(),
                   need.value, _dl.stream_of(x))
    return gx, gw


def tree_row_bytes(row_bytes: int) -> int:
    """Row length the packed block reads best: rows of 16 KiB or more are widened to the next
    odd multiple of 256 bytes.  The block reads one 256-byte column window of every input row
    while it works on that window (the window's rows are reused from L2 by every output
    channel); rows a large power of two apart put the whole window into the same few L2 sets,
    and its reads then miss again and again.  Rows an odd number of 256-byte blocks apart
    spread it over all sets."""
    if row_bytes < 16384:
        return row_bytes
    nbytes = -(-row_bytes // 256) * 256
    return nbytes + 256 if (nbytes // 256) % 2 == 0 else nbytes


def widen_rows(t: torch.Tensor, row_bytes: int) -> torch.Tensor:
    """Copy of packed rows t [rows, words] widened to row_bytes with zero words."""
    words = row_bytes // t.element_size()
    out = torch.empty((t.shape[0], words), dtype=t.dtype, device=t.device)
    out[:, :t.shape[1]].copy_(t)
    out[:, t.shape[1]:].zero_()
    return out


def tree_conv_eval_packed(x_words, gates, selection, in_shape, stride, padding, kernel,
                          complete: bool = True):
    """Packed discrete block: x_words [c_in * h * w, words] (rows in NCHW feature order), gates
    uint8 [C_out, nodes] opcodes -> output rows [C_out * Hp * Wp, words] (complete) or
    [C_out * Ho * Wo * 4, words]."""
    _dl._check(x_words, "x")
    c_in, h, w = in_shape
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    kh, kw = _pair(kernel)
    if x_words.dim() != 2 or x_words.shape[0] != c_in * h * w:
        raise RuntimeError(f"x must be [{c_in * h * w}, words], got {tuple(x_words.shape)}")
    c_out = selection.shape[0]
    ho, wo = _out_hw(h, w, sh, sw, ph, pw, kh, kw)
    rows = c_out * (ho // 2) * (wo // 2) if complete else c_out * ho * wo * 4
    y = torch.empty((rows, x_words.shape[1]), dtype=x_words.dtype, device=x_words.device)
    with torch.cuda.device(x_words.device):
        timing.timed(f"cl_tree_conv_eval_packed[{c_in * h * w}->{rows}]", lambda: _capi.call(
            "cl_tree_conv_eval_packed", x_words.data_ptr(),
            x_words.shape[1] * x_words.element_size(), gates.data_ptr(), selection.data_ptr(),
            c_in, h, w, c_out, sh, sw, ph, pw, kh, kw, int(complete), y.data_ptr(),
            _dl.stream_of(x_words)))
    return y


# ----------------------------------------------------------------------------- autograd bridges

class ConvLogicFunction(Function):
    """Conv gates only (convlogic_layer.py:16-33): y [N, C, Ho, Wo, 4]."""

    @staticmethod
    def forward(ctx, x, w_prob, selection, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w):
        x = x.contiguous()
        y = convlogic_forward(x, w_prob, selection, stride_h, stride_w, pad_h, pad_w, kernel_h,
                              kernel_w)
        ctx.save_for_backward(x, w_prob, selection)
        ctx.geom = (stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, w_prob, selection = ctx.saved_tensors
        gx, gw = tree_conv_backward(grad_y, x, w_prob, selection, None, *ctx.geom, complete=False,
                                    need_x=ctx.needs_input_grad[0],
                                    need_w=ctx.needs_input_grad[1])
        return gx, gw, None, None, None, None, None, None, None


class FullConvLogicFunction(Function):
    """Complete block (convlogic_layer.py:36-82): y, plus (x2, x3) with return_intermediate and
    the pooling indices with return_indices, in the reference's order.  Gradients flow from y
    only, as in the reference."""

    @staticmethod
    def forward(ctx, x, w_prob, selection, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w,
                return_intermediate=False, return_indices=False):
        x = x.contiguous()
        y, x2, x3, idx = full_convlogic_forward(x, w_prob, selection, stride_h, stride_w, pad_h,
                                                pad_w, kernel_h, kernel_w,
                                                intermediate=return_intermediate)
        ctx.save_for_backward(x, w_prob, selection, idx)
        ctx.geom = (stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
        extra = []
        if return_intermediate:
            extra += [x2, x3]
        if return_indices:
            extra.append(idx)
        if not extra:
            return y
        ctx.mark_non_differentiable(*extra)
        return (y, *extra)

    @staticmethod
    def backward(ctx, grad_y, *unused):
        x, w_prob, selection, idx = ctx.saved_tensors
        gx, gw = tree_conv_backward(grad_y, x, w_prob, selection, idx, *ctx.geom, complete=True,
                                    need_x=ctx.needs_input_grad[0],
                                    need_w=ctx.needs_input_grad[1])
        return gx, gw, None, None, None, None, None, None, None, None, None


class TreeLogicFunction(Function):
    """One tree level (treelogic_layer.py:15-30)."""

    @staticmethod
    def forward(ctx, x, w_prob):
        x = x.contiguous()
        y = treelogic_forward(x, w_prob)
        ctx.save_for_backward(x, w_prob)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, w_prob = ctx.saved_tensors
        gx, gw = treelogic_backward(grad_y, x, w_prob, need_x=ctx.needs_input_grad[0],
                                    need_w=ctx.needs_input_grad[1])
        return gx, gw


# ----------------------------------------------------------------------------- modules

def generate_selection(in_channels: int, out_channels: int, kernel=3, groups: int = 1,
                       num_chn: int = 2, input_bits: int = 8, device=None) -> torch.Tensor:
    """Random taps [out_channels, input_bits] int32, packed ch << 16 | row << 8 | col, drawn as
    in ConvLogicLayer.generate_selection (convlogic_layer.py:382-468): the input channels are
    split into `groups`; every output channel of a group pre-draws `num_chn` channels of its
    group with replacement (all of them when num_chn == 0) and each tap picks one of those;
    rows and columns are uniform in the kernel; the second tap of a gate is re-drawn until it
    differs from the first when both name the same channel and position."""
    kh, kw = _pair(kernel)
    base, rem = divmod(in_channels, groups)
    sizes = [base + (1 if g < rem else 0) for g in range(groups)]
    starts = [sum(sizes[:g]) for g in range(groups)]
    out_per = max(out_channels // groups, 1)
    group_of = torch.clamp(torch.arange(out_channels) // out_per, 0, groups - 1)
    ch_sel = torch.empty((out_channels, input_bits), dtype=torch.int32)
    for gid in range(groups):
        rows_of = (group_of == gid).nonzero(as_tuple=True)[0]
        cnt, k = rows_of.numel(), sizes[gid]
        if cnt == 0 or k == 0:
            continue
        chans = torch.arange(starts[gid], starts[gid] + k, dtype=torch.int32)
        m = k if num_chn == 0 else min(num_chn, k)
        chosen = torch.stack([chans[torch.randint(0, k, (cnt,))] for _ in range(m)], dim=1)
        picks = torch.randint(0, m, (cnt, input_bits))
        ch_sel[rows_of] = torch.gather(chosen, 1, picks).to(torch.int32)
    rows = torch.randint(0, kh, (out_channels, input_bits), dtype=torch.int32)
    cols = torch.randint(0, kw, (out_channels, input_bits), dtype=torch.int32)
    if kh * kw > 1:
        for k in range(0, input_bits, 2):
            same = ((ch_sel[:, k] == ch_sel[:, k + 1]) & (rows[:, k] == rows[:, k + 1])
                    & (cols[:, k] == cols[:, k + 1])).nonzero(as_tuple=True)[0]
            for i in same.tolist():
                while True:
                    r = int(torch.randint(0, kh, (1,)))
                    c = int(torch.randint(0, kw, (1,)))
                    if (r, c) != (int(rows[i, k]), int(cols[i, k])):
                        rows[i, k + 1], cols[i, k + 1] = r, c
                        break
    packed = (ch_sel << 16) | (rows << 8) | cols
    return packed.to(device) if device is not None else packed


class ConvLogicLayer(nn.Module):
    """Logic-gate convolution (convlogic_layer.py:85-470): eight taps per output channel feed
    four gates; with complete=True, two tree levels (4 -> 2 -> 1) and a 2x2 max pool follow,
    giving [N, C_out, Ho/2, Wo/2].  Constructor, buffers and outputs as in the reference."""

    def __init__(self, in_channels: int, out_channels: int, stride=1, padding=1, kernel=3,
                 groups: int = 1, selection: torch.Tensor | None = None,
                 residual_init: bool = False, implementation: str = "cuda",
                 grad_factor: float = 1.0, complete: bool = False,
                 return_intermediate: bool = False, return_indices: bool = False,
                 num_chn: int = 2):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.kernel = _pair(kernel)
        self.groups = groups
        self.grad_factor = grad_factor
        self.complete = complete
        self.return_intermediate = return_intermediate
        self.return_indices = return_indices
        self.num_chn = num_chn
        self.input_bits = 8
        self.implementation = implementation
        if implementation == "cuda" and not torch.cuda.is_available():
            raise RuntimeError("CUDA implementation requested, but CUDA is not available.")
        if implementation not in ("cuda",):
            raise ValueError(f"implementation {implementation!r} is not available: this build "
                             "runs the HIP kernels only")
        nodes = 7 if complete else 4
        if residual_init:
            w = torch.zeros(out_channels, nodes, 16)
            w[..., 3] = 5.0
            self.weights = nn.Parameter(w)
        else:
            self.weights = nn.Parameter(torch.randn(out_channels, nodes, 16))
        if selection is None:
            selection = self.generate_selection(num_chn)
        self.register_buffer("selection", selection)
        assert selection.shape == (out_channels, 8)
        assert self.weights.shape[-1] == 16, f"Expected 16 logic functions, got {self.weights.shape[-1]}"
        self._uses = None
        self._regular = None
        # training output feature-major (the view of a [C*Hp*Wp, N] buffer) for a block whose
        # output is flattened into a dense layer: no transposes either way (complete only)
        self.rows_output = False

    def __getstate__(self):
        # the caches hold weak references, which do not pickle; they rebuild on the next call
        state = super().__getstate__()
        state["_uses"] = None
        state["_regular"] = None
        return state

    def generate_selection(self, num_chn: int = 2) -> torch.Tensor:
        return generate_selection(self.in_channels, self.out_channels, self.kernel, self.groups,
                                  num_chn, self.input_bits, self.weights.device)

    def unpack_selection(self, selection: torch.Tensor):
        return unpack_selection(selection)

    def _channel_uses(self):
        """The channel-use index of the current selection, cached with a weak reference to
        the selection tensor and its version (a new tensor at a recycled address rebuilds)."""
        sel = self.selection
        hit = self._uses
        if hit is None or hit[0]() is not sel or hit[1] != (sel._version, sel.device):
            self._uses = (weakref.ref(sel), (sel._version, sel.device),
                          channel_uses(sel.to(torch.int32), self.in_channels))
        return self._uses[2]

    def _regular_taps(self) -> bool:
        """Whether every tap of the selection lies in the kernel window and reads an input
        channel (what the selection sampler draws), cached with a weak reference to the
        selection and its version.  A cold cache under HIP graph capture answers False (no host
        read is possible there), which only costs the forward its fix-up launch."""
        sel = self.selection
        key = (sel._version, sel.device)
        hit = self._regular
        if hit is not None and hit[0]() is sel and hit[1] == key:
            return hit[2]
        if sel.is_cuda and torch.cuda.is_current_stream_capturing():
            return False
        s = sel.to(torch.int64).cpu()
        ok = bool((((s >> 16) & 0xFFFF) < self.in_channels).all()
                  and (((s >> 8) & 0xFF) < self.kernel[0]).all()
                  and ((s & 0xFF) < self.kernel[1]).all())
        self._regular = (weakref.ref(sel), key, ok)
        return ok

    def _w_prob(self, dtype):
        if self.training:
            return torch.nn.functional.softmax(self.weights, dim=-1).to(dtype).contiguous()
        idx = self.weights.argmax(-1)
        return torch.nn.functional.one_hot(idx, num_classes=16).to(dtype=dtype).contiguous()

    def forward(self, x):
        if isinstance(x, PackBitsTensor):
            return self.forward_packed(x)
        x = x.contiguous()
        if self.grad_factor != 1.0:
            x = GradFactor.apply(x, self.grad_factor)
        return self.forward_cuda(x)

    def forward_cuda(self, x):
        x = x.contiguous()
        # Training with logits of x's dtype: the kernels take the softmax of the logits
        # themselves (and its backward), so no probability tensor or softmax launch is needed.
        softmax = self.training and self.weights.dtype == x.dtype
        w = self.weights.contiguous() if softmax else self._w_prob(x.dtype)
        sel = self.selection.to(torch.int32).contiguous()
        args = (x, w, sel, self.stride[0], self.stride[1], self.padding[0], self.padding[1],
                self.kernel[0], self.kernel[1])
        regular = softmax and self._regular_taps()
        if self.complete:
            rows = softmax and getattr(self, "rows_output", False)
            return _FullConvLogicWithUses.apply(*args, self.return_intermediate,
                                                self.return_indices, self._channel_uses(),
                                                softmax, regular, rows)
        return _ConvLogicWithUses.apply(*args, self._channel_uses(), softmax, regular)

    def forward_packed(self, x: PackBitsTensor, in_hw=None) -> PackBitsTensor:
        """Bitwise block on packed rows (eval mode): rows = in_channels * h * w features in NCHW
        order.  The spatial size is `in_hw`, or the square root of rows / in_channels."""
        assert not self.training
        rows = x.t.shape[0]
        if in_hw is None:
            if rows % self.in_channels:
                raise ValueError(f"{rows} packed rows do not split into {self.in_channels} channels")
            side = math.isqrt(rows // self.in_channels)
            if side * side * self.in_channels != rows:
                raise ValueError("non-square input: pass in_hw=(h, w) to forward_packed")
            in_hw = (side, side)
        gates = self.weights.argmax(-1).to(torch.uint8).contiguous()
        t = x.t
        nbytes = t.shape[1] * t.element_size()
        want = tree_row_bytes(nbytes)
        if want != nbytes:  # widen once; the output rows (and later blocks) keep the width
            t = timing.timed(f"widen_rows[{rows}]", lambda: widen_rows(x.t, want))
            x.pad_len += (want - nbytes) * 8
        x.t = tree_conv_eval_packed(t, gates, self.selection.to(torch.int32).contiguous(),
                                    (self.in_channels, *in_hw), self.stride, self.padding,
                                    self.kernel, complete=self.complete)
        return x

    def extra_repr(self):
        return f"in_channels={self.in_channels}, out_channels={self.out_channels}, groups={self.groups}"


class _ConvLogicWithUses(Function):
    """ConvLogicFunction with the layer's cached channel-use index; with `softmax`, w holds
    the node logits (the kernels' softmax and its backward)."""

    @staticmethod
    def forward(ctx, x, w, selection, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w,
                uses, softmax=False, regular=False):
        y = convlogic_forward(x, w, selection, stride_h, stride_w, pad_h, pad_w, kernel_h,
                              kernel_w, softmax=softmax, regular=regular)
        ctx.save_for_backward(x, w, selection)
        ctx.geom = (stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
        ctx.uses = uses
        ctx.softmax = softmax
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, w, selection = ctx.saved_tensors
        gx, gw = tree_conv_backward(grad_y, x, w, selection, None, *ctx.geom, complete=False,
                                    need_x=ctx.needs_input_grad[0],
                                    need_w=ctx.needs_input_grad[1], uses=ctx.uses,
                                    softmax=ctx.softmax)
        return gx, gw, None, None, None, None, None, None, None, None, None, None


class _FullConvLogicWithUses(Function):
    """FullConvLogicFunction with the layer's cached channel-use index; with `softmax`, w
    holds the node logits."""

    @staticmethod
    def forward(ctx, x, w, selection, stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w,
                return_intermediate, return_indices, uses, softmax=False, regular=False,
                y_rows=False):
        # the logits path hands the collapsed coefficients from the forward to the backward
        # (autograd's version check on the saved w guards that both see the same logits)
        coefs = (torch.empty((selection.shape[0], 7, 4), dtype=x.dtype, device=x.device)
                 if softmax else None)
        y, x2, x3, idx = full_convlogic_forward(x, w, selection, stride_h, stride_w, pad_h,
                                                pad_w, kernel_h, kernel_w,
                                                intermediate=return_intermediate,
                                                softmax=softmax, regular=regular, y_rows=y_rows,
                                                coefs=coefs)
        ctx.save_for_backward(x, w, selection, idx, coefs)
        ctx.geom = (stride_h, stride_w, pad_h, pad_w, kernel_h, kernel_w)
        ctx.uses = uses
        ctx.softmax = softmax
        extra = []
        if return_intermediate:
            extra += [x2, x3]
        if return_indices:
            extra.append(idx)
        if not extra:
            return y
        ctx.mark_non_differentiable(*extra)
        return (y, *extra)

    @staticmethod
    def backward(ctx, grad_y, *unused):
        x, w, selection, idx, coefs = ctx.saved_tensors
        gx, gw = tree_conv_backward(grad_y, x, w, selection, idx, *ctx.geom, complete=True,
                                    need_x=ctx.needs_input_grad[0],
                                    need_w=ctx.needs_input_grad[1], uses=ctx.uses,
                                    softmax=ctx.softmax, coefs=coefs)
        return gx, gw, None, None, None, None, None, None, None, None, None, None, None, None, None


class TreeLogicLayer(nn.Module):
    """One level of a logic tree over the last dimension (treelogic_layer.py:33-130):
    [N, C, H, W, input_bits] -> [N, C, H, W, input_bits / 2]."""

    def __init__(self, channels: int, input_bits: int, residual_init: bool = False,
                 implementation: str = "cuda", grad_factor: float = 1.0):
        super().__init__()
        assert input_bits % 2 == 0, "input_bits must be even"
        self.channels = channels
        self.input_bits = input_bits
        self.implementation = implementation
        self.grad_factor = grad_factor
        if implementation not in ("cuda",):
            raise ValueError(f"implementation {implementation!r} is not available: this build "
                             "runs the HIP kernels only")
        out_bits = input_bits // 2
        if residual_init:
            w = torch.zeros(channels, out_bits, 16)
            w[..., 3] = 5.0
            self.weights = nn.Parameter(w)
        else:
            self.weights = nn.Parameter(torch.randn(channels, out_bits, 16))

    def forward(self, x):
        assert x.shape[-1] == self.input_bits, (
            f"Expected input last dimension to be {self.input_bits}, but got {x.shape[-1]}")
        x = x.contiguous()
        if self.grad_factor != 1.0:
            x = GradFactor.apply(x, self.grad_factor)
        return self.forward_cuda(x)

    def forward_cuda(self, x):
        if self.training:
            w_prob = torch.nn.functional.softmax(self.weights, dim=-1)
        else:
            idx = self.weights.argmax(-1)
            w_prob = torch.nn.functional.one_hot(idx, num_classes=16).to(dtype=x.dtype)
        return TreeLogicFunction.apply(x, w_prob.to(x.dtype).contiguous())

    def extra_repr(self):
        return f"channels={self.channels}, input_bits={self.input_bits}"


class PoolLogicLayer(nn.Module):
    """2x2 max pool, the OR of a window on {0, 1} values (convlogic_layer.py:473-500): torch's
    max_pool2d, as in the reference; a 5D input must have last dimension 1."""

    def __init__(self, kernel=2, stride=2, return_indices=False):
        super().__init__()
        self.kernel = _pair(kernel)
        self.stride = _pair(stride)
        self.return_indices = return_indices

    def forward(self, x):
        if x.ndim == 5:
            if x.size(4) != 1:
                raise ValueError(f"Expected last dim=1, got {x.size(4)}")
            x = x.view(x.size(0), x.size(1), x.size(2), x.size(3))
        elif x.ndim != 4:
            raise ValueError("Input must be 4D or 5D")
        return nn.functional.max_pool2d(x, self.kernel, self.stride,
                                        return_indices=self.return_indices)
