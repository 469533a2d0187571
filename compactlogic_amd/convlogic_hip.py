"""Tensor-level mirror of the reference's ``convlogic_cuda`` extension
(compactlogic/cuda/convlogic.cpp:49-110), backed by libcompactlogic_hip.so.

Same function names, argument order, dtypes and output shapes.  ``backward_x`` is a
deterministic gather (the reference scatters with float atomics): it walks an inverse index
of the taps bucketed by (input channel, stride phase), built here on the device with
sync-free torch ops and cached per live offsets tensor.
"""
from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass

import torch

from . import _capi
from .difflogic_hip import _check, _same_device, dtype_code, ptr, stream_of


def _dims(x, w, stride, pad, ks):  # argument tuple of the forward entry points
    n, cin, h, wd = x.shape
    cout, g = w.shape
    return n, cin, h, wd, cout, g, stride, pad, ks


def _out_hw(h, w, stride, pad, ks):
    return (h + 2 * pad - ks) // stride + 1, (w + 2 * pad - ks) // stride + 1


def _check_offsets(offsets_ch, offsets_h, offsets_w, cout, g):
    if offsets_ch.dtype != torch.int32:
        raise RuntimeError("offsets_ch must be int32")
    if offsets_h.dtype != torch.int8 or offsets_w.dtype != torch.int8:
        raise RuntimeError("offsets_h and offsets_w must be int8")
    for t in (offsets_ch, offsets_h, offsets_w):
        if tuple(t.shape) != (2, cout, g):
            raise RuntimeError(f"offsets must be [2, {cout}, {g}], got {tuple(t.shape)}")


def forward(x, offsets_ch, offsets_h, offsets_w, w, gate_seq, stride, pad, ks):
    """y[N, Cout, Ho, Wo] = sum_g w * op_g(tap0, tap1) (convlogic_kernel.cu:140-188)."""
    for t, nm in ((x, "x"), (offsets_ch, "offsets_ch"), (offsets_h, "offsets_h"),
                  (offsets_w, "offsets_w"), (w, "w"), (gate_seq, "gate_seq")):
        _check(t, nm)
    _same_device(x, offsets_ch, offsets_h, offsets_w, w, gate_seq)
    d = _dims(x, w, stride, pad, ks)
    _check_offsets(offsets_ch, offsets_h, offsets_w, d[4], d[5])
    ho, wo = _out_hw(d[2], d[3], stride, pad, ks)
    if ho <= 0 or wo <= 0:
        raise RuntimeError(f"Invalid output shape: h_out={ho}, w_out={wo}")
    if w.dtype != x.dtype:
        raise RuntimeError("w must have the dtype of x")
    y = torch.empty((d[0], d[4], ho, wo), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_conv_forward", dtype_code(x), ptr(x), ptr(offsets_ch), ptr(offsets_h),
                   ptr(offsets_w), ptr(w), ptr(gate_seq), ptr(y), *d, stream_of(x))
    return y


def backward_w(x, offsets_ch, offsets_h, offsets_w, gate_seq, grad_y, stride, probs=None):
    """grad_w[Cout, G] = sum over n, oy, ox of grad_y * op_g(tap0, tap1)
    (convlogic_kernel.cu:385-430); the output plane comes from grad_y, as in the reference
    binding.  ``probs`` (optional, not in the reference) applies the softmax backward, so the
    result is the gradient of the logits."""
    for t, nm in ((x, "x"), (offsets_ch, "offsets_ch"), (offsets_h, "offsets_h"),
                  (offsets_w, "offsets_w"), (gate_seq, "gate_seq"), (grad_y, "grad_y")):
        _check(t, nm)
    if probs is not None:
        _check(probs, "probs")
    n, cin, h, wd = x.shape
    cout, g = gate_seq.shape
    _check_offsets(offsets_ch, offsets_h, offsets_w, cout, g)
    if tuple(grad_y.shape[:2]) != (n, cout):
        raise RuntimeError(f"grad_y must be [{n}, {cout}, h_out, w_out], got {tuple(grad_y.shape)}")
    dims = (n, cin, h, wd, cout, g, stride, grad_y.shape[2], grad_y.shape[3])
    need = ctypes.c_int64(0)
    _capi.call("cl_conv_backward_w_workspace", dtype_code(x), *dims, ctypes.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    grad_w = torch.empty((cout, g), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_conv_backward_w", dtype_code(x), ptr(x), ptr(offsets_ch), ptr(offsets_h),
                   ptr(offsets_w), ptr(gate_seq), ptr(grad_y), ptr(probs), ptr(grad_w), ptr(ws),
                   need.value, *dims, stream_of(x))
    return grad_w


_INDEX_CACHE: dict = {}


def inverse_index(offsets_ch, offsets_h, offsets_w, c_in, stride):
    """(inv_ptr int32 [c_in * s^2 + 1], inv_ent int32 [2 * Cout * G]) with the taps bucketed
    by (channel, dh mod s, dw mod s); entries 2 * (c * G + g) + side in ascending order inside
    a bucket.  Built with device ops that do not synchronise.  Cached per offsets tensor
    object: an entry is reused only while the very same tensors are alive, unmodified (same
    version counter and storage), so a freed tensor whose memory is reused never hits."""
    key = (id(offsets_ch), id(offsets_h), id(offsets_w), int(c_in), int(stride))
    state = tuple((t.data_ptr(), t._version) for t in (offsets_ch, offsets_h, offsets_w))
    hit = _INDEX_CACHE.get(key)
    if hit is not None:
        refs, hit_state, out = hit
        if all(r() is t for r, t in zip(refs, (offsets_ch, offsets_h, offsets_w))) and hit_state == state:
            return out
    s = int(stride)
    _, cout, g = offsets_ch.shape
    dev = offsets_ch.device
    ch = offsets_ch.reshape(2, -1).t().reshape(-1).to(torch.int64)        # order: (c, g, side)
    dh = torch.remainder(offsets_h.reshape(2, -1).t().reshape(-1).to(torch.int64), s)
    dw = torch.remainder(offsets_w.reshape(2, -1).t().reshape(-1).to(torch.int64), s)
    ent = torch.arange(2 * cout * g, dtype=torch.int64, device=dev)       # 2 * (c*G+g) + side
    valid = (ch >= 0) & (ch < c_in)
    nb = c_in * s * s
    key_b = torch.where(valid, ch * s * s + dh * s + dw, torch.full_like(ch, nb))
    order = torch.sort(key_b, stable=True).indices
    counts = torch.zeros(nb + 1, dtype=torch.int64, device=dev)
    counts.index_add_(0, key_b, torch.ones_like(key_b))
    inv_ptr = torch.zeros(nb + 1, dtype=torch.int64, device=dev)
    inv_ptr[1:] = torch.cumsum(counts[:nb], 0)
    out = (inv_ptr.to(torch.int32).contiguous(), ent[order].to(torch.int32).contiguous())
    live = {k: v for k, v in _INDEX_CACHE.items() if all(r() is not None for r in v[0])}
    _INDEX_CACHE.clear()
    _INDEX_CACHE.update(live)
    _INDEX_CACHE[key] = (tuple(weakref.ref(t) for t in (offsets_ch, offsets_h, offsets_w)), state, out)
    return out


@dataclass
class WindowPlan:
    """Tables of the window path (every output channel reads one input channel; all taps in a
    kw x kw window at offset (oy0, ox0) of the output position times the stride)."""
    kw: int
    oy0: int
    ox0: int
    width: int                # coefficients per channel
    max_group: int            # most output channels reading one input channel
    slot_win: torch.Tensor    # int32 [Cout, G]: window index of operand a | of operand b << 8
    grp_ptr: torch.Tensor     # int32 [Cin + 1]
    chan_order: torch.Tensor  # int32 [Cout]


_WINDOW_CACHE: dict = {}


def window_plan(offsets_ch, offsets_h, offsets_w, c_in: int):
    """The WindowPlan of these offsets, or None when some output channel reads more than one
    input channel or the taps span more than a 3 x 3 window.  Cached like inverse_index (the
    eligibility test reads a few scalars back from the device once per offsets version)."""
    key = (id(offsets_ch), id(offsets_h), id(offsets_w), int(c_in))
    state = tuple((t.data_ptr(), t._version) for t in (offsets_ch, offsets_h, offsets_w))
    hit = _WINDOW_CACHE.get(key)
    if hit is not None:
        refs, hit_state, out = hit
        if all(r() is t for r, t in zip(refs, (offsets_ch, offsets_h, offsets_w))) and hit_state == state:
            return out
    out = _build_window_plan(offsets_ch, offsets_h, offsets_w, int(c_in))
    live = {k: v for k, v in _WINDOW_CACHE.items() if all(r() is not None for r in v[0])}
    _WINDOW_CACHE.clear()
    _WINDOW_CACHE.update(live)
    _WINDOW_CACHE[key] = (tuple(weakref.ref(t) for t in (offsets_ch, offsets_h, offsets_w)), state, out)
    return out


def _build_window_plan(offsets_ch, offsets_h, offsets_w, c_in: int):
    _, cout, g = offsets_ch.shape
    if cout == 0 or g > 64:
        return None
    dev = offsets_ch.device
    ch = offsets_ch.to(torch.int64)
    first = ch[0, :, :1]
    stats = torch.stack((
        (ch != first.unsqueeze(0)).any().to(torch.int64),
        ((first < 0) | (first >= c_in)).any().to(torch.int64),
        offsets_h.min().to(torch.int64), offsets_h.max().to(torch.int64),
        offsets_w.min().to(torch.int64), offsets_w.max().to(torch.int64))).tolist()
    mixed, out_of_range, hmin, hmax, wmin, wmax = stats
    kw = max(hmax - hmin, wmax - wmin) + 1
    if mixed or out_of_range or kw > 3:
        return None
    win = (offsets_h.to(torch.int64) - hmin) * kw + (offsets_w.to(torch.int64) - wmin)
    slot_win = (win[0] | (win[1] << 8)).to(torch.int32).contiguous()
    chan = first.squeeze(1)
    chan_order = torch.sort(chan, stable=True).indices
    counts = torch.bincount(chan, minlength=c_in)
    grp_ptr = torch.zeros(c_in + 1, dtype=torch.int64, device=dev)
    grp_ptr[1:] = torch.cumsum(counts, 0)
    width = ctypes.c_int64(0)
    _capi.call("cl_conv_window_coef_width", kw, ctypes.byref(width))
    return WindowPlan(kw=int(kw), oy0=int(hmin), ox0=int(wmin), width=width.value,
                      max_group=int(counts.max()), slot_win=slot_win,
                      grp_ptr=grp_ptr.to(torch.int32).contiguous(),
                      chan_order=chan_order.to(torch.int32).contiguous())


def backward_x(x, offsets_ch, offsets_h, offsets_w, w, gate_seq, grad_y, stride, pad, index=None):
    """grad_x like x (convlogic_kernel.cu:248-293), as a deterministic gather.  ``pad`` is
    accepted for the reference signature; the taps already carry the padding shift.
    ``index`` (optional) is inverse_index() of these offsets, taken earlier."""
    del pad
    for t, nm in ((x, "x"), (offsets_ch, "offsets_ch"), (offsets_h, "offsets_h"),
                  (offsets_w, "offsets_w"), (w, "w"), (gate_seq, "gate_seq"), (grad_y, "grad_y")):
        _check(t, nm)
    n, cin, h, wd = x.shape
    cout, g = w.shape
    _check_offsets(offsets_ch, offsets_h, offsets_w, cout, g)
    if tuple(grad_y.shape[:2]) != (n, cout):
        raise RuntimeError(f"grad_y must be [{n}, {cout}, h_out, w_out], got {tuple(grad_y.shape)}")
    if index is None:
        index = inverse_index(offsets_ch, offsets_h, offsets_w, cin, stride)
    inv_ptr, inv_ent = index
    grad_x = torch.empty_like(x)
    with torch.cuda.device(x.device):
        _capi.call("cl_conv_backward_x", dtype_code(x), ptr(x), ptr(offsets_ch), ptr(offsets_h),
                   ptr(offsets_w), ptr(w), ptr(gate_seq), ptr(grad_y), ptr(inv_ptr), ptr(inv_ent),
                   ptr(grad_x), n, cin, h, wd, cout, g, stride, grad_y.shape[2], grad_y.shape[3],
                   stream_of(x))
    return grad_x


def eval(x, offsets_ch, offsets_h, offsets_w, w, gate_seq, stride, pad, ks):  # noqa: A001
    """Discrete conv with the argmax slot w[c] (convlogic_kernel.cu:479-530)."""
    for t, nm in ((x, "x"), (offsets_ch, "offsets_ch"), (offsets_h, "offsets_h"),
                  (offsets_w, "offsets_w"), (w, "w"), (gate_seq, "gate_seq")):
        _check(t, nm)
    if w.dtype != torch.uint8:
        raise RuntimeError("w must hold uint8 slot indices")
    n, cin, h, wd = x.shape
    cout, g = gate_seq.shape
    ho, wo = _out_hw(h, wd, stride, pad, ks)
    if ho <= 0 or wo <= 0:
        raise RuntimeError(f"Invalid output shape: h_out={ho}, w_out={wo}")
    y = torch.empty((n, cout, ho, wo), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_conv_eval", dtype_code(x), ptr(x), ptr(offsets_ch), ptr(offsets_h),
                   ptr(offsets_w), ptr(w), ptr(gate_seq), ptr(y), n, cin, h, wd, cout, g, stride,
                   pad, ks, stream_of(x))
    return y


def eval_packed_indexed(x, ia, ib, gate, order=None):
    """Packed layer from index tables (int32, -1 = zero row): y[o] = op(x[ia[o]], x[ib[o]]).
    `order` (int32, a permutation of the output rows) is the order the rows are evaluated in."""
    for t, nm in ((x, "x"), (ia, "ia"), (ib, "ib"), (gate, "gate")):
        _check(t, nm)
    out_dim = ia.numel()
    if order is not None:
        _check(order, "order")
        if order.dtype != torch.int32 or order.numel() != out_dim:
            raise RuntimeError("order must be int32 with one entry per output row")
    y = torch.empty((out_dim, x.shape[1]), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _capi.call("cl_eval_packed_indexed", ptr(x), ptr(ia), ptr(ib), ptr(gate), ptr(order),
                   ptr(y), x.shape[0], out_dim, x.shape[1] * x.element_size(), stream_of(x))
    return y
