"""The allocation-free GroupSum cross-entropy forward (cl_group_sum_cross_entropy_forward_noalloc,
its workspace in a device array of the library) against the workspace entry point
(cl_group_sum_cross_entropy_forward) through the C ABI: bitwise equal results on two calls in
a row, the second with a smaller input, and a clear error for a shape beyond the scratch
limit."""
import ctypes

import pytest
import torch

from compactlogic_amd import _capi

pytestmark = pytest.mark.gpu


def _with_workspace(x, labels, k, tau, ignore):
    batch, features = x.shape
    need = ctypes.c_int64()
    _capi.call("cl_group_sum_cross_entropy_workspace_size", 0, batch, features, k,
               ctypes.byref(need))
    ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty((batch, k), device=x.device)
    probs = torch.empty_like(out)
    loss = torch.empty((), device=x.device)
    count = torch.empty((), device=x.device)
    _capi.call("cl_group_sum_cross_entropy_forward", 0, x.data_ptr(), batch, features,
               x.stride(0), x.stride(1), k, tau, labels.data_ptr(), ignore, out.data_ptr(),
               probs.data_ptr(), loss.data_ptr(), count.data_ptr(), ws.data_ptr(), ws.numel(),
               torch.cuda.current_stream().cuda_stream)
    return out, probs, loss, count


def _no_alloc(x, labels, k, tau, ignore):
    batch, features = x.shape
    out = torch.empty((batch, k), device=x.device)
    probs = torch.empty_like(out)
    loss = torch.empty((), device=x.device)
    count = torch.empty((), device=x.device)
    _capi.call("cl_group_sum_cross_entropy_forward_noalloc", 0, x.data_ptr(), batch, features,
               x.stride(0), x.stride(1), k, tau, labels.data_ptr(), ignore, out.data_ptr(),
               probs.data_ptr(), loss.data_ptr(), count.data_ptr(),
               torch.cuda.current_stream().cuda_stream)
    return out, probs, loss, count


@pytest.mark.parametrize("case", [
    # (batch, features, k, tau), the second call smaller than the first
    [(1024, 12000, 10, 10.0), (300, 1000, 7, 2.0)],
    [(256, 16000, 10, 30.0), (64, 640, 10, 1.0)],
])
def test_no_alloc_matches_workspace_entry_point(device, case):
    g = torch.Generator().manual_seed(3)
    for batch, features, k, tau in case:
        # a LogicLayer's output as GroupSum sees it: the transposed view of [features, batch]
        x = torch.rand((features, batch), generator=g).to(device).t()
        labels = torch.randint(0, k, (batch,), generator=g).to(device)
        labels[::17] = -100                                  # some ignored samples
        ref = _with_workspace(x, labels, k, tau, -100)
        got = _no_alloc(x, labels, k, tau, -100)
        torch.cuda.synchronize()
        for r, o in zip(ref, got):
            assert torch.equal(r, o)
        assert torch.isfinite(got[2]) and float(got[3]) == float((labels != -100).sum())


def test_no_alloc_rejects_shapes_beyond_its_scratch(device):
    limit = ctypes.c_int64()
    _capi.call("cl_group_sum_cross_entropy_scratch_limit", ctypes.byref(limit))
    batch, features, k = 8192, 512 * 64, 512
    need = ctypes.c_int64()
    _capi.call("cl_group_sum_cross_entropy_workspace_size", 0, batch, features, k,
               ctypes.byref(need))
    assert need.value > limit.value
    x = torch.empty((features, 1), device=device).expand(features, batch).t()
    labels = torch.zeros(batch, dtype=torch.int64, device=device)
    with pytest.raises(_capi.CompactLogicError, match="limit"):
        _no_alloc(x, labels, k, 1.0, -100)
