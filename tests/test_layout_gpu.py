"""cl_transpose, the layout change between [batch, features] and [features, batch] rows
(compactlogic/compactlogic.py:100-101 does it with a torch transpose copy): bit-exact against
numpy's transpose for the 16-byte fp32 path (whole and partial 32 x 32 tiles), the general
path (sizes not divisible by 4, fp64) and the cfg2 input."""
import numpy as np
import pytest
import torch

from compactlogic_amd import _capi
from compactlogic_amd import difflogic_hip as _dl

pytestmark = pytest.mark.gpu


def transpose(x):
    rows, cols = x.shape
    out = torch.empty((cols, rows), dtype=x.dtype, device=x.device)
    _capi.call("cl_transpose", _dl.dtype_code(x), x.data_ptr(), out.data_ptr(), rows, cols,
               torch.cuda.current_stream(x.device).cuda_stream)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("shape,dtype", [
    ((1024, 784), torch.float32),   # cfg2 input: 16-byte path, partial tiles along the columns
    ((100, 36), torch.float32),     # 16-byte path, partial tiles both ways
    ((4, 4), torch.float32),
    ((64, 96), torch.float32),      # whole tiles only
    ((37, 53), torch.float32),      # general path
    ((70, 130), torch.float64),
    ((1, 9), torch.float64),
])
def test_transpose_is_exact(device, shape, dtype):
    g = torch.Generator().manual_seed(shape[0] * 1000 + shape[1])
    x = torch.randn(shape, generator=g, dtype=dtype)
    got = transpose(x.to(device)).cpu().numpy()
    np.testing.assert_array_equal(got, x.numpy().T)


def test_transpose_of_a_misaligned_view_takes_the_general_path(device):
    base = torch.randn(1 + 64 * 48, device=device)
    x = base[1:].view(64, 48)  # 4-byte offset: not 16-byte aligned
    np.testing.assert_array_equal(transpose(x).cpu().numpy(), x.cpu().numpy().T)
