"""The HBM calibration streams (yh_hbm_stream) compute what they claim, so the
rates bench.py reports are rates of real copies, reads and writes."""
import pytest
import torch

from yanchor_amd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nt", [0, 1])
def test_streams(nt):
    dev = torch.device("cuda:0")
    n = (1 << 20) + 48  # floats: not a multiple of a workgroup's step
    src = torch.randn(n, device=dev)
    dst = torch.zeros(n, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    grid = 37
    _native.call("yh_hbm_stream", 0, nt, src.data_ptr(), dst.data_ptr(), n * 4, grid, st)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    _native.call("yh_hbm_stream", 1, nt, 0, dst.data_ptr(), n * 4, grid, st)
    torch.cuda.synchronize()
    assert torch.equal(dst, src * 0.5 + 1.0)  # the product by 0.5 is exact: no double rounding
    out = torch.zeros(n, device=dev)
    _native.call("yh_hbm_stream", 2, nt, src.data_ptr(), out.data_ptr(), n * 4, grid, st)
    torch.cuda.synchronize()
    total = out[:grid].double().sum().item()
    ref = src.double().sum().item()
    assert abs(total - ref) <= 1e-3 * src.double().abs().sum().item()
    _native.call("yh_hbm_stream", 3, nt, 0, dst.data_ptr(), n * 4, grid, st)
    torch.cuda.synchronize()
    v = dst.view(-1, 4)
    assert torch.all(v[:, 0] == 1.0) and torch.all(v[:, 1] == 2.0) and torch.all(v[:, 2] == 3.0)
    assert torch.all((v[:, 3] >= 0) & (v[:, 3] <= 3))
