"""Pins the MFMA operand / accumulator layout that every attention kernel assumes."""
import pytest
import torch

from pack3d_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,k", [(torch.bfloat16, 16), (torch.float16, 16), (torch.float32, 2)])
def test_mfma_layout(gpu, dtype, k):
    print(f"selftest mfma {dtype}", flush=True)
    gen = torch.Generator().manual_seed(1)
    a = torch.randn(32, k, generator=gen).to(dtype)
    b = torch.randn(k, 32, generator=gen).to(dtype)
    da, db = a.to(gpu), b.to(gpu)
    d = torch.full((32, 32), float("nan"), device=gpu)
    _lib.call("p3d_selftest_mfma", _lib.DTYPES[dtype], da.data_ptr(), db.data_ptr(), d.data_ptr(),
              _lib.stream_of(gpu))
    torch.cuda.synchronize()
    ref = a.double() @ b.double()
    torch.testing.assert_close(d.cpu().double(), ref, atol=1e-5, rtol=1e-5)
