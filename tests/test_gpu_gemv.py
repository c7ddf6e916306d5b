"""bdm_gemv (the decode-step linear map) against an FP32 torch reference of
F.linear: x @ W^T + bias with FP32 accumulation, rounded once.  BF16 outputs
within one BF16 ulp of the FP32 result rounded (accumulation order differs),
FP32 outputs within 1e-5 of the largest."""

import sys

import pytest
import torch

from _inputs import rel_err

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
@pytest.mark.parametrize('n,k', [(1, 8), (7, 2048), (2064, 2048), (8344, 2048), (2048, 5632), (50257, 2048)])
@pytest.mark.parametrize('rows', [1, 2, 3, 4])
def test_gemv_matches_fp32_linear(device, dtype, n, k, rows):
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(n * 7 + k + rows)
    x = torch.randn(rows, k, generator=gen).to(dtype).to(device)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(dtype).to(device)
    bias = torch.randn(n, generator=gen).to(dtype).to(device) if n % 2 == 0 else None
    announce('gemv', dtype, rows, n, k)
    y = ops.gemv(x, w, bias)
    ref = x.float() @ w.float().t()
    if bias is not None:
        ref = ref + bias.float()
    torch.cuda.synchronize()
    assert y.shape == (rows, n) and y.dtype == dtype
    if dtype == torch.float32:
        assert rel_err(y, ref) < 1e-5
    else:
        diff = (y.float() - ref.to(dtype).float()).abs()
        assert bool((diff <= ref.abs() * 2 ** -7 + 1e-6).all())


def test_linear_dispatch(device):
    """ops.linear takes the GEMV for 1-4 rows without autograd, the library
    GEMM otherwise; both agree with F.linear to rounding."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(96, 64, generator=gen).to(torch.bfloat16).to(device)
    for rows in (1, 4, 5, 64):
        x = torch.randn(rows, 64, generator=gen).to(torch.bfloat16).to(device)
        with torch.no_grad():
            y = ops.linear(x, w)
        ref = torch.nn.functional.linear(x.float(), w.float())
        assert rel_err(y, ref) < 1e-2
