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


@pytest.mark.parametrize('n,k', [(3456, 1024), (1024, 1024), (1000, 96), (17, 2048), (64, 4128)])
@pytest.mark.parametrize('rows', [5, 16, 17, 33, 48, 64])
def test_skinny_matches_fp32_linear(device, n, k, rows):
    """5 to 64 BF16 rows (a decode batch) take the matrix-core tiles: within
    one BF16 rounding of the FP32 product plus the FP32 sum-order error, for
    ragged row counts, ragged column counts and K past one load chunk."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(n * 3 + k + rows)
    x = torch.randn(rows, k, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(n, k, generator=gen) * k ** -0.5).to(torch.bfloat16).to(device)
    bias = torch.randn(n, generator=gen).to(torch.bfloat16).to(device) if n % 2 == 0 else None
    announce('skinny', rows, n, k)
    y = ops.gemv(x, w, bias)
    x64, w64 = x.double(), w.double()
    ref = x64 @ w64.t()
    if bias is not None:
        ref = ref + bias.double()
    magnitude = x64.abs() @ w64.abs().t() + (bias.double().abs() if bias is not None else 0)
    torch.cuda.synchronize()
    assert y.shape == (rows, n) and y.dtype == torch.bfloat16
    diff = (y.double() - ref).abs()
    assert bool((diff <= ref.abs() * 2.0 ** -8 + magnitude * k * 2.0 ** -23 + 1e-30).all())
    # and the library GEMM agrees to a BF16 rounding or two
    lib = torch.nn.functional.linear(x, w, bias)
    assert bool(((y.float() - lib.float()).abs() <= lib.float().abs() * 2 ** -6 + 1e-3).all())


def test_linear_dispatch(device):
    """ops.linear takes the GEMV for 1-4 rows and the matrix-core tiles for
    5-64 BF16 rows without autograd, the library GEMM otherwise; all agree
    with F.linear to rounding."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(3)
    w = torch.randn(96, 64, generator=gen).to(torch.bfloat16).to(device)
    for rows in (1, 4, 5, 64, 65):
        x = torch.randn(rows, 64, generator=gen).to(torch.bfloat16).to(device)
        with torch.no_grad():
            y = ops.linear(x, w)
        ref = torch.nn.functional.linear(x.float(), w.float())
        assert rel_err(y, ref) < 1e-2


def _rows(rows, k, gen, dtype, device, scale=1.0):
    return (torch.randn(rows, k, generator=gen) * scale).to(dtype).to(device)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
@pytest.mark.parametrize('rows', [1, 3])
@pytest.mark.parametrize('k', [520, 2048])
def test_gemv_prologues_equal_the_unfused_kernels(device, dtype, rows, k):
    """Each prologue of bdm_gemv_ex gives exactly the output of its standalone
    kernel followed by the plain GEMV (and the RMS prologue's residual sum
    equals rms_norm's); the one exception, FP32 layer norm, is within an
    FP32 ulp of it."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(k + rows)
    n = 1000
    w = _rows(n, k, gen, dtype, device, k ** -0.5)
    bias = _rows(1, n, gen, dtype, device)[0]
    x = _rows(rows, k, gen, dtype, device, 2.0)
    res = _rows(rows, k, gen, dtype, device)
    for pdt in (torch.float32, torch.bfloat16):
        nw = (1 + 0.1 * torch.randn(k, generator=gen)).to(pdt).to(device)
        nb = (0.1 * torch.randn(k, generator=gen)).to(pdt).to(device)
        announce('gemv prologues', dtype, rows, k, pdt)
        # RMSNorm, plain and after a residual add
        y = ops.gemv_fused(x, w, bias, prologue='rms', norm_weight=nw, eps=1e-5)
        assert torch.equal(y, ops.gemv(ops.rms_norm(x, nw, 1e-5), w, bias))
        y, total = ops.gemv_fused(x, w, bias, prologue='rms', residual=res, norm_weight=nw, eps=1e-5)
        want_total, normed = ops.rms_norm(x, nw, 1e-5, residual=res)
        assert torch.equal(total, want_total) and torch.equal(y, ops.gemv(normed, w, bias))
        # the output interface: layer norm or RMS norm, times sigmoid(gate); the gate a strided slice
        wide = _rows(rows, 3 * k, gen, dtype, device)
        gate = wide[:, k:2 * k]
        for kind in ('layer', 'rms'):
            y = ops.gemv_fused(x, w, bias, prologue='out_' + kind, norm_weight=nw,
                               norm_bias=nb if kind == 'layer' else None, gate=gate, eps=1e-5)
            normed = ops.output_epilogue(x, gate, nw, nb if kind == 'layer' else None, eps=1e-5, kind=kind)
            want = ops.gemv(normed, w, bias)
            if kind == 'layer' and dtype == torch.float32:
                # FP32 layer norm: the row mean may differ in its last bit from the standalone
                # kernel's (widths not a multiple of 512), so the input within one FP32 ulp
                assert rel_err(y, want) < 1e-6, (kind, rel_err(y, want))
            else:
                assert torch.equal(y, want), kind
    # SwiGLU of a [rows, 2k] row
    gu = _rows(rows, 2 * k, gen, dtype, device, 3.0)
    y = ops.gemv_fused(gu, w, None, prologue='swiglu')
    assert torch.equal(y, ops.gemv(ops.swiglu(gu, k), w))
    torch.cuda.synchronize()


def test_lm_fused_decode_equals_unfused(device):
    """The whole model's decode step with the elementwise kernels fused into
    the GEMVs equals the unfused step bit for bit (logits and caches)."""
    from bdm_amd import BSDMConfig
    from bdm_amd.lm import BDMLanguageModel, LanguageModelConfig
    memory = BSDMConfig(dim=256, bank_count=64, bank_size=8, selected_banks=4, value_width=512, num_heads=2)
    config = LanguageModelConfig(memory=memory, vocab_size=1000, layers=3, seed=2)
    model = BDMLanguageModel(config).to(device=device, dtype=torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(4)
    tokens = torch.randint(0, 1000, (2, 30), generator=gen).to(device)
    announce('lm fused decode')
    with torch.no_grad():
        _, caches = model.prefill(tokens[:, :20])
        fused = [c.clone() for c in caches]
        plain = [c.clone() for c in caches]
        assert model._fused_decode_supported(model.tok_embeddings(tokens[:, :1]))
        for t in range(20, 26):
            got, fused = model.step(tokens[:, t:t + 1], fused)
            model._fused_decode_supported = lambda h: False  # the unfused kernels, for comparison
            want, plain = model.step(tokens[:, t:t + 1], plain)
            del model._fused_decode_supported
            assert torch.equal(got, want), t
            for a, b in zip(fused, plain):
                assert torch.equal(a, b), t
        torch.cuda.synchronize()
