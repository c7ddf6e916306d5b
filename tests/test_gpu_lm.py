"""The language-model shell on the GPU.

* ``bdm_rms_norm`` and ``bdm_swiglu`` against torch's FP32 formulas of
  _shell.py:29-35 and :86-91 (tolerances in each test).
* The whole model (FP32 weights) against the reference's logits, loss and
  gradients in tests/golden/lm_small.pt.
* Stateful inference: ``prefill`` then ``step`` against the oracle shell's,
  FP32 weights and caches (routes on FP32 scores have no near-ties).
"""

import os
import sys

import pytest
import torch
import torch.nn.functional as F

from _inputs import rel_err
from conftest import ROOT
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'lm_small.pt')


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def close_rows(out, ref, dtype):
    """BF16: each element within one BF16 ulp of torch's (ulp <= 2^-7 of the
    value); FP32: within 1e-5 relative."""
    tol = 2 ** -7 if dtype == torch.bfloat16 else 1e-5
    return float(((out.float() - ref.float()).abs() / ref.float().abs().clamp_min(1e-3)).max()) <= tol


def torch_rms(x, weight, eps):
    out = x.float() * torch.rsqrt((x.float() * x.float()).mean(-1, keepdim=True) + eps)
    return (out * weight.float()).to(x.dtype)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
@pytest.mark.parametrize('width', [32, 520, 2048, 5120])
def test_rms_norm_matches_torch(device, dtype, width):
    """FP32 sums in another order: BF16 results within one ulp, FP32 within
    1e-5 relative; the residual sum is exact (one rounding)."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(width)
    x = (torch.randn(37, width, generator=gen) * 3).to(dtype).to(device)
    r = torch.randn(37, width, generator=gen).to(dtype).to(device)
    weight = (1 + 0.1 * torch.randn(width, generator=gen)).to(device)
    announce('rms_norm', dtype, width)
    for wdt in (torch.float32, torch.bfloat16):
        w = weight.to(wdt)
        out = ops.rms_norm(x, w, 1e-5)
        ref = torch_rms(x, w, 1e-5)
        assert close_rows(out, ref, dtype)
        total, normed = ops.rms_norm(x, w, 1e-5, residual=r)
        assert torch.equal(total, r + x)
        ref = torch_rms(r + x, w, 1e-5)
        assert close_rows(normed, ref, dtype)
    torch.cuda.synchronize()


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
@pytest.mark.parametrize('width', [8, 520, 2048, 4096])
def test_rms_norm_backward_matches_float64(device, dtype, width):
    """Gradients of the shell's RMSNorm from ``bdm_rms_norm_backward`` against
    the exact (float64) derivative, with torch's autograd of the reference's
    chain in the same dtype as the yardstick: our error at most twice torch's
    plus an FP32 rounding.  100 rows: a ragged last block of 32 rows."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(width + 1)
    x = (torch.randn(100, width, generator=gen) * 2).to(dtype)
    dy = torch.randn(100, width, generator=gen).to(dtype)
    for wdt in (torch.float32, torch.bfloat16):
        weight = (1 + 0.1 * torch.randn(width, generator=gen)).to(wdt)
        x64 = x.double().requires_grad_(True)
        w64 = weight.double().requires_grad_(True)
        y64 = x64 * torch.rsqrt((x64 * x64).mean(-1, keepdim=True) + 1e-5) * w64
        dx64, dw64 = torch.autograd.grad(y64, (x64, w64), dy.double())
        xt = x.to(device).requires_grad_(True)
        wt = weight.to(device).requires_grad_(True)
        dxt, dwt = torch.autograd.grad(torch_rms(xt, wt, 1e-5), (xt, wt), dy.to(device))
        announce('rms_norm_backward', dtype, width, wdt)
        dx, dw = ops.rms_norm_backward(x.to(device), dy.to(device), weight.to(device), 1e-5)
        torch.cuda.synchronize()
        assert dx.dtype == dtype and dw.dtype == wdt
        for ours, yard, exact in ((dx, dxt, dx64), (dw, dwt, dw64)):
            exact = exact.to(device)
            err = float((ours.double() - exact).abs().max())
            bound = 2 * float((yard.double() - exact).abs().max()) + 1e-6 * float(exact.abs().max())
            assert err <= bound, (err, bound)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_swiglu_matches_torch(device, dtype):
    """silu(x1) * x3 with torch's rounding points: BF16 equal but for
    one-ulp exp differences (checked as at most 1 % of elements, each within
    one ulp), FP32 within 1e-6."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(5)
    hidden = 5632
    gate_up = (torch.randn(19, 2 * hidden, generator=gen) * 4).to(dtype).to(device)
    announce('swiglu', dtype)
    out = ops.swiglu(gate_up, hidden)
    ref = F.silu(gate_up[:, :hidden]) * gate_up[:, hidden:]
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert rel_err(out, ref) < 1e-6
    else:
        diff = (out.float() - ref.float()).abs()
        ulp = ref.float().abs() * 2 ** -7
        assert bool((diff <= ulp).all())
        assert float((diff > 0).float().mean()) < 0.01


def _golden_model(device):
    from bdm_amd import BSDMConfig
    from bdm_amd.lm import BDMLanguageModel, LanguageModelConfig
    golden = torch.load(GOLDEN, weights_only=True)
    dim, j, s, k, v, h, vocab, layers, multiple, seed = golden['geometry'].tolist()
    memory = BSDMConfig(dim=dim, bank_count=j, bank_size=s, selected_banks=k, value_width=v, num_heads=h)
    config = LanguageModelConfig(memory=memory, vocab_size=vocab, layers=layers, ffn_multiple_of=multiple,
                                 seed=seed)
    model = BDMLanguageModel(config)
    model.load_state_dict(golden['state'])
    return golden, memory, config, model.to(device)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_swiglu_training_pair_matches_autograd(device, dtype):
    """bdm_swiglu_pair and bdm_swiglu_backward against torch's F.silu(a) * b
    and its autograd in the same dtype: BF16 within one ulp (at most 2 % of
    elements differ: exp and rounding order), FP32 within 1e-5.  37 x 1001
    elements: a ragged tail past the last group of 8."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(11)
    a = (torch.randn(37, 1001, generator=gen) * 4).to(dtype).to(device)
    b = torch.randn(37, 1001, generator=gen).to(dtype).to(device)
    dy = torch.randn(37, 1001, generator=gen).to(dtype).to(device)
    announce('swiglu pair', dtype)
    out = ops.swiglu_pair(a, b)
    ga, gb = ops.swiglu_backward(a, b, dy)
    at, bt = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    ref = F.silu(at) * bt
    ra, rb = torch.autograd.grad(ref, (at, bt), dy)
    torch.cuda.synchronize()
    for ours, theirs in ((out, ref.detach()), (ga, ra), (gb, rb)):
        if dtype == torch.float32:
            assert rel_err(ours, theirs) < 1e-5
        else:
            diff = (ours.float() - theirs.float()).abs()
            assert bool((diff <= theirs.float().abs() * 2 ** -7 + 1e-30).all())
            assert float((diff > 0).float().mean()) < 0.02


def test_lm_matches_reference_fixture(device):
    """FP32 weights; the layer rounds its training state to BF16 every 16
    events as the reference does.  Logits within 1e-4 of the largest, loss
    within 1e-5, gradients of the loss within 2e-2 per tensor."""
    golden, _, _, model = _golden_model(device)
    tokens, target = golden['tokens'].to(device), golden['target'].to(device)
    announce('lm fixture forward')
    logits = model(tokens)
    assert rel_err(logits, golden['logits']) < 1e-4, rel_err(logits, golden['logits'])
    loss = model(tokens, target)
    assert float(loss.detach()) == pytest.approx(float(golden['loss']), rel=1e-5)
    announce('lm fixture backward')
    loss.backward()
    torch.cuda.synchronize()
    params = dict(model.named_parameters())
    for name, grad in golden['grads'].items():
        assert rel_err(params[name].grad, grad) < 2e-2, (name, rel_err(params[name].grad, grad))


@pytest.mark.parametrize('batch', [2, 1])
def test_lm_prefill_and_step_match_oracle(device, batch):
    """FP32 weights and caches; our prefill (fused projections, shell
    kernels, HIP recurrence) and steps (decode GEMVs with fused prologues; at
    batch 1 both route roles in one launch) against the oracle shell's.
    Logits within 1e-3 of the largest, caches within 1e-3."""
    golden, memory, config, model = _golden_model(device)
    oracle = O.OracleLanguageModel(memory, vocab_size=config.vocab_size, layers=config.layers,
                                   multiple_of=config.ffn_multiple_of, seed=config.seed)
    oracle.load_state_dict(golden['state'])
    tokens = golden['tokens'][:batch]
    with torch.no_grad():
        announce('lm prefill', batch)
        caches = [block.attention.create_state(batch, dtype=torch.float32) for block in model.layers]
        ref_caches = [block.attention.create_state(batch, torch.float32) for block in oracle.layers]
        logits, caches = model.prefill(tokens[:, :14].to(device), caches)
        ref, ref_caches = oracle.prefill(tokens[:, :14], ref_caches)
        assert rel_err(logits, ref) < 1e-3, rel_err(logits, ref)
        for c, rc in zip(caches, ref_caches):
            assert rel_err(c, rc) < 1e-3
        for t in range(14, 18):
            announce('lm step', t)
            logits, caches = model.step(tokens[:, t:t + 1].to(device), caches)
            ref, ref_caches = oracle.step(tokens[:, t:t + 1], ref_caches)
            assert rel_err(logits, ref) < 1e-3, (t, rel_err(logits, ref))
        torch.cuda.synchronize()


def test_lm_graph_decoder_matches_eager_steps(device):
    """The whole model's decode step replayed from one HIP graph equals the
    eager steps bit for bit, logits and every layer's cache, with unrelated
    eager work and synchronizations between replays."""
    from bdm_amd import LanguageModelGraphDecoder
    golden, _, _, model = _golden_model(device)
    model = model.to(torch.bfloat16)
    tokens = golden['tokens'].to(device)
    announce('lm graph decoder')
    with torch.no_grad():
        _, caches = model.prefill(tokens[:, :10])
        eager = [c.clone() for c in caches]
        graph = [c.clone() for c in caches]
        decoder = LanguageModelGraphDecoder(model, graph)
        for a, b in zip(graph, caches):
            assert torch.equal(a, b)  # building the graph leaves the caches untouched
        noise = torch.randn(1 << 20, device=device)
        for t in range(10, 18):
            want, eager = model.step(tokens[:, t:t + 1], eager)
            got = decoder.step(tokens[:, t:t + 1])
            assert torch.equal(got, want), t
            for a, b in zip(graph, eager):
                assert torch.equal(a, b), t
            noise.mul_(0.5).add_(1.0)
            torch.cuda.synchronize()
