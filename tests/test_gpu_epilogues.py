"""Inference epilogues against the torch ops they replace, on identical inputs.

The controller epilogue and the output epilogue are compared with the layer's
own torch formulas, and the controller epilogue also with the CPU oracle's
controllers on the same weights (heads.controllers, heads.py:11-22; _normalize_qk and
_project_bank_output, _parameters.py:214-232) applied to the same projection
matrix.  BF16 results may differ by one BF16 ulp (exp/log1p/rsqrt of the
device libm against torch's), FP32 g by 1e-5 relative.  End to end, prefill
and step with the fused projection are checked against the oracle in
test_gpu_parity.py.
"""

import sys

import pytest
import torch
import torch.nn.functional as F

from _inputs import rel_err

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def within_ulp(ours, ref, ulps=1):
    """|ours - ref| <= ulps BF16 ulps of |ref| (or of the FP32 type's epsilon)."""
    ours, ref = ours.float(), ref.float()
    step = 2 ** -7 if ours.dtype == torch.bfloat16 else 2 ** -7
    return bool(((ours - ref).abs() <= ulps * step * ref.abs() + 1e-30).all())


def _layer(device, dtype, qk, norm, dim=128, value_width=256, heads=4, bank_size=8):
    from bdm_amd import BDMConfig, BankedDeltaMemory
    cfg = BDMConfig(dim=dim, bank_count=64, bank_size=bank_size, selected_banks=4, value_width=value_width,
                    num_heads=heads, routed_decay=True, qk_normalization=qk, output_normalization=norm,
                    output_bias=True)
    layer = BankedDeltaMemory(cfg, layer_id=2, seed=7).to(device=device, dtype=dtype)
    with torch.no_grad():  # nonzero router residuals and biases, so every summed term matters
        for p in layer.shared_router.parameters():
            p.add_(torch.randn_like(p) * 0.05)
        layer.output_gate.bias.add_(torch.randn_like(layer.output_gate.bias) * 0.1)
        layer.dt_bias.add_(torch.randn_like(layer.dt_bias) * 0.5)
    return layer


@pytest.mark.parametrize('qk', ['nvidia', 'original'])
@pytest.mark.parametrize('bank_size', [8, 16])
def test_controller_epilogue_matches_torch_ops(device, qk, bank_size):
    from bdm_amd import ops
    layer = _layer(device, torch.bfloat16, qk, 'layer', bank_size=bank_size)
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 37, layer.hidden_size, generator=gen) * 2).to(torch.bfloat16).to(device)
    announce('controller epilogue', qk, bank_size)
    with torch.no_grad():
        (q, k, v, g, b, w), (rr, wr), gate = layer._fused_controllers(x)
        weight, bias, cols = layer._fused_weights()
        # the projections through the layer's own linear map (the matrix-core
        # tiles at these 111 rows), so the check isolates the epilogue
        proj = ops.linear(x.reshape(-1, layer.hidden_size), weight, bias)
        hs, hv, vw = layer.num_heads * layer.bank_size, layer.head_value_width, layer.value_width
        sl = lambda name, width: proj[:, cols[name]:cols[name] + width]  # noqa: E731
        shape = (-1, layer.num_heads, layer.bank_size)
        ref_q = layer._normalize_qk(F.silu(sl('q', hs)).reshape(shape))
        ref_k = layer._normalize_qk(F.silu(sl('k', hs)).reshape(shape))
        ref_v = F.silu(sl('v', vw))
        f = ops.linear(sl('f', hv), layer.f_proj[1].weight)
        ref_g = -layer.A_log.float().exp()[:, None] * F.softplus((f.float() + layer.dt_bias.float()).reshape(shape))
        ref_b = sl('b', hs).sigmoid()
        ref_w = sl('w', vw).sigmoid()
        torch.cuda.synchronize()
    assert within_ulp(q.reshape(shape), ref_q) and within_ulp(k.reshape(shape), ref_k)
    assert within_ulp(v.reshape(-1, vw), ref_v)
    assert within_ulp(b.reshape(-1, hs), ref_b) and within_ulp(w.reshape(-1, vw), ref_w)
    assert rel_err(g.reshape(shape), ref_g) < 1e-5
    # the scores and the gate are the projection's own columns (no copy)
    rw = layer.factor_route_width
    assert torch.equal(rr.reshape(-1, rw), sl('read', rw)) and torch.equal(wr.reshape(-1, rw), sl('write', rw))
    assert torch.equal(gate, sl('gate', vw))
    # the concatenated weight equals the modules' own projections
    with torch.no_grad():
        ref_rr, ref_wr = layer._route_projections(x)
        assert rel_err(rr.reshape(ref_rr.shape), ref_rr) < 1e-2 and rel_err(wr.reshape(ref_wr.shape), ref_wr) < 1e-2


@pytest.mark.parametrize('qk', ['nvidia', 'original'])
def test_controller_epilogue_matches_oracle_controllers(device, qk):
    """The fused projection + controller epilogue against the CPU oracle's own
    controllers and router scores (heads.py:11-22, _parameters.py:189-220,
    routing.py:23-35) on the same weights: GPU and CPU GEMMs round
    differently, so BF16 outputs agree to a few BF16 ulps of each row."""
    from oracle import bdm_oracle as O
    layer = _layer(device, torch.bfloat16, qk, 'layer')
    oracle = O.OracleBankedDeltaMemory(layer.config, layer_id=2, seed=7).to(torch.bfloat16)
    oracle.load_state_dict({k_: t.cpu() for k_, t in layer.state_dict().items()})
    gen = torch.Generator().manual_seed(55)
    x = torch.randn(2, 41, layer.hidden_size, generator=gen).to(torch.bfloat16)
    announce('controller epilogue vs oracle', qk)
    with torch.no_grad():
        (q, k, v, g, b, w), (rr, wr), _ = layer._fused_controllers(x.to(device))
        torch.cuda.synchronize()
        ref = oracle.controllers(x)
        ref_rr, ref_wr = oracle.shared_router.read(x), oracle.shared_router.write(x)
    for name, ours, theirs in zip('qkvgbw', (q, k, v, g, b, w), ref):
        width = theirs.shape[-1]
        err = rel_err(ours.reshape(-1, width), theirs.reshape(-1, width))
        assert ours.dtype == theirs.dtype, name
        assert err < 2e-2, (name, err)
    width = ref_rr.shape[-1]
    assert rel_err(rr.reshape(-1, width), ref_rr.reshape(-1, width)) < 2e-2
    assert rel_err(wr.reshape(-1, width), ref_wr.reshape(-1, width)) < 2e-2


@pytest.mark.parametrize('norm', ['layer', 'rms'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_output_epilogue_matches_torch_ops(device, norm, dtype):
    from bdm_amd import ops
    layer = _layer(device, dtype, 'nvidia', norm)
    gen = torch.Generator().manual_seed(6)
    n, vw = 301, layer.value_width
    raw = (torch.randn(n, vw, generator=gen) * 3 + 0.5).to(dtype).to(device)
    wide = torch.randn(n, vw + 40, generator=gen).to(dtype).to(device)
    gate = wide[:, 24:24 + vw]  # a strided slice, as the fused projection hands it over
    with torch.no_grad():
        layer.output_norm_weight.mul_(1 + 0.2 * torch.randn_like(layer.output_norm_weight))
        if norm == 'layer':
            layer.output_norm_bias.add_(0.1 * torch.randn_like(layer.output_norm_bias))
    announce('output epilogue', norm, dtype)
    with torch.no_grad():
        ours = ops.output_epilogue(raw, gate, layer.output_norm_weight,
                                   layer.output_norm_bias if norm == 'layer' else None, eps=layer.norm_eps,
                                   kind=norm)
        if norm == 'layer':
            normalized = F.layer_norm(raw, (vw,), layer.output_norm_weight, layer.output_norm_bias, layer.norm_eps)
        else:
            variance = raw.float().square().mean(dim=-1, keepdim=True)
            normalized = raw * torch.rsqrt(variance + layer.norm_eps).to(raw.dtype)
            normalized = normalized * layer.output_norm_weight.to(raw.dtype)
        ref = normalized * torch.sigmoid(gate).to(raw.dtype)
        torch.cuda.synchronize()
    if dtype == torch.bfloat16:
        assert within_ulp(ours, ref, ulps=2), float((ours.float() - ref.float()).abs().max())
    else:
        assert rel_err(ours, ref) < 1e-5


def test_fused_prefill_matches_unfused_path(device):
    """The fused inference path and the torch path give the same layer output
    and cache up to the projection GEMMs' rounding (inputs whose route scores
    have no near-ties, so both select the same banks)."""
    layer = _layer(device, torch.bfloat16, 'nvidia', 'layer')
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(2, 33, layer.hidden_size, generator=gen).to(torch.bfloat16).to(device)
    announce('fused prefill vs torch path')
    with torch.no_grad():
        out, state = layer.prefill(x, state_dtype=torch.float32)
        (_, (rr, wr), _) = layer._inference_inputs(x)
        ref_rr, ref_wr = layer._route_projections(x)
        same_routes = all(torch.equal(layer._route(a, 4)[1], layer._route(b_, 4)[1])
                          for a, b_ in ((rr, ref_rr), (wr, ref_wr)))
        layer._fused_supported = lambda hidden: False  # the torch path for the same call
        ref_out, ref_state = layer.prefill(x, state_dtype=torch.float32)
        torch.cuda.synchronize()
    # A route-score near-tie can select other banks under the two GEMMs.  A
    # token's output depends on the writes up to it, so the outputs are
    # compared before each sequence's first token whose routes differ, and the
    # final cache only where no route differs.
    differ = torch.zeros(x.shape[:2], dtype=torch.bool, device=device)
    for a, b_ in ((rr, ref_rr), (wr, ref_wr)):
        differ |= (layer._route(a, 4)[1] != layer._route(b_, 4)[1]).any(-1)
    first = torch.where(differ.any(-1), differ.float().argmax(-1), torch.full_like(differ[:, 0], x.shape[1],
                                                                                   dtype=torch.long))
    keep = torch.arange(x.shape[1], device=device)[None, :] < first[:, None]
    assert float(keep.float().mean()) >= 0.75, 'too many near-ties for this seed'
    assert rel_err(out[keep], ref_out[keep]) < 1e-2
    if same_routes:
        assert rel_err(state, ref_state) < 1e-2
