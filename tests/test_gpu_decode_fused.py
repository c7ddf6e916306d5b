"""The fused decode step (controller epilogue + both routes + decode in one
launch) against the three kernels it replaces, bit for bit.

``ops.decode_fused`` reads the fused projection row of each sequence: the
q, k, v, b, w slices, the read and write route scores and the f_proj output.
The chain it replaces is ``controller_epilogue`` (heads.py:11-22),
``router_select_pair`` (gdn2_banks.py:74-114) and ``decode_step``
(inference.py:161-194); y and the updated state must be identical.
"""

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def layout(heads, s, hv, j1, j2):
    """Column offsets of a fused projection row: q, k, v, f, b, w, read, write, gate."""
    widths = [('q', heads * s), ('k', heads * s), ('v', heads * hv), ('f', hv), ('b', heads * s),
              ('w', heads * hv), ('read', j1 + j2), ('write', j1 + j2), ('gate', heads * hv)]
    cols, at = {}, 0
    for name, width in widths:
        cols[name] = at
        at += (width + 7) // 8 * 8
    return cols, at


CASES = [
    # batch, heads, head width, J, qk_norm, routed decay, state dtype, param dtype
    (64, 8, 128, 256, 'nvidia', True, torch.bfloat16, torch.float32),
    (1, 8, 128, 256, 'nvidia', True, torch.bfloat16, torch.float32),
    (3, 2, 64, 2048, 'original', False, torch.float32, torch.bfloat16),
    (5, 1, 512, 64, 'nvidia', True, torch.bfloat16, torch.bfloat16),
    (2, 4, 96, 256, 'original', True, torch.float32, torch.float32),
]


@pytest.mark.parametrize('case', CASES, ids=lambda c: f'b{c[0]}h{c[1]}v{c[2]}J{c[3]}{c[4]}')
def test_fused_decode_matches_kernel_chain(device, case):
    from bdm_amd import ops
    from bdm_amd.config import near_square_factors
    batch, heads, hv, j, qk_norm, routed, state_dtype, param_dtype = case
    s, kk = 8, 8
    j1, j2 = near_square_factors(j)
    cols, width = layout(heads, s, hv, j1, j2)
    gen = torch.Generator().manual_seed(batch * 131 + heads * 17 + hv + j)
    announce('fused decode', case)
    proj = torch.randn(batch, width, generator=gen).to(torch.bfloat16).to(device)
    f = torch.randn(batch, heads * s, generator=gen).to(torch.bfloat16).to(device)
    a_log = (torch.rand(heads, generator=gen) * 2 - 1).to(param_dtype).to(device)
    dt_bias = torch.randn(heads * s, generator=gen).to(param_dtype).to(device)
    state0 = (torch.randn(batch, j, heads, s, hv, generator=gen) * 0.02).to(state_dtype).to(device)
    geometry = dict(heads=heads, bank_size=s, head_width=hv, bank_count=j, selected_banks=kk)
    assert ops.decode_fused_supported(proj, f, cols, a_log, dt_bias, state0, **geometry)

    # the chain of three kernels
    state_ref = state0.clone()
    q, k, v, g, b, w = ops.controller_epilogue(proj, f, cols, a_log, dt_bias, heads=heads, bank_size=s,
                                               head_width=hv, qk_norm=qk_norm)
    (ww, wi), (rw, ri) = ops.router_select_pair(proj[:, cols['write']:cols['write'] + j1 + j2],
                                                proj[:, cols['read']:cols['read'] + j1 + j2],
                                                bank_count=j, selected_banks=kk)
    y_ref = ops.decode_step(q, k, v, g, b, w, wi, ww, ri, rw, state_ref, bank_count=j, scale=s ** -0.5,
                            routed_decay=routed)
    # the fused step, twice in a row on its own copy of the state
    state = state0.clone()
    for step in range(2):
        y = ops.decode_fused(proj, f, cols, a_log, dt_bias, state, **geometry, qk_norm=qk_norm, routed_decay=routed,
                             scale=s ** -0.5)
        torch.cuda.synchronize()
        if step == 0:
            assert torch.equal(y, y_ref)
            assert torch.equal(state, state_ref)
            y_ref = ops.decode_step(q, k, v, g, b, w, wi, ww, ri, rw, state_ref, bank_count=j, scale=s ** -0.5,
                                    routed_decay=routed)
    assert torch.equal(y, y_ref)
    assert torch.equal(state, state_ref)


F_CASES = [c for c in CASES if c[2] >= 64]


@pytest.mark.parametrize('case', F_CASES, ids=lambda c: f'b{c[0]}h{c[1]}v{c[2]}J{c[3]}{c[4]}')
def test_fused_decode_forms_f(device, case):
    """f formed in the launch from f_proj's second factor: the f it forms is
    the GEMM's within one BF16 rounding, and fed to the kernel chain it gives
    the fused step's y and state bit for bit."""
    from bdm_amd import ops
    from bdm_amd.config import near_square_factors
    batch, heads, hv, j, qk_norm, routed, state_dtype, param_dtype = case
    s, kk = 8, 8
    j1, j2 = near_square_factors(j)
    cols, width = layout(heads, s, hv, j1, j2)
    gen = torch.Generator().manual_seed(batch * 71 + heads * 5 + hv + j)
    announce('fused decode forms f', case)
    proj = torch.randn(batch, width, generator=gen).to(torch.bfloat16).to(device)
    f_weight = (torch.randn(heads * s, hv, generator=gen) * hv ** -0.5).to(torch.bfloat16).to(device)
    a_log = (torch.rand(heads, generator=gen) * 2 - 1).to(param_dtype).to(device)
    dt_bias = torch.randn(heads * s, generator=gen).to(param_dtype).to(device)
    state0 = (torch.randn(batch, j, heads, s, hv, generator=gen) * 0.02).to(state_dtype).to(device)
    geometry = dict(heads=heads, bank_size=s, head_width=hv, bank_count=j, selected_banks=kk)
    assert ops.decode_fused_supported(proj, None, cols, a_log, dt_bias, state0, **geometry, f_weight=f_weight)

    state = state0.clone()
    f_out = torch.full((batch, heads * s), float('nan'), device=device, dtype=torch.bfloat16)
    y = ops.decode_fused(proj, None, cols, a_log, dt_bias, state, **geometry, qk_norm=qk_norm, routed_decay=routed,
                         scale=s ** -0.5, f_weight=f_weight, f_out=f_out)
    torch.cuda.synchronize()
    # f against an FP64 product of the same BF16 operands: one BF16 rounding
    # (2^-8 relative) after an FP32 sum of hv exact products (hv * 2^-24 of
    # the sum of magnitudes, with margin)
    x64 = proj[:, cols['f']:cols['f'] + hv].double()
    f64 = x64 @ f_weight.double().t()
    bound = f64.abs() * 2.0 ** -8 + (x64.abs() @ f_weight.double().abs().t()) * hv * 2.0 ** -23
    assert torch.all((f_out.double() - f64).abs() <= bound)

    state_ref = state0.clone()
    q, k, v, g, b, w = ops.controller_epilogue(proj, f_out, cols, a_log, dt_bias, heads=heads, bank_size=s,
                                               head_width=hv, qk_norm=qk_norm)
    (ww, wi), (rw, ri) = ops.router_select_pair(proj[:, cols['write']:cols['write'] + j1 + j2],
                                                proj[:, cols['read']:cols['read'] + j1 + j2],
                                                bank_count=j, selected_banks=kk)
    y_ref = ops.decode_step(q, k, v, g, b, w, wi, ww, ri, rw, state_ref, bank_count=j, scale=s ** -0.5,
                            routed_decay=routed)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert torch.equal(state, state_ref)


def test_fused_decode_rejects_other_geometries(device):
    from bdm_amd import ops
    heads, s, hv, j1, j2 = 2, 8, 32, 16, 16  # a 32-column head: too few lanes for the fused step
    cols, width = layout(heads, s, hv, j1, j2)
    proj = torch.zeros(1, width, device=device, dtype=torch.bfloat16)
    f = torch.zeros(1, heads * s, device=device, dtype=torch.bfloat16)
    a_log = torch.zeros(heads, device=device)
    dt_bias = torch.zeros(heads * s, device=device)
    state = torch.zeros(1, 256, heads, s, hv, device=device, dtype=torch.bfloat16)
    geometry = dict(heads=heads, bank_size=s, head_width=hv, bank_count=256, selected_banks=8)
    assert not ops.decode_fused_supported(proj, f, cols, a_log, dt_bias, state, **geometry)
    with pytest.raises(NotImplementedError):
        ops.decode_fused(proj, f, cols, a_log, dt_bias, state, **geometry, qk_norm='nvidia', routed_decay=True,
                         scale=s ** -0.5)


def relative_error(got, want):
    got, want = got.float().flatten(1), want.float().flatten(1)
    return ((got - want).norm(dim=1) / want.norm(dim=1).clamp_min(1e-6)).max().item()


@pytest.mark.parametrize('batch', [1, 64])
def test_module_step_fused_equals_unfused(device, batch):
    """BankedDeltaMemory.step at the C3 geometry: the fused launch against
    the separate kernels over several tokens (y and the cache).  The fused
    launch forms f itself (FP32 dot products in its own order), so f can
    differ from the GEMM's by one BF16 rounding: y and the cache agree to a
    relative 1e-2 per token."""
    from bdm_amd import BSDMConfig, BankedDeltaMemory
    cfg = BSDMConfig(dim=1024, bank_count=256, bank_size=8, selected_banks=8, value_width=1024, num_heads=8)
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device=device, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(batch)
    announce('module step fused', batch)
    with torch.no_grad():
        cache = layer.create_state(batch, dtype=torch.bfloat16)
        cache.copy_((torch.randn(cache.shape, generator=gen) * 0.02).to(cache.dtype))
        cache_ref = cache.clone()
        for _ in range(3):
            x = torch.randn(batch, 1, cfg.dim, generator=gen).to(torch.bfloat16).to(device)
            layer.fused_decode = True
            y, cache = layer.step(x, cache)
            layer.fused_decode = False
            y_ref, cache_ref = layer.step(x, cache_ref)
            torch.cuda.synchronize()
            assert relative_error(y, y_ref) < 1e-2
            assert relative_error(cache.flatten(1), cache_ref.flatten(1)) < 1e-2
        layer.fused_decode = True
