"""C1 on the HIP path, and the narrow-head readout rule.

C1 is the configuration the reference's CPU path is timed on: one BDM layer,
batch 1, T = 512, d_model = 512, H = 4 heads of v = 64 (value width 256),
J = 256 banks (16 x 16 product key), S = 8, K = 8 read and 8 write banks,
FP32 weights and controllers, ``training_state_dtype='float32'``
(`implementation/bdm/heads.py:25-66`, `model.py:88-140`).  At 512 tokens the
oracle module runs the whole layer on the CPU, so the check is at full size.
"""

import sys

import pytest
import torch

from _inputs import oracle_reads, rel_err, routes
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def c1_config():
    from bdm_amd import BSDMConfig
    return BSDMConfig(dim=512, bank_count=256, bank_size=8, selected_banks=8, value_width=256, num_heads=4,
                      training_state_dtype='float32')


def test_c1_module_forward_matches_oracle(device):
    from bdm_amd import BankedDeltaMemory
    cfg = c1_config()
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device)
    oracle = O.OracleBankedDeltaMemory(cfg, layer_id=0, seed=0)
    assert next(layer.parameters()).dtype == torch.float32
    gen = torch.Generator().manual_seed(512)
    x = torch.randn(1, 512, cfg.dim, generator=gen)
    announce('C1 module forward (fp32, B1 T512 d512 H4 v64 J256 K8)')
    with torch.no_grad():
        xd = x.to(device)
        q, k, v, g, b, w = layer._controllers(xd)
        rr, wr = layer._route_projections(xd)
        raw = layer.bank_reads(xd)
        out = layer(xd)
        torch.cuda.synchronize()
        # (1) the recurrence and combine: the oracle sees the GPU's controller and score tensors
        ww, wi = O.product_key_route(wr.cpu(), bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
        rw, ri = O.product_key_route(rr.cpu(), bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
        ref_raw = oracle_reads(*(t.cpu() for t in (q, k, v, g, b, w)), wi, ww, ri, rw,
                               oracle.materialize_initial_state(), cfg.bank_count, routed_decay=True,
                               state_dtype=torch.float32)
        assert raw.dtype == torch.float32 and raw.shape == (1, 512, cfg.value_width)
        err = rel_err(raw, ref_raw, block=cfg.head_value_width)
        assert err < 1e-4, err
        assert rel_err(out, oracle.project_output(x, raw.cpu())) < 1e-4
        # (2) end to end: the oracle module's own CPU controllers, routes and
        # readout (the reference backend='reference' forward, model.py:120-131)
        ref_out = oracle(x)
        o_ww, o_wi, o_rw, o_ri = oracle.routes(x)
    same = (o_wi == wi).all(-1) & (o_ri == ri).all(-1)  # [1, T]: tokens routed identically
    assert same.float().mean() > 0.99, float(same.float().mean())
    err = rel_err(out.cpu()[same], ref_out[same])
    assert err < 1e-3, err


def _exact_case(batch, time, heads, v, j, kk, gen):
    """Reads whose values are exact in FP32, so the HIP and oracle read rows are
    the same BF16 numbers and only the combine rule can differ: S = 4 (scale
    1/2), only state row 0 nonzero (multiples of 1/16 below 4), q = e_0,
    read weights k/8, and write weights 0 (a write then leaves the state
    unchanged: decay exp(0), erase bf(b*0) and value bf(w*0) are exact)."""
    s = 4
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    ww = torch.zeros_like(ww)
    rw = (torch.randint(1, 9, rw.shape, generator=gen).float() / 8).to(torch.bfloat16)
    shape = (batch, time, heads)
    q = torch.zeros(*shape, s, dtype=torch.bfloat16)
    q[..., 0] = 1
    k = torch.nn.functional.normalize(torch.randn(*shape, s, generator=gen), dim=-1).to(torch.bfloat16)
    g = -torch.rand(*shape, s, generator=gen)
    b = torch.rand(*shape, s, generator=gen).to(torch.bfloat16)
    vv = torch.randn(*shape, v, generator=gen).to(torch.bfloat16)
    w = torch.rand(*shape, v, generator=gen).to(torch.bfloat16)
    state = torch.zeros(j, heads, s, v)
    state[:, :, 0] = torch.randint(-63, 64, (j, heads, v), generator=gen).float() / 16
    return (q, k, vv, g, b, w, wi, ww, ri, rw, state), s


@pytest.mark.parametrize('v', [16, 32, 64])
def test_readout_rule_by_head_width(device, v):
    """Heads of at most 32 columns sum a token's reads in FP32 and round once
    (index_add_, role_bank_dispatch.py:222-226); wider heads fold them in bank
    order rounding after every add (:209-215).  Bit-exact either way."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(3200 + v)
    batch, time, heads, j, kk = 2, 64, 2, 32, 8
    tensors, s = _exact_case(batch, time, heads, v, j, kk, gen)
    ref = {c: oracle_reads(*tensors, j, routed_decay=True, state_dtype=torch.bfloat16, interval=16)
           if c == 'role' else torch.cat([O.bank_forward(*(t[:, :, h].contiguous() for t in tensors[:6]),
                                                         *tensors[6:10], tensors[10][:, h], j, s ** -0.5,
                                                         routed_decay=True, state_dtype=torch.bfloat16,
                                                         interval=16, combine=c) for h in range(heads)], -1)
           for c in ('role', 'ordered', 'index_add')}
    differ = (ref['ordered'] != ref['index_add']).float().mean()
    assert differ > 0.05, float(differ)  # the two rules are told apart on these inputs
    dev = [t.to(device) for t in tensors]
    announce('readout rule', v)
    meta = ops.dispatch_build(dev[6], dev[8], j)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=16)
    torch.cuda.synchronize()
    expect = ref['index_add'] if v <= 32 else ref['ordered']
    assert torch.equal(ref['role'], expect)
    assert torch.equal(y.cpu(), expect)
