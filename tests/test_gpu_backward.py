"""Backward of the routed path on the GPU against autograd through the CPU oracle.

The oracle's gradients are those of the reference's CPU backend (pinned by
tests/golden/layer_small.pt).  Tolerance: per row of a gradient tensor
(``_inputs.rel_err``; the route-weight gradients over the whole tensor),
max|hip - oracle| / max|oracle| <= 2e-2 (BF16 controllers and state, FP32
arithmetic; the BF16 rounding points of the token VJP differ from autograd's
in order, not in kind).  FP32 controllers with an FP32 state: 1e-4.
"""

import sys

import pytest
import torch

from _inputs import controllers, global_rel_err, initial_state, rel_err, routes
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def oracle_grads(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, dy, *, routed_decay, state_dtype,
                 interval=None):
    """Autograd of sum(y * dy) through the oracle, per head (heads.py:34-46)."""
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, g, b, w, ww, rw, state)]
    lq, lk, lv, lg, lb, lw, lww, lrw, lst = leaves
    heads = q.shape[2]
    outs = []
    for h in range(heads):
        sl = lambda x: x[:, :, h]  # noqa: E731
        outs.append(O.bank_forward(sl(lq), sl(lk), sl(lv), sl(lg), sl(lb), sl(lw), wi, lww, ri, lrw, lst[:, h],
                                   bank_count, q.shape[-1] ** -0.5, routed_decay=routed_decay,
                                   state_dtype=state_dtype, interval=interval, combine='role', lockstep=True))
    y = torch.cat(outs, -1)
    (y.float() * dy.float()).sum().backward()
    return y.detach(), [t.grad for t in leaves]


CASES = [
    # batch, time, heads, S, v, J, K, routed, state_dtype, ctrl dtype
    (2, 48, 2, 8, 128, 16, 4, True, torch.bfloat16, torch.bfloat16),
    (2, 48, 2, 8, 128, 16, 4, True, torch.float32, torch.bfloat16),
    (1, 40, 3, 8, 64, 12, 3, False, torch.bfloat16, torch.bfloat16),
    (2, 33, 2, 4, 16, 6, 2, True, torch.float32, torch.bfloat16),
    (2, 30, 2, 16, 64, 16, 4, True, torch.bfloat16, torch.bfloat16),
    (1, 64, 1, 8, 128, 4, 2, True, torch.bfloat16, torch.bfloat16),
    (2, 24, 2, 8, 32, 16, 4, True, torch.float32, torch.float32),
    (1, 20, 2, 8, 200, 16, 4, True, torch.bfloat16, torch.bfloat16),
    # every token writes and reads all 4 banks: 200-event segments, 13 chunks of 16
    (1, 100, 2, 8, 128, 4, 4, True, torch.bfloat16, torch.bfloat16),
    (1, 100, 1, 8, 128, 4, 4, True, torch.float32, torch.bfloat16),
    # 64 banks, 12 tokens: empty and 1..8-event segments
    (2, 12, 2, 8, 128, 64, 2, True, torch.bfloat16, torch.bfloat16),
    # heads wider than 256 columns: 128-column virtual heads forward, column tiles backward
    (1, 24, 1, 8, 2048, 8, 4, True, torch.bfloat16, torch.bfloat16),
    (1, 20, 2, 8, 384, 16, 4, True, torch.float32, torch.bfloat16),
]


def check_against_oracle(device, case, seed, gmap=None, compact_replay=None):
    from bdm_amd import bank_training, role_bank_training
    batch, time, heads, s, v, j, kk, routed, sdt, dt = case
    gen = torch.Generator().manual_seed(seed)
    _, ww, wi = routes(batch, time, j, kk, gen, dtype=dt)
    _, rw, ri = routes(batch, time, j, kk, gen, dtype=dt)
    q, k, val, g, b, w = controllers(batch, time, heads, s, v, gen, dtype=dt)
    if gmap is not None:
        g = gmap(g, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.1)
    dy = torch.randn(batch, time, heads * v, generator=gen).to(dt)
    # compact_replay=True with BF16 controllers: 8-event replay chunks, and a
    # BF16 state rounded at each of them (role_bank_kernel.py:153-165)
    interval = 8 if (compact_replay is True and dt == torch.bfloat16) else None
    ref_y, ref = oracle_grads(q, k, val, g, b, w, wi, ww, ri, rw, state, j, dy, routed_decay=routed,
                              state_dtype=sdt, interval=interval)
    leaves = [t.to(device).requires_grad_(True) for t in (q, k, val, g, b, w, ww, rw, state)]
    lq, lk, lv, lg, lb, lw, lww, lrw, lst = leaves
    op = bank_training if routed else role_bank_training
    y = op(lq, lk, lv, lg, lb, lw, wi.to(device), lww, ri.to(device), lrw, lst, j, s ** -0.5, state_dtype=sdt,
           compact_replay=compact_replay)
    (y.float() * dy.to(device).float()).sum().backward()
    torch.cuda.synchronize()
    tol = 1e-4 if (dt == torch.float32 and sdt == torch.float32) else 2e-2
    assert rel_err(y, ref_y) < max(tol, 1e-2)
    names = ('q', 'k', 'v', 'g', 'b', 'w', 'ww', 'rw', 'state')
    for name, ours, theirs in zip(names, (t.grad for t in leaves), ref):
        assert ours is not None, name
        assert ours.shape == theirs.shape and ours.dtype == theirs.dtype, name
        # Route-weight gradients are per-(token, route) sums over all S rows and
        # v columns of products that largely cancel (role_bank_dispatch.py:
        # 99-131), so a token's value can be far below its terms' size and its
        # own relative error is set by their rounding: judged on the tensor's
        # scale.  Every other gradient is judged per row (a token's S or v
        # values, a state row).
        err = global_rel_err(ours, theirs) if name in ('ww', 'rw') else rel_err(ours, theirs)
        assert err < tol, (name, err)


@pytest.mark.parametrize('case', range(len(CASES)))
def test_backward_matches_oracle_autograd(device, case):
    announce('backward', CASES[case])
    check_against_oracle(device, CASES[case], 100 + case)


@pytest.mark.parametrize('case', [0, 8])
def test_compact_replay_chunk(device, case):
    """compact_replay=True: the BF16 state is rounded (and replayed) every 8
    events instead of 16; forward and gradients against the oracle run with
    that interval."""
    announce('compact replay', CASES[case])
    check_against_oracle(device, CASES[case], 300 + case, compact_replay=True)


# Decay regimes of the S = 8 chunk kernel: products of a chunk's decays far
# below 2^-40 (every chunk in eager form), a mix of eager and lazy chunks,
# and decays above 1 (g > 0 on some rows).
DECAYS = {
    'strong': lambda g, gen: g * 100.0,
    'mixed': lambda g, gen: g * torch.where(torch.rand(g.shape[:2], generator=gen) < 0.3, 60.0, 1.0)[..., None, None],
    'growth': lambda g, gen: (torch.rand(g.shape, generator=gen) - 0.5) * 0.6,
}


@pytest.mark.parametrize('regime', sorted(DECAYS))
@pytest.mark.parametrize('sdt', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_backward_decay_regimes(device, regime, sdt):
    case = (2, 48, 2, 8, 128, 16, 4, True, sdt, torch.bfloat16)
    announce('backward decay', regime, case)
    check_against_oracle(device, case, 300, DECAYS[regime])


def test_backward_per_head_layout_matches_multi_head(device):
    """The reference's per-head call (q [B,T,S], state [J,S,v]) and the
    multi-head layout give the same gradients for one head."""
    from bdm_amd import bank_training
    gen = torch.Generator().manual_seed(7)
    batch, time, s, v, j, kk = 2, 50, 8, 128, 16, 4
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, val, g, b, w = controllers(batch, time, 1, s, v, gen)
    state = initial_state(j, 1, s, v, gen, scale=0.1)
    dy = torch.randn(batch, time, v, generator=gen).to(torch.bfloat16).to(device)
    announce('backward per-head layout')
    grads = []
    for per_head in (True, False):
        tensors = [t.to(device) for t in (q, k, val, g, b, w, ww, rw, state)]
        if per_head:
            tensors = [t[:, :, 0].contiguous() for t in tensors[:6]] + tensors[6:8] + [tensors[8][:, 0].contiguous()]
        leaves = [t.requires_grad_(True) for t in tensors]
        y = bank_training(*leaves[:6], wi.to(device), leaves[6], ri.to(device), leaves[7], leaves[8], j, s ** -0.5,
                          state_dtype=torch.bfloat16)
        (y.float().reshape(batch, time, v) * dy.float()).sum().backward()
        grads.append([t.grad.reshape(-1) for t in leaves])
    for a, c in zip(*grads):
        assert torch.equal(a, c)


def test_backward_is_deterministic(device):
    from bdm_amd import bank_training
    gen = torch.Generator().manual_seed(8)
    batch, time, heads, s, v, j, kk = 2, 64, 2, 8, 128, 16, 4
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    tensors = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.1)
    dy = torch.randn(batch, time, heads * v, generator=gen).to(torch.bfloat16).to(device)
    announce('backward determinism')
    runs = []
    for _ in range(2):
        leaves = [t.to(device).requires_grad_(True) for t in (*tensors, ww, rw, state)]
        y = bank_training(*leaves[:6], wi.to(device), leaves[6], ri.to(device), leaves[7], leaves[8], j, s ** -0.5,
                          state_dtype=torch.bfloat16)
        (y.float() * dy.float()).sum().backward()
        runs.append([t.grad.clone() for t in leaves])
    for a, c in zip(*runs):
        assert torch.equal(a, c)


def test_module_gradients_match_oracle(device):
    """C5-style layer (BSDM, H=8 heads, S=8, BF16 training state) at a small
    size: forward and the gradients of every parameter the path reaches
    (controller projections, router, decay, initial-memory factors) against
    the oracle module with the same state dict, in FP32 parameters."""
    from bdm_amd import BSDMConfig, BankedDeltaMemory
    cfg = BSDMConfig(dim=64, bank_count=16, bank_size=8, selected_banks=4, value_width=128, num_heads=4)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(2, 40, cfg.dim, generator=gen)
    dy = torch.randn(2, 40, cfg.dim, generator=gen)
    oracle = O.OracleBankedDeltaMemory(cfg, layer_id=2, seed=5)
    layer = BankedDeltaMemory(cfg, layer_id=2, seed=5)
    layer.load_state_dict(oracle.state_dict())
    layer = layer.to(device)
    announce('module gradients')
    out_ref = oracle(x, combine='role')
    (out_ref * dy).sum().backward()
    out = layer(x.to(device))
    (out * dy.to(device)).sum().backward()
    torch.cuda.synchronize()
    assert rel_err(out, out_ref) < 1e-2
    checked = 0
    for name, p_ref in oracle.named_parameters():
        p = dict(layer.named_parameters())[name]
        if p_ref.grad is None:
            assert p.grad is None or float(p.grad.abs().max()) == 0.0, name
            continue
        err = rel_err(p.grad, p_ref.grad)
        assert err < 2e-2, (name, err)
        checked += 1
    assert checked >= 12
