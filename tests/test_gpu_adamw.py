"""The fused AdamW step against the reference's recipe run with torch
(reproduction/experiments/optim.py:30-50, "wiki"): clip_grad_norm_(1.0),
FP32 master gradients, torch's fused AdamW on the masters, masters copied
into the BF16 weights.  Bit-exact on weights, masters and both moments over
several steps, with the clip active and inactive and a ragged tensor tail."""

import pytest
import torch

pytestmark = pytest.mark.gpu

SIZES = [(5,), (4099,), (64, 33), (3,), (128, 256), (70000,)]


def make_params(device, seed):
    gen = torch.Generator().manual_seed(seed)
    params = []
    for i, shape in enumerate(SIZES):
        p = torch.nn.Parameter((torch.randn(shape, generator=gen) * 0.05).to(torch.bfloat16).to(device))
        if i % 3 == 1:
            p._no_weight_decay = True
        params.append(p)
    return params


def reference_step(params, masters, optimizer, lr):
    for group in optimizer.param_groups:
        group['lr'] = lr
    norm = torch.nn.utils.clip_grad_norm_(params, 1.0)
    for p, m in zip(params, masters):
        m.grad = p.grad.float()
    optimizer.step()
    for p, m in zip(params, masters):
        p.data.copy_(m)
    return norm


def test_fused_adamw_matches_the_reference_recipe():
    from bdm_amd.optim import MasterAdamW
    device = torch.device('cuda', 0)
    ours = make_params(device, 0)
    ref = make_params(device, 0)
    masters = [torch.nn.Parameter(p.detach().float().clone()) for p in ref]
    groups = [{'params': [m for m, p in zip(masters, ref) if bool(getattr(p, '_no_weight_decay', False)) == nd],
               'weight_decay': 0.0 if nd else 0.01} for nd in (False, True)]
    optimizer = torch.optim.AdamW(groups, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, fused=True)
    fused = MasterAdamW(ours, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.01)
    gen = torch.Generator().manual_seed(1)
    # gradient scales: clipped (norm >> 1), unclipped (norm < 1), clipped again
    for step, (scale, lr) in enumerate([(1.0, 3e-4), (1e-4, 2e-4), (0.3, 1e-3), (2e-5, 5e-4)]):
        for p, q in zip(ours, ref):
            g = (torch.randn(p.shape, generator=gen) * scale).to(torch.bfloat16).to(device)
            p.grad = g.clone()
            q.grad = g.clone()
        n_ref = reference_step(ref, masters, optimizer, lr)
        n_ours = fused.step(lr)
        torch.cuda.synchronize()
        assert torch.equal(n_ours, n_ref), step
        for i, (p, q, m) in enumerate(zip(ours, ref, masters)):
            state = optimizer.state[m]
            ea, eas = fused.moments_of(i)
            assert torch.equal(fused.master_of(i), m.detach()), (step, i, 'master')
            assert torch.equal(ea, state['exp_avg']), (step, i, 'exp_avg')
            assert torch.equal(eas, state['exp_avg_sq']), (step, i, 'exp_avg_sq')
            assert torch.equal(p.detach(), q.detach()), (step, i, 'weight')
        fused.zero_grad()


def test_state_dict_round_trip_resumes_bit_exact():
    """Save after two steps, restore into a fresh optimizer on copies of the
    weights, and take a third step on both: weights, masters and moments stay
    bit-identical.  Invalid checkpoints raise as the reference's do."""
    from bdm_amd.optim import MasterAdamW
    device = torch.device('cuda', 0)
    params = make_params(device, 3)
    opt = MasterAdamW(params, lr=1e-3)
    gen = torch.Generator().manual_seed(4)
    grads = [[(torch.randn(p.shape, generator=gen) * s).to(torch.bfloat16).to(device) for p in params]
             for s in (1.0, 0.01, 0.5)]
    for step in range(2):
        for p, g in zip(params, grads[step]):
            p.grad = g.clone()
        opt.step()
    saved = opt.state_dict()
    copies = [torch.nn.Parameter(p.detach().clone()) for p in params]
    for p, c in zip(params, copies):
        if hasattr(p, '_no_weight_decay'):
            c._no_weight_decay = True
    resumed = MasterAdamW(copies, lr=5.0)  # hyperparameters come from the checkpoint
    resumed.load_state_dict(saved)
    assert resumed.step_count == 2 and resumed.lr == opt.lr
    for ps in (params, copies):
        for p, g in zip(ps, grads[2]):
            p.grad = g.clone()
    opt.step()
    resumed.step()
    torch.cuda.synchronize()
    for i, (p, c) in enumerate(zip(params, copies)):
        assert torch.equal(p.detach(), c.detach()), i
        assert torch.equal(opt.master_of(i), resumed.master_of(i)), i
        assert all(torch.equal(a, b) for a, b in zip(opt.moments_of(i), resumed.moments_of(i))), i
    bad = dict(saved, masters=[t.to(torch.bfloat16) for t in saved['masters']])
    with pytest.raises(ValueError, match='master'):
        resumed.load_state_dict(bad)
    # weights edited after construction: reload_masters makes them the masters
    with torch.no_grad():
        copies[0].add_(1.0)
    resumed.reload_masters()
    assert torch.equal(resumed.master_of(0), copies[0].detach().float())
