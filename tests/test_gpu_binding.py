"""The operator as the reference's injection point calls it.

``heads.forward_heads(m, hidden, training_function=f)`` (heads.py:25-46) runs
one call per head, ``f(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count,
scale, None, None, compact_replay=...)`` with one head's controllers
(q [B,T,S]) and state ([J,S,v]), and concatenates the heads' reads.  The loop
below makes that call for every head and compares the result with the
multi-head call of the same operator: the reads and the per-head gradients of
q, k, v, g, b, w and the state bit for bit.  The route-weight gradients are
sums over heads: the multi-head kernel adds the heads in FP32 and rounds once,
while autograd adds the per-head BF16 gradients, so those two are held to one
BF16 rounding per head instead.
"""

import inspect
import sys

import pytest
import torch

from _inputs import controllers, global_rel_err, initial_state, routes


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def per_head_reads(training_function, tensors, wi, ww, ri, rw, state, bank_count, scale, compact_replay):
    """One injected call per head, heads concatenated along the value axis."""
    reads = []
    for head in range(tensors[0].shape[2]):
        q, k, v, g, b, w = (t[:, :, head].contiguous() for t in tensors)
        raw = training_function(q, k, v, g, b, w, wi, ww, ri, rw, state[:, head].contiguous(),
                                bank_count, scale, None, None, compact_replay=compact_replay)
        reads.append(raw)
    return torch.cat(reads, dim=-1)


def test_injected_call_shape_binds():
    """The injection point's argument shape binds to both operators (CPU)."""
    import bdm_amd
    for op in (bdm_amd.bank_training, bdm_amd.role_bank_training):
        bound = inspect.signature(op).bind(*range(11), 16, 0.35, None, None, compact_replay=None)
        assert bound.arguments['compact_slot'] is None and bound.arguments['dtype_slot'] is None


def test_injected_call_options_are_checked():
    from bdm_amd.routed_update import _options
    assert _options(None, None, None, torch.float32) == (None, torch.float32)
    assert _options(True, None, None, torch.float32) == (True, torch.float32)
    assert _options(None, torch.bfloat16, False, torch.float32) == (False, torch.bfloat16)
    with pytest.raises(ValueError):
        _options(True, None, False, torch.float32)
    with pytest.raises(ValueError):
        _options(None, torch.float16, None, torch.float32)
    with pytest.raises(ValueError):
        _options(None, None, 1, torch.float32)


@pytest.mark.gpu
@pytest.mark.parametrize('routed', [True, False], ids=['routed', 'role'])
@pytest.mark.parametrize('compact_replay', [None, True])
def test_injected_per_head_calls_equal_multi_head(device, routed, compact_replay):
    import bdm_amd
    op = bdm_amd.bank_training if routed else bdm_amd.role_bank_training
    gen = torch.Generator().manual_seed(31)
    batch, time, heads, s, v, j, kk = 2, 80, 3, 8, 64, 16, 4
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    tensors = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.1)
    dy = torch.randn(batch, time, heads * v, generator=gen).to(torch.bfloat16).to(device)
    wi, ri = wi.to(device), ri.to(device)
    announce('injected call shape', routed, compact_replay)
    results = []
    for injected in (True, False):
        leaves = [t.to(device).requires_grad_(True) for t in (*tensors, ww, rw, state)]
        ctrl, lww, lrw, lstate = leaves[:6], leaves[6], leaves[7], leaves[8]
        if injected:
            y = per_head_reads(op, ctrl, wi, lww, ri, lrw, lstate, j, s ** -0.5, compact_replay)
        else:
            y = op(*ctrl, wi, lww, ri, lrw, lstate, j, s ** -0.5, compact_replay=compact_replay)
        (y.float() * dy.float()).sum().backward()
        results.append((y.detach(), [t.grad for t in leaves]))
    (y_inj, g_inj), (y_all, g_all) = results
    assert y_inj.shape == y_all.shape == (batch, time, heads * v)
    assert torch.equal(y_inj, y_all)
    for a, c in zip(g_inj[:6] + g_inj[8:], g_all[:6] + g_all[8:]):
        assert torch.equal(a, c)
    for a, c in zip(g_inj[6:8], g_all[6:8]):
        assert global_rel_err(a, c) <= heads * 2.0 ** -8
