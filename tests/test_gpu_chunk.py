"""The matrix-core recurrence (chunk_forward.hip, FP32 MFMA) against the
oracle and the vector-ALU recurrence on the same inputs.

The matrix-core path runs S = 8 with BF16 controllers and the state rounded
to BF16 every 16 events (the reference module forward's policy at H > 1,
heads.py:40-46 with role_bank_kernel.py:153-165).  It must match the oracle
to the forward tolerance (1e-2 per token), write the same final states, and
write the snapshots the backward replays from (the BF16 state at every
16-event boundary, role_bank_kernel.py:57-66).  ``BDM_FORWARD_KERNEL=vector``
selects the vector-ALU kernel for the comparison.
"""

import os
import sys

import pytest
import torch

from _inputs import controllers, initial_state, oracle_reads, rel_err, routes

pytestmark = pytest.mark.gpu
TOL = 1e-2


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def run_forward(device, tensors, j, s, *, kernel, snapshots=False):
    from bdm_amd import ops
    q, k, v, g, b, w, wi, ww, ri, rw, state = tensors
    batch, time, heads, width = v.shape
    dev = [t.to(device) for t in tensors]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    final = torch.empty(batch, j, heads, s, width, device=device, dtype=torch.float32)
    snap = None
    if snapshots:
        x = ops.prepare_routed(*dev[:10], dev[10], bank_count=j)
        snap = ops.snapshot_buffer(x, 16, torch.bfloat16)
        snap.fill_(0)
    old = os.environ.get('BDM_FORWARD_KERNEL')
    os.environ['BDM_FORWARD_KERNEL'] = kernel
    try:
        y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                               round_interval=16, final_state=final, snapshots=snap,
                               snapshot_interval=16 if snapshots else 0)
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ['BDM_FORWARD_KERNEL']
        else:
            os.environ['BDM_FORWARD_KERNEL'] = old
    return y, final, snap


CASES = [
    # batch, time, heads, v, J, K
    (2, 96, 2, 128, 16, 4),     # ~48-event segments: 3-4 chunks, ragged ends
    (1, 200, 1, 128, 4, 4),     # every token writes and reads every bank: 400-event segments
    (2, 24, 2, 128, 64, 2),     # empty and 1..8-event segments
    (1, 64, 3, 64, 8, 4),       # 64-column heads (2 tiles)
    (1, 64, 2, 256, 8, 4),      # 256-column heads (8 tiles)
    (1, 40, 1, 384, 8, 4),      # a 384-column head: three 128-column virtual heads
    (1, 60, 4, 128, 256, 8),    # the C2 head geometry at small T
]


@pytest.mark.parametrize('case', CASES, ids=[str(c) for c in CASES])
def test_chunk_forward_matches_oracle(device, case):
    batch, time, heads, v, j, kk = case
    s = 8
    gen = torch.Generator().manual_seed(7000 + CASES.index(case))
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen)
    tensors = (q, k, v_, g, b, w, wi, ww, ri, rw, state)
    ref, ref_final = oracle_reads(*tensors, j, routed_decay=True, state_dtype=torch.bfloat16, interval=16,
                                  return_final=True)
    announce('chunk forward', case)
    y, final, snap = run_forward(device, tensors, j, s, kernel='mfma', snapshots=True)
    announce('vector forward', case)
    y_vec, final_vec, snap_vec = run_forward(device, tensors, j, s, kernel='vector', snapshots=True)
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    err_y, err_f = rel_err(y, ref), rel_err(final, ref_final)
    assert err_y < TOL and err_f < TOL, (err_y, err_f)
    assert rel_err(y, y_vec) < TOL and rel_err(final, final_vec) < TOL
    # snapshots: the same BF16 boundary states as the vector kernel's (a value
    # may differ by the last BF16 bit where the two FP32 sums round apart)
    assert rel_err(snap, snap_vec) < TOL, rel_err(snap, snap_vec)


@pytest.mark.parametrize('decay', ['strong', 'mixed', 'none', 'growth'])
def test_chunk_forward_decay_extremes(device, decay):
    """Decays that vanish within a chunk ('strong', g down to -40), spikes
    among mild ones, none at all, and decays above 1 (g > 0): the chunk's
    coefficients come from the recurrence itself, with no division by
    cumulative decays, so every regime matches the oracle."""
    batch, time, heads, s, v, j, kk = 2, 96, 2, 8, 128, 8, 4
    gen = torch.Generator().manual_seed({'strong': 1, 'mixed': 2, 'none': 3, 'growth': 4}[decay])
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    if decay == 'strong':
        g = -torch.rand(g.shape, generator=gen) * 40
    elif decay == 'mixed':
        spikes = torch.rand(batch, time, 1, 1, generator=gen) < 0.05
        g = torch.where(spikes, -torch.rand(g.shape, generator=gen) * 60, g)
    elif decay == 'none':
        g = torch.zeros_like(g)
    else:
        g = (torch.rand(g.shape, generator=gen) - 0.5) * 0.2
    state = initial_state(j, heads, s, v, gen)
    tensors = (q, k, v_, g, b, w, wi, ww, ri, rw, state)
    ref, ref_final = oracle_reads(*tensors, j, routed_decay=True, state_dtype=torch.bfloat16, interval=16,
                                  return_final=True)
    announce('chunk forward decay', decay)
    y, final, _ = run_forward(device, tensors, j, s, kernel='mfma')
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    err_y, err_f = rel_err(y, ref), rel_err(final, ref_final)
    assert err_y < TOL and err_f < TOL, (err_y, err_f)



def test_chunk_forward_full_size_c2(device):
    """The C2 geometry (B8 T4096 H8 S8 v128 J256 K8) on the matrix cores:
    reads and final states of the first and the last sequence against the
    oracle recurrence, per token, to the forward tolerance."""
    batch, time, heads, s, v, j, kk = 8, 4096, 8, 8, 128, 256, 8
    gen = torch.Generator().manual_seed(2027)
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    tensors = (q, k, v_, g, b, w, wi, ww, ri, rw, state)
    announce('chunk forward full size C2')
    y, final, _ = run_forward(device, tensors, j, s, kernel='mfma')
    for seq in (0, batch - 1):
        one = lambda t: t[seq:seq + 1]  # noqa: E731
        ref_y, ref_final = oracle_reads(*(one(t) for t in (q, k, v_, g, b, w, wi, ww, ri, rw)), state, j,
                                        routed_decay=True, state_dtype=torch.bfloat16, interval=16,
                                        return_final=True)
        err_y, err_f = rel_err(one(y), ref_y), rel_err(one(final), ref_final)
        print(f'chunk forward C2 sequence {seq}: read err {err_y:.4f}, state err {err_f:.4f}', flush=True)
        assert err_y < TOL and err_f < TOL, (seq, err_y, err_f)
