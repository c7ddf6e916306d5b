"""bdm_route_dispatch: both routers and the dispatch in one call.

Its routes and dispatch must equal, bit for bit, those of the separate calls
(bdm_router_select_pair, then bdm_dispatch_build), which the other parity
tests pin against the oracle; its segment order must be each XCD range's
segments by decreasing length (ties by index), the order bdm_forward computes
itself, and a forward given it must produce the same reads and final state.
"""

import sys

import pytest
import torch

from _inputs import controllers, initial_state

pytestmark = pytest.mark.gpu

CASES = [
    # batch, time, J, K: fused routing + tile count, ranking in the scatter (C2 geometry)
    (8, 4096, 256, 8),
    # fused, time not a multiple of the 32-token tile, 4 sequences (two ranges per sequence)
    (4, 333, 64, 8),
    # fused, 16 sequences: ranges span two sequences, ranked by the standalone kernel
    (16, 100, 256, 8),
    # 3 sequences: batch * J not a multiple of 8, no segment order
    (3, 70, 64, 8),
    # factors 32 x 64 (C4's): routing by the quad kernel, dispatch separate, standalone ranking
    (4, 512, 2048, 8),
    # 4 banks per role (not the fused geometry)
    (2, 90, 16, 4),
    # ranges of 128 segments, 4 and 8 of them per sequence, each sorted by one wave
    (2, 200, 512, 8),
    (1, 300, 1024, 8),
    # ranges of 512 segments: ranked pairwise
    (8, 64, 512, 8),
]


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize('case', CASES, ids=[str(c) for c in CASES])
def test_route_dispatch_equals_separate_calls(device, case):
    from bdm_amd import ops
    from bdm_amd.config import near_square_factors
    batch, time, j, kk = case
    j1, j2 = near_square_factors(j)
    gen = torch.Generator().manual_seed(sum(case))
    scores = torch.randn(2, batch, time, j1 + j2, generator=gen).to(torch.bfloat16).to(device)
    announce('route dispatch', case)
    (ww, wi), (rw, ri), meta = ops.route_dispatch(scores[0], scores[1], bank_count=j, selected_banks=kk, maps=True)
    (ww2, wi2), (rw2, ri2) = ops.router_select_pair(scores[0], scores[1], bank_count=j, selected_banks=kk)
    ref = ops.dispatch_build(wi2, ri2, j)
    torch.cuda.synchronize()
    for a, b in ((ww, ww2), (wi, wi2), (rw, rw2), (ri, ri2), (meta.order, ref.order), (meta.inverse, ref.inverse),
                 (meta.tokens, ref.tokens), (meta.cu_seqlens, ref.cu_seqlens), (meta.status, ref.status)):
        assert torch.equal(a, b)
    # without the inverse and token maps: the same order and bounds
    _, _, lean = ops.route_dispatch(scores[0], scores[1], bank_count=j, selected_banks=kk)
    torch.cuda.synchronize()
    assert lean.inverse is None and lean.tokens is None
    assert torch.equal(lean.order, ref.order) and torch.equal(lean.cu_seqlens, ref.cu_seqlens)
    nseg = batch * j
    if nseg % 8 == 0 and nseg // 8 <= 1024:
        lengths = (ref.cu_seqlens[1:] - ref.cu_seqlens[:-1]).cpu()
        order = lean.segment_order.cpu().long()
        rng = nseg // 8
        for x in range(8):
            part = order[x * rng:(x + 1) * rng]
            assert sorted(part.tolist()) == list(range(x * rng, (x + 1) * rng))
            key = [(-int(lengths[s]), int(s)) for s in part]
            assert key == sorted(key)


def test_forward_with_the_dispatch_order_is_bit_identical(device):
    """C2 geometry: bdm_forward given bdm_route_dispatch's segment order and
    computing its own give the same reads and final state."""
    from bdm_amd import ops
    batch, time, heads, s, v, j, kk = 8, 4096, 8, 8, 128, 256, 8
    gen = torch.Generator().manual_seed(4242)
    scores = torch.randn(2, batch, time, 32, generator=gen).to(torch.bfloat16).to(device)
    q, k, v_, g, b, w = (t.to(device) for t in controllers(batch, time, heads, s, v, gen))
    state = initial_state(j, heads, s, v, gen, scale=0.05).to(device)
    announce('forward with the dispatch order')
    (ww, wi), (rw, ri), meta = ops.route_dispatch(scores[0], scores[1], bank_count=j, selected_banks=kk)
    outs = []
    for given in (True, False):
        m = meta if given else ops.Dispatch(meta.order, None, None, meta.cu_seqlens, meta.status)
        final = torch.full((batch, j, heads, s, v), float('nan'), device=device, dtype=torch.bfloat16)
        y = ops.routed_forward(q, k, v_, g, b, w, wi, ww, ri, rw, state, m, bank_count=j, scale=s ** -0.5,
                               routed_decay=True, round_interval=16, final_state=final)
        torch.cuda.synchronize()
        outs.append((y, final))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
