"""The BASELINE configurations at full size, checked through properties that do
not need the CPU oracle to run the whole workload.

* C3 decode (batch 64, H8, J256, S8, v128, K8): one step against the oracle
  step (cheap per token) and untouched banks bit-identical.
* C4 skewed forward (batch 4, T8192, J2048 = 32x64, Zipf s=1.1 on the factor
  scores): router and dispatch bit-exact over all 524,288 events; causality —
  the reads of the first tokens depend only on those tokens, so they equal the
  oracle on the truncated sequence; the final states of the longest (hottest)
  segments against the per-event oracle loop.
* C5 training (batch 4, T2048, H8, BF16 state): with the upstream gradient
  zero after the first tokens of sequence 0, every gradient equals the
  oracle's on the truncated sequence and is exactly zero elsewhere.
"""

import sys

import pytest
import torch

from _inputs import controllers, initial_state, oracle_reads, rel_err, routes, tie_dependent_rows
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def test_c3_decode_full_size(device):
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(33)
    batch, heads, s, v, j, kk = 64, 8, 8, 128, 256, 8
    _, ww, wi = routes(batch, 1, j, kk, gen)
    _, rw, ri = routes(batch, 1, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, 1, heads, s, v, gen)
    state = (torch.randn(batch, j, heads, s, v, generator=gen) * 0.02).to(torch.bfloat16)
    expect = state.clone()
    rows = torch.arange(batch)
    ys = []
    for h in range(heads):
        st = expect[:, :, h]
        for jj in range(kk):
            bank, p = wi[:, 0, jj], ww[:, 0, jj]
            new = O.write_update(st[rows, bank].float(), k[:, 0, h], g[:, 0, h] * p.float()[:, None],
                                 (b[:, 0, h] * p[:, None]).to(b.dtype), (w[:, 0, h] * p[:, None]).to(w.dtype),
                                 v_[:, 0, h])
            st[rows, bank] = new.to(torch.bfloat16)
        vals = torch.stack([O.read_value(st[rows, ri[:, 0, jj]].float(),
                                         (q[:, 0, h] * rw[:, 0, jj][:, None]).to(q.dtype), s ** -0.5)
                            .to(torch.bfloat16) for jj in range(kk)], 1)
        order = torch.argsort(ri[:, 0], dim=-1, stable=True)
        total = torch.zeros(batch, v)
        for jj in range(kk):
            total = (total + vals[rows, order[:, jj]].float()).to(torch.bfloat16).float()
        ys.append(total)
    announce('C3 decode full size')
    dstate = state.to(device)
    y = ops.decode_step(*(t[:, 0].to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw)), dstate,
                        bank_count=j, scale=s ** -0.5, routed_decay=True)
    torch.cuda.synchronize()
    assert rel_err(dstate, expect) < TOL
    assert rel_err(y, torch.cat(ys, -1)) < TOL
    touched = torch.zeros(batch, j, dtype=torch.bool)
    touched[rows[:, None], wi[:, 0]] = True
    assert torch.equal(dstate.cpu()[~touched], state[~touched])


def test_c2_router_full_size_with_ties(device):
    """C2 score geometry (B8 T4096, 16 + 16 BF16 factor scores, B = 8) for both
    roles: indices and weights bit-exact against the oracle on every row,
    including the ~11% whose selected set depends on a tie."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(2222)
    for role in ('write', 'read'):
        scores = torch.randn(8, 4096, 32, generator=gen).to(torch.bfloat16)
        announce('C2 router full size', role)
        w_, i_ = ops.router_select(scores.to(device), bank_count=256, selected_banks=8)
        torch.cuda.synchronize()
        wr, ir = O.product_key_route(scores, bank_count=256, selected_banks=8)
        ties = tie_dependent_rows(scores, 256, 8)
        print(f'C2 {role} tie-dependent router rows: {float(ties.float().mean()):.4f}', flush=True)
        assert float(ties.float().mean()) > 0.01  # the check covers tied rows
        assert torch.equal(i_.cpu(), ir)
        # weights within one BF16 ulp (the softmax exp's last FP32 bits differ
        # between torch's CPU kernel and the device libm)
        diff = (w_.cpu().float() - wr.float()).abs()
        assert bool((diff <= wr.float().abs() * 2 ** -7 + 1e-12).all()), float(diff.max())


@pytest.fixture(scope='module')
def c4(device):
    gen = torch.Generator().manual_seed(44)
    batch, time, heads, s, v, j, kk = 4, 8192, 8, 8, 128, 2048, 8
    scores_w, ww, wi = routes(batch, time, j, kk, gen, zipf=1.1)
    scores_r, rw, ri = routes(batch, time, j, kk, gen, zipf=1.1)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    return dict(batch=batch, time=time, heads=heads, s=s, v=v, j=j, kk=kk, scores_w=scores_w, scores_r=scores_r,
                ww=ww, wi=wi, rw=rw, ri=ri, q=q, k=k, v_=v_, g=g, b=b, w=w, state=state)


def test_c4_router_and_dispatch_bit_exact(device, c4):
    from bdm_amd import ops
    announce('C4 router')
    for scores, ww, wi in ((c4['scores_w'], c4['ww'], c4['wi']), (c4['scores_r'], c4['rw'], c4['ri'])):
        w_, i_ = ops.router_select(scores.to(device), bank_count=c4['j'], selected_banks=c4['kk'])
        assert torch.equal(i_.cpu(), wi)
        assert torch.equal(w_.cpu(), ww)
        # rows whose selected set depends on the tie order (equal BF16 scores
        # or pair sums at a top-s or top-B boundary) match too: both sides keep
        # the lower index first
        ties = tie_dependent_rows(scores, c4['j'], c4['kk'])
        print(f'C4 tie-dependent router rows: {float(ties.float().mean()):.4f}', flush=True)
        assert torch.equal(i_.cpu()[ties], wi[ties])
    announce('C4 dispatch')
    meta = ops.dispatch_build(c4['wi'].to(device), c4['ri'].to(device), c4['j'])
    ref = O.dispatch_metadata(c4['wi'], c4['ri'], c4['j'])
    assert torch.equal(meta.order.cpu(), ref.order)
    assert torch.equal(meta.cu_seqlens.cpu(), ref.cu_seqlens)
    lengths = ref.cu_seqlens[1:] - ref.cu_seqlens[:-1]
    assert int(lengths.max()) > 4000  # the skew this configuration exists for


def test_c4_forward_causal_prefix_and_hot_segments(device, c4):
    from bdm_amd import ops
    names = ('q', 'k', 'v_', 'g', 'b', 'w', 'wi', 'ww', 'ri', 'rw')
    dev = [c4[n].to(device) for n in names]
    j, s = c4['j'], c4['s']
    announce('C4 forward full size')
    meta = ops.dispatch_build(dev[6], dev[8], j)
    final = torch.empty(c4['batch'], j, c4['heads'], s, c4['v'], device=device, dtype=torch.float32)
    y = ops.routed_forward(*dev, c4['state'].to(device), meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=0, final_state=final)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    # causality: tokens [:t0] of sequence 0 against the oracle on that prefix alone
    t0 = 384
    prefix = [c4[n][:1, :t0] for n in names]
    ref_y = oracle_reads(*prefix, c4['state'], j, routed_decay=True, state_dtype=torch.float32)
    assert rel_err(y[:1, :t0], ref_y) < TOL, rel_err(y[:1, :t0], ref_y)
    # the three longest segments of sequence 0, head 0: per-event oracle loop
    ref_meta = O.dispatch_metadata(c4['wi'][:1], c4['ri'][:1], j)
    lengths = ref_meta.cu_seqlens[1:] - ref_meta.cu_seqlens[:-1]
    hot = torch.argsort(lengths, descending=True)[:3]
    sl = lambda t: t[:1, :, 0].contiguous()  # noqa: E731
    ev = O.pack_events(*(sl(c4[n]) for n in ('q', 'k', 'v_', 'g', 'b', 'w')), c4['wi'][:1], c4['ww'][:1],
                       c4['ri'][:1], c4['rw'][:1], ref_meta.order, routed_decay=True)
    for bank in hot.tolist():
        lo, hi = int(ref_meta.cu_seqlens[bank]), int(ref_meta.cu_seqlens[bank + 1])
        sub = O.PackedEvents(*(getattr(ev, f)[lo:hi] for f in ('q', 'k', 'v', 'g', 'b', 'w', 'is_read', 'tokens')))
        _, fin = O.packed_recurrence(sub, c4['state'][bank, 0][None].float(), torch.tensor([0, hi - lo]),
                                     s ** -0.5, return_final=True)
        announce('C4 hot segment', bank, hi - lo)
        assert rel_err(final[0, bank, 0], fin[0]) < TOL, (bank, rel_err(final[0, bank, 0], fin[0]))


def test_c5_backward_full_size_truncated_gradient(device):
    """C5 geometry with the upstream gradient nonzero only on the first t0
    tokens of sequence 0: by causality the gradients equal those of the
    truncated problem (oracle autograd) and vanish on every other token."""
    from bdm_amd import bank_training
    gen = torch.Generator().manual_seed(55)
    batch, time, heads, s, v, j, kk, t0 = 4, 2048, 8, 8, 128, 256, 8, 96
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dy = torch.zeros(batch, time, heads * v)
    dy[0, :t0] = torch.randn(t0, heads * v, generator=gen)
    dy = dy.to(torch.bfloat16)
    announce('C5 backward full size')
    leaves = [t.to(device).requires_grad_(True) for t in (q, k, v_, g, b, w, ww, rw, state)]
    y = bank_training(*leaves[:6], wi.to(device), leaves[6], ri.to(device), leaves[7], leaves[8], j, s ** -0.5,
                      state_dtype=torch.bfloat16)
    (y.float() * dy.to(device).float()).sum().backward()
    torch.cuda.synchronize()
    # oracle on the truncated first sequence
    cut = [t[:1, :t0].detach().clone().requires_grad_(True) for t in (q, k, v_, g, b, w, ww, rw)]
    st = state.clone().requires_grad_(True)
    outs = []
    for h in range(heads):
        hs = lambda x: x[:, :, h]  # noqa: E731
        outs.append(O.bank_forward(hs(cut[0]), hs(cut[1]), hs(cut[2]), hs(cut[3]), hs(cut[4]), hs(cut[5]),
                                   wi[:1, :t0], cut[6], ri[:1, :t0], cut[7], st[:, h], j, s ** -0.5,
                                   routed_decay=True, state_dtype=torch.bfloat16, combine='role'))
    (torch.cat(outs, -1).float() * dy[:1, :t0].float()).sum().backward()
    names = ('q', 'k', 'v', 'g', 'b', 'w', 'ww', 'rw')
    for name, leaf, ref in zip(names, leaves[:8], cut):
        grad = leaf.grad.cpu()
        assert rel_err(grad[:1, :t0], ref.grad) < 2e-2, (name, rel_err(grad[:1, :t0], ref.grad))
        rest = torch.cat([grad[:1, t0:].flatten(), grad[1:].flatten()])
        assert float(rest.abs().max()) == 0.0, name
    assert rel_err(leaves[8].grad, st.grad) < 2e-2


def test_c5_segment_order_bit_identical(device, monkeypatch):
    """C5 geometry: the forward and the backward chunk kernel run each XCD's
    segments longest first; every gradient and the output must equal those of
    the bank-order launches (BDM_SEGMENT_ORDER=0) bit for bit."""
    from bdm_amd import bank_training
    gen = torch.Generator().manual_seed(56)
    batch, time, heads, s, v, j, kk = 4, 2048, 8, 8, 128, 256, 8
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dy = torch.randn(batch, time, heads * v, generator=gen).to(torch.bfloat16).to(device)

    def run():
        leaves = [t.to(device).requires_grad_(True) for t in (q, k, v_, g, b, w, ww, rw, state)]
        y = bank_training(*leaves[:6], wi.to(device), leaves[6], ri.to(device), leaves[7], leaves[8], j,
                          s ** -0.5, state_dtype=torch.bfloat16)
        (y.float() * dy.float()).sum().backward()
        torch.cuda.synchronize()
        return [y.detach()] + [leaf.grad for leaf in leaves]

    announce('C5 segment order')
    ordered = run()
    monkeypatch.setenv('BDM_SEGMENT_ORDER', '0')
    banked = run()
    names = ('y', 'q', 'k', 'v', 'g', 'b', 'w', 'ww', 'rw', 'state')
    for name, a, b_ in zip(names, ordered, banked):
        assert torch.equal(a, b_), name
