"""Stage path of the rounding policy (module forward: BF16 state rounded every
16 events).

The state is rounded at every stage start, so a segment is affine in its start
state only stage by stage.  Segments longer than the piece length (512 events)
run as MODE 3 (every 16-event stage from zero: its R and P, and for each read
the zero-start row and its coefficients on the stage's start state) and a scan
along the stages (M_(k+1) = round(P_k M_k + R_k), each read = c^T M_k + z0),
beside the sequential kernel, which runs the other segments.  The path is
opt-in (BDM_STAGE_PATH=1).  It sums in another FP32 association than the
sequential form, so it is compared within tolerance: against the sequential
kernel (the default) and against the per-event oracle.
"""

import sys

import pytest
import torch

from _inputs import controllers, initial_state, oracle_reads, rel_err, routes

pytestmark = pytest.mark.gpu
TOL = 1e-2


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def skewed_inputs(seed, batch=2, time=4096, heads=8, s=8, v=128, j=1024, kk=8, decay_scale=1.0):
    """Half the tokens route slot 0 of both roles to one of banks 0..3 (banks
    stay distinct per token): those banks' segments hold ~1,100 events (three
    pieces), the other 2,040 segments ~64.  2,048 segments and 4 head groups
    make the forward run its head groups as two overlapped parts, the launch
    the stage path runs beside."""
    gen = torch.Generator().manual_seed(seed)
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    for t in (wi, ri):
        hot = torch.rand(batch, time, generator=gen) < 0.5
        bank = torch.randint(0, 4, (batch, time), generator=gen)
        present = (t == bank[..., None]).any(-1)
        t[..., 0] = torch.where(hot & ~present, bank, t[..., 0])
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    g = g * decay_scale
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    return (q, k, v_, g, b, w, wi, ww, ri, rw, state), (batch, heads, s, v, j)


def forward(ops, dev, meta, geom, final_dtype=torch.bfloat16):
    batch, heads, s, v, j = geom
    final = torch.full((batch, j, heads, s, v), float('nan'), device=dev[0].device, dtype=final_dtype)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=16, final_state=final)
    torch.cuda.synchronize()
    return y, final


@pytest.mark.parametrize('decay', ['mild', 'strong'])
def test_stage_path_matches_sequential_and_oracle(device, monkeypatch, decay):
    """Skewed routes under the rounding policy: the hot sequence of the stage
    path and of the sequential kernel against the per-event oracle (1e-2
    each), and the two paths against each other over every sequence (1e-2:
    they differ in FP32 association and in the BF16 state roundings that
    flips).  'strong' scales the log decays by 200, so stages take the eager
    form."""
    from bdm_amd import ops
    cpu, geom = skewed_inputs(41 if decay == 'mild' else 42, decay_scale=1.0 if decay == 'mild' else 200.0)
    dev = [t.to(device) for t in cpu]
    j = geom[-1]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    lengths = (meta.cu_seqlens[1:] - meta.cu_seqlens[:-1]).cpu()
    assert int((lengths > 512).sum()) >= 8 and int(lengths.max()) > 1024
    announce('stage path', decay)
    monkeypatch.setenv('BDM_STAGE_PATH', '1')
    y_st, f_st = forward(ops, dev, meta, geom)
    monkeypatch.delenv('BDM_STAGE_PATH')
    announce('sequential', decay)
    y_sq, f_sq = forward(ops, dev, meta, geom)
    assert torch.isfinite(y_st).all() and torch.isfinite(f_st).all()
    # the stage path ran: its FP32 sums are associated differently
    assert not (torch.equal(y_st, y_sq) and torch.equal(f_st, f_sq))
    err_y, err_f = rel_err(y_st, y_sq), rel_err(f_st, f_sq)
    print('stage vs sequential', decay, err_y, err_f, flush=True)
    assert err_y < TOL and err_f < TOL, (err_y, err_f)
    # the hot sequence against the oracle (sequences are independent)
    announce('oracle, sequence 0', decay)
    q, k, v_, g, b, w, wi, ww, ri, rw, state = cpu
    one = lambda t: t[:1]  # noqa: E731
    ref_y, ref_f = oracle_reads(*(one(t) for t in (q, k, v_, g, b, w, wi, ww, ri, rw)), state, j,
                                routed_decay=True, state_dtype=torch.bfloat16, interval=16, return_final=True)
    err_y, err_f = rel_err(one(y_st), ref_y), rel_err(one(f_st), ref_f)
    err_y_sq, err_f_sq = rel_err(one(y_sq), ref_y), rel_err(one(f_sq), ref_f)
    print('oracle', decay, 'stage', err_y, err_f, 'sequential', err_y_sq, err_f_sq, flush=True)
    assert err_y < TOL and err_f < TOL, (err_y, err_f)
    assert err_y_sq < TOL and err_f_sq < TOL, (err_y_sq, err_f_sq)


def test_stage_path_fp32_final_state(device, monkeypatch):
    """The final state of a long segment is the scan's unrounded last map,
    stored in FP32 when asked: equal to the BF16 final state after rounding."""
    from bdm_amd import ops
    monkeypatch.setenv('BDM_STAGE_PATH', '1')
    cpu, geom = skewed_inputs(43)
    dev = [t.to(device) for t in cpu]
    meta = ops.dispatch_build(dev[6], dev[8], geom[-1])
    announce('stage path, FP32 final state')
    y32, f32 = forward(ops, dev, meta, geom, torch.float32)
    y16, f16 = forward(ops, dev, meta, geom, torch.bfloat16)
    assert torch.equal(y32, y16)
    assert torch.equal(f32.to(torch.bfloat16), f16)


def test_stage_path_graph_replays_equal_eager(device, monkeypatch):
    """The stage path's launches (on the forward's stage stream, joined to the
    caller's by an event) captured in a HIP graph replay to the eager results,
    with eager launches between the replays."""
    from bdm_amd import ops
    monkeypatch.setenv('BDM_STAGE_PATH', '1')
    cpu, geom = skewed_inputs(44)
    dev = [t.to(device) for t in cpu]
    batch, heads, s, v, j = geom
    meta = ops.dispatch_build(dev[6], dev[8], j)
    x = ops.prepare_routed(*dev[:10], dev[10], bank_count=j)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.bfloat16)

    def run():
        final.fill_(float('nan'))
        return ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                                  round_interval=16, final_state=final, prepared=x)

    announce('stage path eager')
    y = run()
    torch.cuda.synchronize()
    want = (y.clone(), final.clone())
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    announce('stage path under graph capture')
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = run()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, want[0]) and torch.equal(final, want[1])
        run()
        torch.cuda.synchronize()
    del graph
