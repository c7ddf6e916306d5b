"""HIP path against the CPU oracle, through the C ABI (bdm_amd.ops wraps it).

Bit-exact: router indices, dispatch permutation/inverse/tokens/bounds.
Tolerance (BF16 state, FP32 math): max|hip - oracle| / max|oracle| <= 1e-2
for read outputs and final bank states; router weights within one BF16 ulp.
"""

import sys

import pytest
import torch

from _inputs import controllers, initial_state, oracle_reads, rel_err, routes
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------------------- router

@pytest.mark.parametrize('bank_count,selected', [(16, 4), (256, 8), (2048, 8), (12, 3), (6, 2), (256, 16),
                                                  (131072, 8), (512, 8), (576, 8), (768, 8), (4096, 8)])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_router_bit_exact(device, bank_count, selected, dtype):
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(bank_count * 31 + selected)
    j1, j2 = O.near_square_factors(bank_count)
    if selected > min(j1, j2) and selected > 8:
        pytest.skip('geometry outside BDMConfig')
    for kind in ('normal', 'ties'):
        if kind == 'normal':
            scores = torch.randn(3, 1000, j1 + j2, generator=gen).to(dtype)
        else:  # coarse grid: many equal factor scores and pair sums
            scores = (torch.randint(-3, 4, (3, 1000, j1 + j2), generator=gen).float() / 2).to(dtype)
        announce('router', bank_count, selected, dtype, kind)
        w, i = ops.router_select(scores.to(device), bank_count=bank_count, selected_banks=selected)
        torch.cuda.synchronize()
        wr, ir = O.product_key_route(scores, bank_count=bank_count, selected_banks=selected)
        assert torch.equal(i.cpu(), ir), (bank_count, selected, dtype, kind)
        # weights: one BF16 ulp (the softmax exp differs in the last FP32 bits
        # between torch's CPU kernel and the device libm), or 1e-6 for FP32 scores
        diff = (w.cpu().float() - wr.float()).abs()
        ulp = wr.float().abs() * (2 ** -7 if dtype == torch.bfloat16 else 1e-6)
        assert bool((diff <= ulp + 1e-12).all()), float(diff.max())
        # few rows (a decode step) take the one-wave-per-row kernel for BF16
        # scores: identical weights and indices to the many-row kernels (one
        # lane per row, or four for B = 8 from factors of 8..64)
        few = scores[:1, :37]
        wf, idf = ops.router_select(few.to(device), bank_count=bank_count, selected_banks=selected)
        torch.cuda.synchronize()
        assert torch.equal(idf.cpu(), i.cpu()[:1, :37]) and torch.equal(wf.cpu(), w.cpu()[:1, :37]), kind


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('bank_count', [256, 2048, 12])
def test_router_pair_equals_two_single_launches(device, dtype, bank_count):
    """Both roles in one launch give the two single-role results bit for bit,
    for contiguous scores and for column slices of one projection (row stride
    wider than the scores)."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(bank_count + 5)
    j1, j2 = O.near_square_factors(bank_count)
    kk = min(8, j1, j2)
    proj = torch.randn(3, 777, 3 * (j1 + j2) + 8, generator=gen).to(dtype).to(device)
    layouts = {'contiguous': (proj[..., :j1 + j2].contiguous(), proj[..., j1 + j2:2 * (j1 + j2)].contiguous()),
               'slices': (proj[..., 8:8 + j1 + j2], proj[..., 8 + j1 + j2:8 + 2 * (j1 + j2)])}
    for name, (a, b) in layouts.items():
        announce('router pair', bank_count, dtype, name)
        (wa, ia), (wb, ib) = ops.router_select_pair(a, b, bank_count=bank_count, selected_banks=kk)
        wa1, ia1 = ops.router_select(a, bank_count=bank_count, selected_banks=kk)
        wb1, ib1 = ops.router_select(b, bank_count=bank_count, selected_banks=kk)
        torch.cuda.synchronize()
        assert torch.equal(ia, ia1) and torch.equal(ib, ib1) and torch.equal(wa, wa1) and torch.equal(wb, wb1), name


def test_router_module_autograd(device):
    from bdm_amd.routing import product_key_route
    gen = torch.Generator().manual_seed(5)
    scores = torch.randn(2, 64, 32, generator=gen)
    dy = torch.randn(2, 64, 8, generator=gen)
    cpu = scores.clone().requires_grad_(True)
    wr, _ = O.product_key_route(cpu, bank_count=256, selected_banks=8)
    (wr * dy).sum().backward()
    announce('router autograd')
    gpu = scores.to(device).requires_grad_(True)
    w, _ = product_key_route(gpu, bank_count=256, selected_banks=8)
    (w * dy.to(device)).sum().backward()
    assert rel_err(gpu.grad, cpu.grad) < 1e-5


# -------------------------------------------------------------------------- dispatch

@pytest.mark.parametrize('batch,time,bank_count,kw,kr', [
    (2, 100, 16, 4, 4), (3, 64, 256, 8, 8), (1, 7, 12, 3, 5), (4, 33, 2048, 8, 8), (2, 40, 16, 0, 4),
    # the per-batch scan: a wave's tile range reloaded (256 tiles over 16 ranges), 2 and 4 chunks of 256 banks,
    # a partial last chunk with a range of 17 tiles (two full loads and a tail); 15 banks take the per-chunk scan
    (1, 8192, 256, 8, 8), (2, 200, 512, 4, 4), (2, 300, 1024, 8, 8), (1, 2100, 1000, 8, 8), (2, 90, 15, 3, 3),
    # the largest bank count of the LDS-mask path (masks and segment starts: 96 KiB of LDS)
    (2, 70, 8192, 8, 8), (1, 5, 4096, 2, 3),
    # above 8192 banks: the radix-sort path
    (2, 50, 16384, 8, 8), (3, 20, 9000, 4, 0), (1, 300, 131072, 8, 8)])
def test_dispatch_bit_exact(device, batch, time, bank_count, kw, kr):
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(batch * 1000 + time)
    wi = torch.stack([torch.randperm(bank_count, generator=gen)[:kw] for _ in range(batch * time)])
    ri = torch.stack([torch.randperm(bank_count, generator=gen)[:kr] for _ in range(batch * time)])
    wi, ri = wi.reshape(batch, time, kw), ri.reshape(batch, time, kr)
    announce('dispatch', batch, time, bank_count, kw, kr)
    meta = ops.dispatch_build(wi.to(device), ri.to(device), bank_count)
    meta.check_routes()
    ref = O.dispatch_metadata(wi, ri, bank_count)
    assert torch.equal(meta.cu_seqlens.cpu(), ref.cu_seqlens)
    assert torch.equal(meta.order.cpu(), ref.order)
    assert torch.equal(meta.inverse.cpu(), ref.inverse)
    assert torch.equal(meta.tokens.cpu(), ref.tokens)


@pytest.mark.parametrize('bank_count', [4, 10000])
def test_dispatch_flags_bad_routes(device, bank_count):
    from bdm_amd import ops
    wi = torch.tensor([[[0, 1], [2, 2]]])  # duplicate bank in one token's writes
    ri = torch.tensor([[[0, 3], [1, 2]]])
    announce('dispatch duplicate flag', bank_count)
    meta = ops.dispatch_build(wi.to(device), ri.to(device), bank_count)
    with pytest.raises(ValueError, match='same bank twice'):
        meta.check_routes()
    wi = torch.tensor([[[0, bank_count + 5], [2, 1]]])  # out of range
    announce('dispatch range flag', bank_count)
    meta = ops.dispatch_build(wi.to(device), ri.to(device), bank_count)
    with pytest.raises(ValueError, match='outside'):
        meta.check_routes()


def test_route_validation_on_the_product_path(device):
    """With route validation on, the routed operator itself raises on
    malformed routes; off (the default), it runs without a host sync."""
    import bdm_amd
    gen = torch.Generator().manual_seed(9)
    q, k, v, g, b, w = controllers(1, 4, 1, 8, 32, gen)
    wi = torch.tensor([[[0, 1], [2, 2], [0, 1], [3, 1]]])  # token 1 writes bank 2 twice
    ri = torch.tensor([[[0, 3], [1, 2], [2, 3], [0, 1]]])
    ww = torch.full((1, 4, 2), 0.5, dtype=torch.bfloat16)
    state = initial_state(4, 1, 8, 32, gen)[:, 0]
    args = [t.to(device) for t in (q[:, :, 0], k[:, :, 0], v[:, :, 0], g[:, :, 0], b[:, :, 0], w[:, :, 0], wi, ww,
                                   ri, ww, state)]
    assert not bdm_amd.route_validation()
    announce('route validation')
    bdm_amd.bank_training(*args, 4, 8 ** -0.5)  # unchecked by default
    bdm_amd.set_route_validation(True)
    try:
        with pytest.raises(ValueError, match='same bank twice'):
            bdm_amd.bank_training(*args, 4, 8 ** -0.5)
    finally:
        bdm_amd.set_route_validation(False)
    torch.cuda.synchronize()


# --------------------------------------------------------------------------- forward

FORWARD_CASES = [
    # batch, time, heads, S, v, J, K, ctrl dtype, routed, state dtype
    (2, 64, 2, 8, 32, 16, 4, torch.bfloat16, True, torch.bfloat16),
    (2, 80, 2, 8, 32, 16, 4, torch.bfloat16, True, torch.float32),
    (1, 50, 1, 4, 16, 12, 3, torch.bfloat16, False, torch.bfloat16),
    (2, 48, 3, 8, 24, 16, 4, torch.float32, True, torch.float32),
    (2, 40, 2, 16, 64, 64, 8, torch.bfloat16, True, torch.bfloat16),
    (1, 60, 4, 8, 128, 256, 8, torch.bfloat16, True, torch.bfloat16),
    (1, 30, 1, 32, 8, 16, 4, torch.bfloat16, True, torch.bfloat16),
    (3, 17, 2, 8, 12, 16, 4, torch.bfloat16, True, torch.bfloat16),
    # heads wider than 256 columns run as 128-column virtual heads on the S = 8 path
    (1, 40, 1, 8, 2048, 16, 4, torch.bfloat16, True, torch.bfloat16),
    (2, 36, 2, 8, 384, 16, 4, torch.bfloat16, True, torch.float32),
    # more than 8192 banks: the radix-sort dispatch
    (1, 40, 2, 8, 32, 16384, 4, torch.bfloat16, True, torch.bfloat16),
]


@pytest.mark.parametrize('case', FORWARD_CASES, ids=[str(i) for i in range(len(FORWARD_CASES))])
def test_forward_matches_oracle(device, case):
    from bdm_amd import ops
    from bdm_amd.config import replay_interval
    batch, time, heads, s, v, j, kk, dtype, routed, state_dtype = case
    gen = torch.Generator().manual_seed(1000 + FORWARD_CASES.index(case))
    _, ww, wi = routes(batch, time, j, kk, gen, dtype)
    _, rw, ri = routes(batch, time, j, kk, gen, dtype)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen, dtype)
    state = initial_state(j, heads, s, v, gen)
    interval = replay_interval(s) if state_dtype == torch.bfloat16 else 0
    ref, ref_final = oracle_reads(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, routed_decay=routed,
                                  state_dtype=state_dtype, interval=interval or 16, return_final=True)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    announce('forward', case)
    meta = ops.dispatch_build(dev[6], dev[8], j)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.float32)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=routed,
                           round_interval=interval, final_state=final)
    torch.cuda.synchronize()
    assert y.shape == (batch, time, heads * v) and y.dtype == dtype
    assert rel_err(y, ref) < TOL, rel_err(y, ref)
    assert rel_err(final, ref_final) < TOL, rel_err(final, ref_final)


@pytest.mark.parametrize('state_dtype', [torch.bfloat16, torch.float32])
def test_forward_long_read_runs_match_oracle(device, state_dtype):
    """Segments whose events are runs of more than one 16-event stage of reads
    only, between runs of writes (the write of a later stage must not use the
    value/gate rows of an earlier one)."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(77)
    batch, time, heads, s, v, j = 2, 160, 2, 8, 128, 4
    t = torch.arange(time)
    # one write and one read bank per token: bank 0 is read by every token and
    # written only in tokens [40, 56) and [120, 128); the other banks share the rest
    wi = torch.where(((t >= 40) & (t < 56)) | ((t >= 120) & (t < 128)), 0, 1 + t % 3)
    wi = wi.expand(batch, time)[..., None].contiguous()
    ri = torch.zeros(batch, time, 1, dtype=torch.long)
    ri[1] = (t % j)[:, None]
    ww = torch.rand(batch, time, 1, generator=gen).to(torch.bfloat16)
    rw = torch.rand(batch, time, 1, generator=gen).to(torch.bfloat16)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen)
    interval = 16 if state_dtype == torch.bfloat16 else 0
    ref, ref_final = oracle_reads(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, routed_decay=True,
                                  state_dtype=state_dtype, interval=16, return_final=True)
    dev = [x.to(device) for x in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    announce('forward long read runs', state_dtype)
    meta = ops.dispatch_build(dev[6], dev[8], j)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.float32)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=interval, final_state=final)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    assert rel_err(y, ref) < TOL, rel_err(y, ref)
    assert rel_err(final, ref_final) < TOL, rel_err(final, ref_final)


@pytest.mark.parametrize('heads,v', [(2, 128), (1, 512)], ids=['h2v128', 'h1v512'])
@pytest.mark.parametrize('decay', ['mild', 'strong'])
def test_forward_cut_segments_match_oracle(device, decay, heads, v):
    """Prefill policy (no rounding inside the recurrence): segments longer
    than the piece length (512 events) run as pieces whose affine summaries
    are composed; every read and every final state must equal the per-event
    oracle.  4 banks, one write and one read bank per token, T = 1100, so a
    segment holds about 550 events, cut into 2 pieces (3 for the hottest).
    v = 512 runs as four 128-column virtual heads."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(91)
    batch, time, s, j = 2, 1100, 8, 4
    wi = torch.randint(0, j, (batch, time, 1), generator=gen)
    wi[0, :400] = 0  # bank 0 of sequence 0 gets the most events
    ri = torch.randint(0, j, (batch, time, 1), generator=gen)
    ri[0, :400] = 0
    ww = torch.rand(batch, time, 1, generator=gen).to(torch.bfloat16)
    rw = torch.rand(batch, time, 1, generator=gen).to(torch.bfloat16)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    if decay == 'strong':  # stages whose scale would underflow run in eager form
        g = g * 200.0
    state = initial_state(j, heads, s, v, gen)
    ref, ref_final = oracle_reads(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, routed_decay=True,
                                  state_dtype=torch.float32, interval=16, return_final=True)
    dev = [x.to(device) for x in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    announce('forward cut segments', decay, heads, v)
    meta = ops.dispatch_build(dev[6], dev[8], j)
    lengths = (meta.cu_seqlens[1:] - meta.cu_seqlens[:-1]).cpu()
    assert int(lengths.max()) > 1024 and int((lengths > 512).sum()) >= 4  # several cut segments, one in 3 pieces
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.float32)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=0, final_state=final)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    assert rel_err(y, ref) < TOL, rel_err(y, ref)
    assert rel_err(final, ref_final) < TOL, rel_err(final, ref_final)


@pytest.mark.parametrize('decay', ['strong', 'mixed', 'none'])
@pytest.mark.parametrize('state_dtype', [torch.bfloat16, torch.float32])
def test_forward_decay_extremes_match_oracle(device, decay, state_dtype):
    """The forward keeps the decay of a stage lazily in a per-row scale and
    switches a stage to explicit decay when that scale would underflow:
    'strong' (g down to -40: every stage explicit), 'mixed' (a few tokens with
    g down to -60 among mild ones) and 'none' (g = 0, the scale stays 1) all
    match the oracle, with final states."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed({'strong': 1, 'mixed': 2, 'none': 3}[decay])
    batch, time, heads, s, v, j, kk = 2, 96, 2, 8, 128, 8, 4
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    if decay == 'strong':
        g = -torch.rand(g.shape, generator=gen) * 40
    elif decay == 'mixed':
        spikes = torch.rand(batch, time, 1, 1, generator=gen) < 0.05
        g = torch.where(spikes, -torch.rand(g.shape, generator=gen) * 60, g)
    else:
        g = torch.zeros_like(g)
    state = initial_state(j, heads, s, v, gen)
    interval = 16 if state_dtype == torch.bfloat16 else 0
    ref, ref_final = oracle_reads(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, routed_decay=True,
                                  state_dtype=state_dtype, interval=16, return_final=True)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    announce('forward decay', decay, state_dtype)
    meta = ops.dispatch_build(dev[6], dev[8], j)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.float32)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=interval, final_state=final)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(final).all()
    assert rel_err(y, ref) < TOL, rel_err(y, ref)
    assert rel_err(final, ref_final) < TOL, rel_err(final, ref_final)


def test_forward_per_head_layout_and_determinism(device):
    from bdm_amd import bank_training
    gen = torch.Generator().manual_seed(11)
    batch, time, heads, s, v, j = 2, 96, 3, 8, 32, 16
    _, ww, wi = routes(batch, time, j, 4, gen)
    _, rw, ri = routes(batch, time, j, 4, gen)
    q, k, v_, g, b, w = (t.to(device) for t in controllers(batch, time, heads, s, v, gen))
    state = initial_state(j, heads, s, v, gen).to(device)
    wi, ww, ri, rw = (t.to(device) for t in (wi, ww, ri, rw))
    announce('per-head layout')
    full = bank_training(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, s ** -0.5, state_dtype=torch.bfloat16)
    again = bank_training(q, k, v_, g, b, w, wi, ww, ri, rw, state, j, s ** -0.5, state_dtype=torch.bfloat16)
    assert torch.equal(full, again)
    for h in range(heads):
        one = bank_training(q[:, :, h], k[:, :, h], v_[:, :, h], g[:, :, h], b[:, :, h], w[:, :, h], wi, ww,
                            ri, rw, state[:, h].contiguous(), j, s ** -0.5, state_dtype=torch.bfloat16)
        assert one.shape == (batch, time, v)
        assert torch.equal(one, full[..., h * v:(h + 1) * v])


# ---------------------------------------------------------------------------- module

def _small_config(**kw):
    from bdm_amd import BSDMConfig
    base = dict(dim=64, bank_count=16, bank_size=8, selected_banks=4, value_width=64, num_heads=2)
    base.update(kw)
    return BSDMConfig(**base)


def test_module_state_dict_interchanges_with_oracle():
    from bdm_amd import BankedDeltaMemory
    cfg = _small_config()
    ours = BankedDeltaMemory(cfg, layer_id=2, seed=3)
    oracle = O.OracleBankedDeltaMemory(cfg, layer_id=2, seed=3)
    a, b = ours.state_dict(), oracle.state_dict()
    assert set(a) == set(b)
    for key in a:
        assert torch.equal(a[key], b[key]), key


def test_module_forward_matches_oracle(device):
    from bdm_amd import BankedDeltaMemory
    cfg = _small_config()
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=1).to(device=device, dtype=torch.bfloat16)
    oracle = O.OracleBankedDeltaMemory(cfg, layer_id=0, seed=1).to(torch.bfloat16)
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(2, 96, cfg.dim, generator=gen).to(torch.bfloat16)
    announce('module forward')
    with torch.no_grad():
        xd = x.to(device)
        q, k, v, g, b, w = layer._controllers(xd)
        rr, wr = layer._route_projections(xd)
        raw = layer.bank_reads(xd)
        out = layer(xd)
        torch.cuda.synchronize()
        # the oracle sees the GPU's controller and score tensors
        ww, wi = O.product_key_route(wr.cpu(), bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
        rw, ri = O.product_key_route(rr.cpu(), bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
        state = oracle.materialize_initial_state()
        ref = oracle_reads(*(t.cpu() for t in (q, k, v, g, b, w)), wi, ww, ri, rw, state, cfg.bank_count,
                           routed_decay=True, state_dtype=torch.bfloat16)
        assert rel_err(raw, ref) < TOL
        # the output interface on the same reads: 0.0000 measured (rms and layer norm)
        ref_out = oracle.project_output(x, raw.cpu())
        assert rel_err(out, ref_out) < TOL


def test_prefill_and_step_match_oracle(device):
    from bdm_amd import BankedDeltaMemory
    cfg = _small_config()
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=4).to(device=device, dtype=torch.bfloat16)
    oracle = O.OracleBankedDeltaMemory(cfg, layer_id=0, seed=4).to(torch.bfloat16)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(2, 40, cfg.dim, generator=gen).to(torch.bfloat16)
    nxt = torch.randn(2, 1, cfg.dim, generator=gen).to(torch.bfloat16)
    for cache_dtype in (torch.float32, torch.bfloat16):
        announce('prefill', cache_dtype)
        with torch.no_grad():
            out, state = layer.prefill(x.to(device), state_dtype=cache_dtype)
            # the controllers and scores prefill used (fused projection + epilogue)
            ctrl, scores, _ = layer._inference_inputs(x.to(device))
            q, k, v, g, b, w = (t.cpu() for t in ctrl)
            rr, wr = (t.cpu() for t in scores)
            ww, wi = O.product_key_route(wr, bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
            rw, ri = O.product_key_route(rr, bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
            init = oracle.create_state(2, torch.float32)
            raw_ref, final_ref = oracle_reads(q, k, v, g, b, w, wi, ww, ri, rw, init.float(), cfg.bank_count,
                                              routed_decay=True, state_dtype=torch.float32, return_final=True)
            assert state.dtype == cache_dtype
            assert rel_err(state, final_ref) < TOL
            announce('step', cache_dtype)
            cpu_state = state.cpu().clone()
            out1, state = layer.step(nxt.to(device), state)
            # oracle step on the same controllers/routes as the GPU step
            ctrl1, scores1, _ = layer._inference_inputs(nxt.to(device))
            q1, k1, v1, g1, b1, w1 = (t.cpu() for t in ctrl1)
            rr1, wr1 = (t.cpu() for t in scores1)
            ww1, wi1 = O.product_key_route(wr1, bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
            rw1, ri1 = O.product_key_route(rr1, bank_count=cfg.bank_count, selected_banks=cfg.selected_banks)
            oracle_state = cpu_state
            heads = []
            for h in range(cfg.num_heads):
                st = oracle_state[:, :, h].float()
                for jj in range(cfg.selected_banks):
                    rows = torch.arange(2)
                    bank = wi1[:, 0, jj]
                    p = ww1[:, 0, jj]
                    eg = g1[:, 0, h].float() * p.float()[:, None]
                    eb = (b1[:, 0, h] * p[:, None]).to(torch.bfloat16)
                    ew = (w1[:, 0, h] * p[:, None]).to(torch.bfloat16)
                    new = O.write_update(st[rows, bank], k1[:, 0, h], eg, eb, ew, v1[:, 0, h])
                    st[rows, bank] = new.to(cache_dtype).float()
                oracle_state[:, :, h] = st.to(cache_dtype)
                vals = []
                for jj in range(cfg.selected_banks):
                    eq = (q1[:, 0, h] * rw1[:, 0, jj][:, None]).to(torch.bfloat16)
                    vals.append(O.read_value(st[torch.arange(2), ri1[:, 0, jj]], eq,
                                             cfg.bank_size ** -0.5).to(torch.bfloat16))
                order = torch.argsort(ri1[:, 0], dim=-1, stable=True)
                total = torch.zeros(2, vals[0].shape[-1])
                stacked = torch.stack(vals, 1)
                for jj in range(cfg.selected_banks):
                    total = (total + stacked[torch.arange(2), order[:, jj]].float()).to(torch.bfloat16).float()
                heads.append(total)
            raw1 = torch.cat(heads, -1)
            assert rel_err(state, oracle_state) < TOL
            ref_out1 = oracle.project_output(nxt, raw1.to(torch.bfloat16).unsqueeze(1))
            assert rel_err(out1, ref_out1) < TOL


@pytest.mark.parametrize('heads,v', [(3, 128), (2, 384), (1, 2048)], ids=['h3v128', 'h2v384', 'h1v2048'])
def test_decode_kernel_matches_oracle(device, heads, v):
    """Wide heads run as column spans (v = 384: 4 spans of 96, v = 2048: 16
    spans of 128); the state and output must not depend on the split."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(21)
    batch, s, j, kk = 6, 8, 64, 8
    _, ww, wi = routes(batch, 1, j, kk, gen)
    _, rw, ri = routes(batch, 1, j, kk, gen)
    ri[0, 0, :3] = wi[0, 0, :3]  # reads of banks written by the same token
    q, k, v_, g, b, w = controllers(batch, 1, heads, s, v, gen)
    for state_dtype in (torch.bfloat16, torch.float32):
        state = (torch.randn(batch, j, heads, s, v, generator=gen) * 0.02).to(state_dtype)
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
                st[rows, bank] = new.to(state_dtype)
            vals = torch.stack([O.read_value(st[rows, ri[:, 0, jj]].float(),
                                             (q[:, 0, h] * rw[:, 0, jj][:, None]).to(q.dtype), s ** -0.5)
                                .to(torch.bfloat16) for jj in range(kk)], 1)
            order = torch.argsort(ri[:, 0], dim=-1, stable=True)
            total = torch.zeros(batch, v)
            for jj in range(kk):
                total = (total + vals[rows, order[:, jj]].float()).to(torch.bfloat16).float()
            ys.append(total)
        announce('decode', heads, v, state_dtype)
        dstate = state.to(device)
        y = ops.decode_step(*(t[:, 0].to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw)), dstate,
                            bank_count=j, scale=s ** -0.5, routed_decay=True)
        torch.cuda.synchronize()
        assert rel_err(dstate, expect) < TOL
        assert rel_err(y, torch.cat(ys, -1)) < TOL
        touched = torch.zeros(batch, j, dtype=torch.bool)
        touched[rows[:, None], wi[:, 0]] = True
        assert torch.equal(dstate.cpu()[~touched], state[~touched])  # untouched banks are bit-identical


# ---------------------------------------------------------------- full benchmark size

@pytest.mark.gpu
def test_segment_order_bit_identical(device, monkeypatch):
    """At C2 size under the module policy the recurrence runs each XCD's
    segments longest first; y and the final state must equal those of the
    bank-order launch (BDM_SEGMENT_ORDER=0) bit for bit, from workspaces
    filled with 0xff (the read rows, then the order: the rounding policy's
    stage path, whose buffers would follow, is switched off; no segment here
    is long enough for it)."""
    from bdm_amd import ops
    monkeypatch.setenv('BDM_STAGE_PATH', '0')
    gen = torch.Generator().manual_seed(77)
    batch, time, heads, s, v, j, kk = 8, 4096, 8, 8, 128, 256, 8
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    ws_bytes = batch * time * kk * heads * v * 2 + batch * j * 4

    def run():
        ws = torch.full((ws_bytes,), 0xff, device=device, dtype=torch.uint8)
        final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.bfloat16)
        y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                               round_interval=16, final_state=final, workspace=ws)
        torch.cuda.synchronize()
        return y, final, ws

    announce('segment order at C2 size')
    y_lpt, f_lpt, ws = run()
    # the order: every segment once, each XCD range in decreasing length
    order = ws[-batch * j * 4:].view(torch.int32).cpu().long()
    lengths = (meta.cu_seqlens[1:] - meta.cu_seqlens[:-1]).cpu()
    rng = batch * j // 8
    for x in range(8):
        part = order[x * rng:(x + 1) * rng]
        assert sorted(part.tolist()) == list(range(x * rng, (x + 1) * rng))
        assert bool((lengths[part][1:] <= lengths[part][:-1]).all())
    monkeypatch.setenv('BDM_SEGMENT_ORDER', '0')
    y_ref, f_ref, _ = run()
    assert torch.equal(y_lpt, y_ref)
    assert torch.equal(f_lpt, f_ref)

@pytest.mark.gpu
@pytest.mark.parametrize('size', ['small', 'c2'])
def test_combine_fold_bit_exact(device, monkeypatch, size):
    """The ordered read combine against a CPU fold of the same read rows: each
    token's KR rows (from the forward's workspace) added in increasing bank id
    (route slot for equal banks), each sum formed in FP32 and rounded to BF16,
    as torch adds BF16 tensors (role_bank_dispatch.py:209-215).  Bit for bit,
    for every token and column.  (The workspace holds the read rows first; the
    stage path's buffers are left out, as no segment is long enough for it.)"""
    from bdm_amd import ops
    monkeypatch.setenv('BDM_STAGE_PATH', '0')
    gen = torch.Generator().manual_seed(79)
    batch, time, heads, s, v, j, kk = (2, 300, 2, 8, 128, 16, 8) if size == 'small' else (8, 4096, 8, 8, 128, 256, 8)
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    nt, hv = batch * time, heads * v
    ws = torch.zeros(nt * kk * hv * 2 + (1 << 20) + batch * j * 4, device=device, dtype=torch.uint8)
    announce('combine fold bit-exact', size)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=16, workspace=ws)
    torch.cuda.synchronize()
    rows = ws[:nt * kk * hv * 2].view(torch.bfloat16).view(nt, kk, hv).cpu()
    banks = ri.reshape(nt, kk)
    order = torch.sort(banks * kk + torch.arange(kk), dim=-1).indices  # bank, then slot
    total = torch.zeros(nt, hv, dtype=torch.bfloat16)
    for step in range(kk):
        total = total + rows[torch.arange(nt), order[:, step]]  # BF16 + BF16: FP32 sum, rounded
    assert torch.equal(y.reshape(nt, hv).cpu().view(torch.int16), total.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize('snapshots', [False, True], ids=['prefill', 'training'])
def test_combine_overlap_bit_identical(device, monkeypatch, snapshots):
    """At C2 size the head-group rounds run as separate launches on two
    streams with each round's combine beside the next round; y, the final
    state and the snapshots must equal those of the serial order
    (BDM_COMBINE_OVERLAP=0) bit for bit, from sentinel-filled outputs; and the
    overlapped sequence captured in a HIP graph must replay to the same
    results, with eager launches between the replays."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(78)
    batch, time, heads, s, v, j, kk = 8, 4096, 8, 8, 128, 256, 8
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    x = ops.prepare_routed(*dev[:10], dev[10], bank_count=j)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.bfloat16)
    snap = ops.snapshot_buffer(x, 16, torch.bfloat16) if snapshots else None

    def run():
        final.fill_(float('nan'))
        if snap is not None:
            snap.fill_(-3.0)  # a finite sentinel: slots past a segment's last boundary stay unwritten
        return ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                                  round_interval=16, final_state=final, snapshots=snap,
                                  snapshot_interval=16 if snapshots else 0, prepared=x)

    def outputs(y):
        torch.cuda.synchronize()
        return [y.clone(), final.clone()] + ([snap.clone()] if snap is not None else [])

    announce('combine overlap at C2 size', snapshots)
    got = outputs(run())
    monkeypatch.setenv('BDM_COMBINE_OVERLAP', '0')
    want = outputs(run())
    for a, c in zip(got, want):
        assert torch.equal(a, c)
    monkeypatch.delenv('BDM_COMBINE_OVERLAP')
    announce('combine overlap under graph capture', snapshots)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = run()
    for _ in range(3):
        graph.replay()
        replayed = outputs(y_graph)
        for a, c in zip(replayed, want):
            assert torch.equal(a, c)
        outputs(run())  # eager work between the replays
    del graph


def test_cut_segment_order_bit_identical(device, monkeypatch):
    """Prefill policy with skewed routes (long segments cut into pieces, many
    short uncut ones): MODE 1 runs every head group's pieces first and the
    segments longest first.  y and the final state must equal those of the
    bank-order launch (BDM_SEGMENT_ORDER=0) bit for bit."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(92)
    batch, time, heads, s, v, j, kk = 2, 2048, 4, 8, 128, 64, 8
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    for t in (wi, ri):  # half the tokens route slot 0 to one of banks 0..3 (banks stay distinct per token)
        hot = torch.rand(batch, time, generator=gen) < 0.5
        bank = torch.randint(0, 4, (batch, time), generator=gen)
        present = (t == bank[..., None]).any(-1)
        t[..., 0] = torch.where(hot & ~present, bank, t[..., 0])
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dev = [x.to(device) for x in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    meta = ops.dispatch_build(dev[6], dev[8], j)
    lengths = (meta.cu_seqlens[1:] - meta.cu_seqlens[:-1]).cpu()
    assert int((lengths > 512).sum()) >= 8 and int((lengths <= 512).sum()) >= 64

    def run():
        final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.float32)
        y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                               round_interval=0, final_state=final)
        torch.cuda.synchronize()
        return y, final

    announce('cut-segment order')
    y_o, f_o = run()
    monkeypatch.setenv('BDM_SEGMENT_ORDER', '0')
    y_b, f_b = run()
    assert torch.equal(y_o, y_b)
    assert torch.equal(f_o, f_b)


@pytest.mark.parametrize('policy', ['module', 'prefill'])
def test_full_size_prefill_c2(device, policy):
    """C2 geometry (B8 T4096 H8 S8 v128 J256 K8): dispatch bit-exact against the
    CPU oracle over all 524,288 events; read outputs and final states of the
    first and the last sequence against the oracle recurrence (sequences are
    independent).  ``module`` is the reference module forward's policy at this
    geometry (BF16 state rounded every 16 events, heads.py:40-46 with
    training_state_dtype='bfloat16'), ``prefill`` the stateful prefill's (FP32
    state, rounded at the handoff, inference.py:1-7)."""
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(2026)
    batch, time, heads, s, v, j, kk = 8, 4096, 8, 8, 128, 256, 8
    _, ww, wi = routes(batch, time, j, kk, gen)
    _, rw, ri = routes(batch, time, j, kk, gen)
    q, k, v_, g, b, w = controllers(batch, time, heads, s, v, gen)
    state = initial_state(j, heads, s, v, gen, scale=0.05)
    dev = [t.to(device) for t in (q, k, v_, g, b, w, wi, ww, ri, rw, state)]
    announce('full size C2 dispatch')
    meta = ops.dispatch_build(dev[6], dev[8], j)
    ref = O.dispatch_metadata(wi, ri, j)
    assert torch.equal(meta.order.cpu(), ref.order)
    assert torch.equal(meta.cu_seqlens.cpu(), ref.cu_seqlens)
    assert torch.equal(meta.inverse.cpu(), ref.inverse)
    announce('full size C2 forward', policy)
    interval = 16 if policy == 'module' else 0
    state_dtype = torch.bfloat16 if policy == 'module' else torch.float32
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.bfloat16)
    y = ops.routed_forward(*dev[:10], dev[10], meta, bank_count=j, scale=s ** -0.5, routed_decay=True,
                           round_interval=interval, final_state=final)
    torch.cuda.synchronize()
    for seq in (0, batch - 1):
        one = lambda t: t[seq:seq + 1]  # noqa: E731
        ref_y, ref_final = oracle_reads(*(one(t) for t in (q, k, v_, g, b, w, wi, ww, ri, rw)), state, j,
                                        routed_decay=True, state_dtype=state_dtype, interval=16,
                                        return_final=True)
        err_y = rel_err(one(y), ref_y)  # per token (its H*v outputs)
        err_s = rel_err(one(final), ref_final)
        assert err_y < TOL and err_s < TOL, (seq, err_y, err_s)
