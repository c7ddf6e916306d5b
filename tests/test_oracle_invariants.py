"""Pins for oracle functions that no reference fixture covers.

The production readout (role_bank_dispatch.py:201-231), the multi-head
prefill/step (the reference serves H=1, S=8 only: inference.py:88-104) and the
recurrence's closed forms are checked here against facts the mathematics
fixes, chosen so that a plausible mistake fails one of them.
"""

import math

import pytest
import torch

from oracle import bdm_oracle as O


def _bf(x):
    return x.to(torch.bfloat16)


# ------------------------------------------------------------------ ordered readout

def test_ordered_readout_exact_sums_equal_index_add():
    """When every partial sum is exact in BF16, the fold order cannot matter:
    the ordered readout equals the index_add_ combine of gdn2_banks.py:280-283."""
    gen = torch.Generator().manual_seed(0)
    nt, kw, kr, width, j = 6, 2, 3, 16, 8
    wi = torch.stack([torch.randperm(j, generator=gen)[:kw] for _ in range(nt)]).reshape(1, nt, kw)
    ri = torch.stack([torch.randperm(j, generator=gen)[:kr] for _ in range(nt)]).reshape(1, nt, kr)
    meta = O.dispatch_metadata(wi, ri, j)
    events = _bf(torch.randint(-8, 9, (meta.order.numel(), width), generator=gen).float())
    is_read = meta.order >= nt * kw
    events[~is_read] = 0
    ordered = O.ordered_readout(events, meta.inverse, nt, kw, kr)
    summed = O.scatter_bank_outputs(events, meta.tokens, nt)
    assert torch.equal(ordered, summed)


def test_ordered_readout_folds_in_increasing_bank_order():
    """1 + 2^-8 - 1 in BF16 depends on the order: folding (1, 2^-8, -1) gives 0,
    folding (-1, 1, 2^-8) gives 2^-8.  Reads in banks 5, 1, 3 carry 2^-8, 1, -1:
    increasing bank id (1, 3, 5) folds 1, -1, 2^-8 -> 2^-8; route order
    (5, 1, 3) folds 2^-8, 1, -1 -> 0."""
    nt, kw, kr, j = 1, 0, 3, 8
    wi = torch.zeros(1, nt, kw, dtype=torch.long)
    ri = torch.tensor([[[5, 1, 3]]])
    meta = O.dispatch_metadata(wi, ri, j)
    slot_value = {0: 2.0 ** -8, 1: 1.0, 2: -1.0}  # original read slot -> value
    events = torch.zeros(3, 2, dtype=torch.bfloat16)
    for slot, value in slot_value.items():
        events[int(meta.inverse[slot])] = value
    out = O.ordered_readout(events, meta.inverse, nt, kw, kr)
    assert float(out[0, 0]) == 2.0 ** -8
    route_order = _bf(_bf(_bf(torch.tensor(2.0 ** -8)) + 1.0) - 1.0)
    assert float(route_order) == 0.0


# ------------------------------------------------------------------ recurrence closed forms

def test_zero_weight_write_leaves_state_unchanged():
    """p = 0: eg = 0, eb = ew = 0, so M' = M (APPENDIX: p scales g, b, w)."""
    gen = torch.Generator().manual_seed(1)
    s, v = 8, 16
    m0 = torch.randn(s, v, generator=gen)
    k = torch.nn.functional.normalize(torch.randn(s, generator=gen), dim=0)
    out = O.write_update(m0, k, torch.zeros(s), torch.zeros(s), torch.zeros(v), torch.randn(v, generator=gen))
    assert torch.equal(out, m0)


def test_single_write_on_zero_state_is_rank_one():
    """From M = 0 one write gives M' = k (w*v)^T exactly (the erase term is 0)."""
    gen = torch.Generator().manual_seed(2)
    s, v = 8, 16
    k, g, b = torch.randn(s, generator=gen), -torch.rand(s, generator=gen), torch.rand(s, generator=gen)
    w, val = torch.rand(v, generator=gen), torch.randn(v, generator=gen)
    out = O.write_update(torch.zeros(s, v), k, g, b, w, val)
    assert torch.allclose(out, k[:, None] * (w * val)[None, :], rtol=0, atol=1e-7)


def test_write_matches_dense_transition_form():
    """M' = (I - k a^T) D M + k (w*v)^T with D = diag(exp g), a = b*k: the
    matrix form of the delta rule, built independently of write_update."""
    gen = torch.Generator().manual_seed(3)
    s, v = 8, 12
    m = torch.randn(s, v, generator=gen, dtype=torch.float64)
    k = torch.randn(s, generator=gen, dtype=torch.float64)
    g = -torch.rand(s, generator=gen, dtype=torch.float64)
    b = torch.rand(s, generator=gen, dtype=torch.float64)
    w = torch.rand(v, generator=gen, dtype=torch.float64)
    val = torch.randn(v, generator=gen, dtype=torch.float64)
    a = b * k
    dense = (torch.eye(s, dtype=torch.float64) - torch.outer(k, a)) @ torch.diag(g.exp()) @ m + torch.outer(k, w * val)
    ours = O.write_update(m.float(), k.float(), g.float(), b.float(), w.float(), val.float())
    assert torch.allclose(ours.double(), dense, rtol=1e-5, atol=1e-6)


def test_reads_are_affine_in_the_initial_state():
    """FP32 state: every read is affine in M0, so
    out(a*A + (1-a)*B) = a*out(A) + (1-a)*out(B) (APPENDIX.md:137-146)."""
    gen = torch.Generator().manual_seed(4)
    batch, time, s, v, j, kk = 1, 24, 8, 16, 4, 2
    q = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    val = torch.randn(batch, time, v, generator=gen)
    g = -torch.rand(batch, time, s, generator=gen) * 0.5
    b, w = torch.rand(batch, time, s, generator=gen), torch.rand(batch, time, v, generator=gen)
    wi = torch.stack([torch.randperm(j, generator=gen)[:kk] for _ in range(time)]).reshape(1, time, kk)
    ri = torch.stack([torch.randperm(j, generator=gen)[:kk] for _ in range(time)]).reshape(1, time, kk)
    ww, rw = torch.rand(1, time, kk, generator=gen), torch.rand(1, time, kk, generator=gen)
    sa, sb = torch.randn(j, s, v, generator=gen), torch.randn(j, s, v, generator=gen)
    run = lambda st: O.bank_forward(q, k, val, g, b, w, wi, ww, ri, rw, st, j, s ** -0.5,  # noqa: E731
                                    routed_decay=True, combine='index_add', lockstep=False)
    alpha = 0.3
    mixed = run(alpha * sa + (1 - alpha) * sb)
    assert torch.allclose(mixed, alpha * run(sa) + (1 - alpha) * run(sb), rtol=1e-4, atol=1e-5)


def test_writes_precede_reads_of_the_same_token():
    """A token that writes and reads one bank reads the post-write state
    (gdn2_banks.py:181-185): from M0 = 0 the read is scale * q.k * (w*v)."""
    s, v = 4, 3
    q = torch.tensor([[[1.0, 0, 0, 0]]])
    k = torch.tensor([[[1.0, 0, 0, 0]]])
    val = torch.tensor([[[2.0, -1.0, 0.5]]])
    g, b = torch.zeros(1, 1, s), torch.zeros(1, 1, s)
    w = torch.ones(1, 1, v)
    wi = ri = torch.tensor([[[0]]])
    one = torch.ones(1, 1, 1)
    out = O.bank_forward(q, k, val, g, b, w, wi, one, ri, one, torch.zeros(2, s, v), 2, 0.5,
                         routed_decay=True, combine='index_add', lockstep=False)
    assert torch.allclose(out[0, 0], 0.5 * val[0, 0])


# ------------------------------------------------------------------ router

def test_product_route_equals_brute_force_on_tie_free_scores():
    """Exact top-B over all J1*J2 pair sums equals the product-key shortcut
    (APPENDIX.md:80-84) when no two candidates tie."""
    gen = torch.Generator().manual_seed(5)
    for bank_count, sel in ((16, 4), (256, 8), (2048, 8)):
        j1, j2 = O.near_square_factors(bank_count)
        scores = torch.randn(2, 50, j1 + j2, generator=gen, dtype=torch.float64)
        w, i = O.product_key_route(scores, bank_count=bank_count, selected_banks=sel)
        wb, ib = O.brute_force_route(scores, bank_count, sel)
        assert torch.equal(i, ib)
        assert torch.allclose(w, wb, rtol=1e-6)  # the reference softmax runs in FP32 (:114)


def test_stable_topk_equals_torch_topk_without_ties():
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(100, 37, generator=gen)
    v1, i1 = O.topk_stable(x, 8)
    v2, i2 = torch.topk(x, 8)
    assert torch.equal(v1, v2) and torch.equal(i1, i2)
    ties = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]])
    assert O.topk_stable(ties, 3)[1].tolist() == [[1, 2, 4]]


# ------------------------------------------------------------------ multi-head prefill / step

def _small_layer(seed=0):
    from bdm_amd import BSDMConfig
    cfg = BSDMConfig(dim=32, bank_count=16, bank_size=4, selected_banks=3, value_width=16, num_heads=2)
    return cfg, O.OracleBankedDeltaMemory(cfg, layer_id=1, seed=seed)


def test_step_equals_one_token_forward_from_the_cache():
    """step(x) from an FP32 cache equals the routed forward of the single token
    x with that cache as per-sequence initial state (FP32 state, ordered
    combine), and leaves the same final state."""
    cfg, layer = _small_layer()
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(3, 1, cfg.dim, generator=gen)
    cache = torch.randn(3, cfg.bank_count, cfg.num_heads, cfg.bank_size, cfg.value_width // cfg.num_heads,
                        generator=gen) * 0.1
    with torch.no_grad():
        raw_fwd, final_fwd = layer.bank_reads(x, state=cache.clone(), state_dtype=torch.float32, return_final=True)
        out_step, state = layer.step(x, cache.clone())
    assert torch.allclose(out_step, layer.project_output(x, raw_fwd), rtol=1e-5, atol=1e-6)
    assert torch.allclose(state, final_fwd, rtol=1e-6, atol=1e-7)


def test_prefill_then_step_equals_longer_prefill():
    """FP32 cache: prefill(x[:T]) then step(x[T]) reproduces prefill(x[:T+1]):
    the same last-token output and the same final state."""
    cfg, layer = _small_layer(seed=3)
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(2, 9, cfg.dim, generator=gen)
    with torch.no_grad():
        full, full_state = layer.prefill(x, state_dtype=torch.float32)
        _, cache = layer.prefill(x[:, :-1], state_dtype=torch.float32)
        last, cache = layer.step(x[:, -1:], cache)
    assert torch.allclose(last, full[:, -1:], rtol=1e-4, atol=1e-5)
    assert torch.allclose(cache, full_state, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize('routed', [True, False])
def test_serial_and_packed_oracles_agree_in_fp32(routed):
    """The literal token-by-token equations (gdn2_banks.py:286-348) and the
    packed per-segment loop compute the same reads with an FP32 state."""
    gen = torch.Generator().manual_seed(9 + routed)
    batch, time, s, v, j, kk = 2, 12, 4, 8, 6, 2
    q = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    val = torch.randn(batch, time, v, generator=gen)
    g = -torch.rand(batch, time, s, generator=gen) * 0.5
    b, w = torch.rand(batch, time, s, generator=gen), torch.rand(batch, time, v, generator=gen)
    wi = torch.stack([torch.randperm(j, generator=gen)[:kk] for _ in range(batch * time)]).reshape(batch, time, kk)
    ri = torch.stack([torch.randperm(j, generator=gen)[:kk] for _ in range(batch * time)]).reshape(batch, time, kk)
    ww = torch.softmax(torch.randn(batch, time, kk, generator=gen), -1)
    rw = torch.softmax(torch.randn(batch, time, kk, generator=gen), -1)
    st = torch.randn(j, s, v, generator=gen) * 0.1
    packed = O.bank_forward(q, k, val, g, b, w, wi, ww, ri, rw, st, j, s ** -0.5, routed_decay=routed,
                            combine='index_add', lockstep=False)
    serial, _ = O.serial_banked_gdn2(q, k, val, g, b, w, st.expand(batch, -1, -1, -1), wi, ww, ri, rw,
                                     scale=s ** -0.5, routed_decay=routed)
    assert torch.allclose(packed, serial, rtol=1e-5, atol=1e-6)
    assert math.isfinite(float(packed.abs().max()))


# ------------------------------------------------------------------ bank occupancy

def _occupancy_inputs(seed=3, batch=3, time=11, banks=20, k=4):
    gen = torch.Generator().manual_seed(seed)
    indices = torch.stack([torch.stack([torch.randperm(banks, generator=gen)[:k] for _ in range(time)])
                           for _ in range(batch)])
    weights = torch.rand(batch, time, k, generator=gen, dtype=torch.float64).float()
    valid = torch.rand(batch, time, generator=gen) < 0.7
    return weights, indices, banks, valid


@pytest.mark.parametrize('masked', [False, True])
def test_bank_occupancy_matches_sets_and_products(masked):
    """hard: the written-bank union by brute force; soft: mean over banks of
    1 - prod(1 - p) by the direct product in FP64 (the closed form of the
    reference's expm1(sum log1p))."""
    weights, indices, banks, valid = _occupancy_inputs()
    value, hard, soft = O.bank_occupancy(weights, indices, banks, valid if masked else None)
    for b in range(weights.shape[0]):
        seen, survive = set(), [1.0] * banks
        for t in range(weights.shape[1]):
            if masked and not bool(valid[b, t]):
                continue
            for j in range(indices.shape[-1]):
                bank = int(indices[b, t, j])
                seen.add(bank)
                survive[bank] *= 1.0 - min(max(float(weights[b, t, j]), 0.0), 1 - 1e-6)
        assert float(hard[b]) == pytest.approx(len(seen) / banks, abs=1e-7)
        assert float(soft[b]) == pytest.approx(sum(1 - s for s in survive) / banks, rel=1e-5)
    assert torch.allclose(value, hard)  # straight-through: the value is the hard union


def test_bank_occupancy_gradient_is_the_soft_union_gradient():
    """d value / d p_e = prod(1 - p) over the other writes to that bank / J."""
    weights, indices, banks, _ = _occupancy_inputs(seed=4)
    w = weights.clone().requires_grad_(True)
    value, _, _ = O.bank_occupancy(w, indices, banks)
    value.sum().backward()
    for b in range(weights.shape[0]):
        for t in range(weights.shape[1]):
            for j in range(indices.shape[-1]):
                bank = int(indices[b, t, j])
                others = 1.0
                for t2 in range(weights.shape[1]):
                    for j2 in range(indices.shape[-1]):
                        if (t2, j2) != (t, j) and int(indices[b, t2, j2]) == bank:
                            others *= 1.0 - float(weights[b, t2, j2])
                # FP32 log-space sums: 1 - p loses digits for p near 1, hence 1e-2
                assert float(w.grad[b, t, j]) == pytest.approx(others / banks, rel=1e-2)


# ------------------------------------------------------------------ copy-on-write state count

@pytest.mark.parametrize('masked', [False, True])
def test_written_bank_curve_matches_sets(masked):
    """Written banks after each prefix, by brute force over the token sets,
    and the first-write positions by a scan in time order."""
    _, indices, banks, valid = _occupancy_inputs(seed=9, batch=3, time=13)
    mask = valid if masked else None
    prefixes = [0, 1, 2, 5, 12, 13, 40]
    curve = O.written_bank_curve(indices, banks, prefixes, mask)
    first = O.first_write_positions(indices, banks, mask)
    for b in range(indices.shape[0]):
        seen_at = {}
        for t in range(indices.shape[1]):
            if masked and not bool(valid[b, t]):
                continue
            for bank in indices[b, t].tolist():
                seen_at.setdefault(bank, t)
        for bank in range(banks):
            assert int(first[b, bank]) == seen_at.get(bank, 2**31 - 1)
        for i, end in enumerate(prefixes):
            assert int(curve[b, i]) == sum(1 for t in seen_at.values() if t < end)


def test_written_bank_curve_boundaries():
    """Known answers: nothing before position 0; the first token writes its K
    distinct banks (the reference's memory data records K / J for one token in
    every layer); the count never decreases, never exceeds min(J, K * t), and
    at the full length equals the hard union of bank_occupancy."""
    weights, indices, banks, _ = _occupancy_inputs(seed=10, batch=4, time=30, banks=64, k=6)
    prefixes = list(range(0, 31))
    curve = O.written_bank_curve(indices, banks, prefixes)
    _, hard, _ = O.bank_occupancy(weights, indices, banks)
    assert torch.all(curve[:, 0] == 0) and torch.all(curve[:, 1] == 6)
    assert torch.all(curve[:, 1:] >= curve[:, :-1])
    for i, t in enumerate(prefixes):
        assert torch.all(curve[:, i] <= min(banks, 6 * t))
    assert torch.equal(curve[:, -1].float() / banks, hard)


def test_index_add_combine_is_one_fp32_sum():
    """The CPU reference's readout, index_add_ on BF16 rows
    (gdn2_banks.py:280-283), adds a token's reads in FP32 and rounds once;
    the 'ordered' fold rounds after every add.  The HIP combine takes the
    former for heads of <= 32 columns, so the fact is pinned here."""
    gen = torch.Generator().manual_seed(17)
    nt, kr, width = 64, 8, 32
    rows = (torch.randn(nt * kr, width, generator=gen) * 3).to(torch.bfloat16)
    tokens = torch.arange(nt).repeat_interleave(kr)
    got = O.scatter_bank_outputs(rows, tokens, nt)
    want = rows.float().reshape(nt, kr, width).sum(1).to(torch.bfloat16)
    assert torch.equal(got, want)
    # the per-add fold differs on these rows, so the two rules are distinct
    inverse = torch.cat([torch.zeros(0, dtype=torch.long), torch.arange(nt * kr)])
    folded = O.ordered_readout(rows, inverse, nt, 0, kr)
    assert not torch.equal(folded, got)
    # and 'role' picks index_add at <= 32 columns, the fold above
    total = torch.zeros(nt, width)
    for j in range(kr):
        total = (total + rows.reshape(nt, kr, width)[:, j].float()).to(torch.bfloat16).float()
    assert torch.equal(folded, total.to(torch.bfloat16))
