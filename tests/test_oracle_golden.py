"""The CPU oracle against fixtures written by the reference's own code.

The fixtures come from tests/golden/make_golden.py, which imported the
reference's pure-torch modules in the build container.  Bit-exact unless a
comment says otherwise.
"""

import torch

from conftest import load_golden
from oracle import bdm_oracle as O


class _Cfg:
    """Duck-typed config with the reference field names."""

    def __init__(self, **kw):
        defaults = dict(norm_eps=1e-5, routed_decay=False, qk_normalization='original',
                        output_normalization='rms', output_bias=False, training_state_dtype='bfloat16')
        defaults.update(kw)
        self.__dict__.update(defaults)

    @property
    def logical_rows(self):
        return self.bank_count * self.num_heads * self.bank_size


CONFIGS = {
    'bsdm_h2': _Cfg(dim=64, bank_count=16, bank_size=8, selected_banks=4, value_width=32, num_heads=2,
                    routed_decay=True, qk_normalization='nvidia', output_normalization='layer', output_bias=True),
    'bdm_h1': _Cfg(dim=48, bank_count=12, bank_size=4, selected_banks=3, value_width=16, num_heads=1,
                   training_state_dtype='bfloat16'),
}


def test_init_matches_reference_state_dict():
    golden = load_golden('init_small.pt')
    for name, cfg in CONFIGS.items():
        layer = O.OracleBankedDeltaMemory(cfg, layer_id=3, seed=2)
        ours = layer.state_dict()
        ref = golden[name]
        assert set(ours) == set(ref), (name, set(ours) ^ set(ref))
        for key in ref:
            assert torch.equal(ours[key], ref[key]), (name, key)


def test_router_matches_reference():
    golden = load_golden('route_small.pt')
    for key, case in golden.items():
        bank_count, sel, tag = key.split('.')
        bank_count, sel = int(bank_count), int(sel)
        scores = case['scores']
        w, i = O.product_key_route(scores, bank_count=bank_count, selected_banks=sel)
        wb, ib = O.product_key_route(scores, bank_count=bank_count, selected_banks=sel, batch_factors=True)
        assert torch.equal(w, wb) and torch.equal(i, ib)
        # Weights are functions of the selected values only: equal even where
        # torch.topk orders tied values differently.
        assert torch.equal(w, case['weights']), key
        assert torch.equal(case['weights'], case['weights_batched'])
        assert_same_up_to_ties(scores, i, case['indices'], bank_count, sel, key)


def assert_same_up_to_ties(scores, ours, theirs, bank_count, sel, key):
    """Indices must be equal in every row whose selection involves no tie.

    ``torch.topk`` orders equal values by its selection algorithm; the oracle
    pins lower-index-first.  A row may therefore differ only where two
    selected pair sums are equal, or where the last selected sum equals the
    best unselected one.  Both selections must pick the same pair values."""
    j1, j2 = O.near_square_factors(bank_count)
    first, second = scores[..., :j1], scores[..., j1:]

    def pair_values(index):
        a = torch.gather(first, -1, torch.div(index, j2, rounding_mode='floor'))
        b = torch.gather(second, -1, index.remainder(j2))
        return a + b  # in the score dtype, as the reference forms pair sums

    assert torch.equal(pair_values(ours), pair_values(theirs)), key
    mismatch = (ours != theirs).any(-1)
    s = min(sel, j1, j2)
    fv, _ = O.topk_stable(first, s)
    sv, _ = O.topk_stable(second, s)
    table, _ = torch.sort((fv.unsqueeze(-1) + sv.unsqueeze(-2)).flatten(-2), dim=-1, descending=True)
    for row in mismatch.nonzero():
        row = tuple(row)
        chosen = pair_values(ours)[row]
        inner_tie = chosen.unique().numel() < chosen.numel()
        boundary_tie = table[row].numel() > sel and bool(table[row][sel - 1] == table[row][sel])
        assert inner_tie or boundary_tie, (key, row, ours[row], theirs[row])


def test_dispatch_and_packing_match_reference():
    golden = load_golden('dispatch_small.pt')
    inp = golden['inputs']
    j = int(inp['bank_count'])
    meta = O.dispatch_metadata(inp['wi'], inp['ri'], j)
    for dtype_name, dtype in (('f32', torch.float32), ('bf16', torch.bfloat16)):
        cast = [inp[n].to(dtype) for n in ('q', 'k', 'v')] + [inp['g']] + [inp[n].to(dtype) for n in ('b', 'w')]
        for routed in (False, True):
            ref = golden[f'{dtype_name}.routed{int(routed)}']
            assert torch.equal(meta.cu_seqlens, ref['cu_seqlens'])
            assert torch.equal(meta.tokens, ref['token_indices'])
            ev = O.pack_events(*cast, inp['wi'], inp['ww'].to(dtype), inp['ri'], inp['rw'].to(dtype), meta.order,
                               routed_decay=routed)
            assert torch.equal(ev.is_read, ref['read_events'])
            for field in ('q', 'k', 'v', 'g', 'b', 'w'):
                assert torch.equal(getattr(ev, field), ref[field][0, :, 0]), (dtype_name, routed, field)


def test_packed_recurrence_matches_reference():
    golden = load_golden('dispatch_small.pt')
    packed = load_golden('packed_small.pt')
    inp = golden['inputs']
    j = int(inp['bank_count'])
    batch, time, s = inp['q'].shape
    v = inp['v'].shape[-1]
    meta = O.dispatch_metadata(inp['wi'], inp['ri'], j)
    initial = inp['state'].unsqueeze(0).expand(batch, -1, -1, -1).reshape(batch * j, s, v).float()
    for dtype_name, dtype in (('f32', torch.float32), ('bf16', torch.bfloat16)):
        cast = [inp[n].to(dtype) for n in ('q', 'k', 'v')] + [inp['g']] + [inp[n].to(dtype) for n in ('b', 'w')]
        for routed in (False, True):
            ev = O.pack_events(*cast, inp['wi'], inp['ww'].to(dtype), inp['ri'], inp['rw'].to(dtype), meta.order,
                               routed_decay=routed)
            for sd_name, sd in (('f32', torch.float32), ('bf16', torch.bfloat16)):
                ref = packed[f'{dtype_name}.routed{int(routed)}.state_{sd_name}'][0, :, 0]
                loop = O.packed_recurrence(ev, initial, meta.cu_seqlens, s ** -0.5, state_dtype=sd, interval=16)
                assert torch.equal(loop, ref), (dtype_name, routed, sd_name)
                lock = O.lockstep_recurrence(ev, initial, meta.cu_seqlens, s ** -0.5, state_dtype=sd, interval=16)
                torch.testing.assert_close(lock.float(), ref.float(), rtol=1e-2, atol=1e-5)


def test_serial_oracle_matches_reference():
    golden = load_golden('dispatch_small.pt')['inputs']
    serial = load_golden('serial_small.pt')
    batch = golden['q'].shape[0]
    for routed in (False, True):
        out, final = O.serial_banked_gdn2(
            golden['q'], golden['k'], golden['v'], golden['g'], golden['b'], golden['w'],
            golden['state'].unsqueeze(0).expand(batch, -1, -1, -1), golden['wi'], golden['ww'], golden['ri'],
            golden['rw'], scale=golden['q'].shape[-1] ** -0.5, routed_decay=routed)
        assert torch.equal(out, serial[f'routed{int(routed)}']['out'])
        assert torch.equal(final, serial[f'routed{int(routed)}']['final'])


def test_layer_forward_and_gradients_match_reference():
    golden = load_golden('layer_small.pt')
    for name, cfg in CONFIGS.items():
        ref = golden[name]
        layer = O.OracleBankedDeltaMemory(cfg, layer_id=1, seed=5)
        out = layer(ref['x'], combine='index_add', lockstep=False)
        assert torch.equal(out, ref['out']), name
        (out * ref['dy']).sum().backward()
        # Gradients differ only in FP32 accumulation order (the oracle gathers
        # packed fields by token once; the reference concatenates role halves).
        for pname, p in layer.named_parameters():
            if pname in ref['grads']:
                scale = ref['grads'][pname].abs().max().clamp_min(1e-30)
                assert ((p.grad - ref['grads'][pname]).abs().max() / scale) < 1e-6, (name, pname)
        bf = O.OracleBankedDeltaMemory(cfg, layer_id=1, seed=5).to(torch.bfloat16)
        with torch.no_grad():
            out_bf = bf(ref['x'].to(torch.bfloat16), combine='index_add', lockstep=False)
        assert torch.equal(out_bf, ref['out_bf16']), name
