"""Writes the golden fixtures in this folder from the reference's own CPU code.

Run once, in the build container (which holds the read-only reference at
/root/reference); the GPU box never runs this.  It imports only the
reference's pure-torch modules (bdm.config, bdm.model with backend='reference',
bdm.gdn2_banks), never its Triton kernels, and stores inputs and outputs as
plain tensors:

* ``init_small.pt``     state dict of a seeded layer (pins the role-seeded init)
* ``route_small.pt``    product_key_route on tie-free FP32 and on BF16 scores
* ``dispatch_small.pt`` pack_bank_events permutation, segment bounds, tokens
* ``packed_small.pt``   reference_packed_gdn2 outputs (FP32 and BF16 state)
* ``layer_small.pt``    module forward (backend='reference'), FP32 and BF16,
                        and FP32 gradients of sum(out * dy)
* ``serial_small.pt``   serial_banked_gdn2 outputs and final state

Usage:  python tests/golden/make_golden.py [/root/reference/implementation]
"""

from __future__ import annotations

import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main(reference_root: str) -> None:
    sys.path.insert(0, reference_root)
    from bdm.gdn2_banks import (pack_bank_events, product_key_route, reference_packed_gdn2,  # noqa: E402
                                serial_banked_gdn2)
    from bsdm import BSDMConfig  # noqa: E402
    from bdm import BDMConfig, BankedDeltaMemory  # noqa: E402

    torch.manual_seed(1234)
    configs = {
        'bsdm_h2': dict(cls='bsdm', dim=64, bank_count=16, bank_size=8, selected_banks=4, value_width=32,
                        num_heads=2),
        'bdm_h1': dict(cls='bdm', dim=48, bank_count=12, bank_size=4, selected_banks=3, value_width=16,
                       num_heads=1, training_state_dtype='bfloat16'),
    }

    def build(name, layer_id, seed):
        spec = dict(configs[name])
        cls = BSDMConfig if spec.pop('cls') == 'bsdm' else BDMConfig
        return cls(**spec), BankedDeltaMemory(cls(**spec), layer_id=layer_id, seed=seed, backend='reference')

    # -- init --------------------------------------------------------------
    init = {}
    for name in configs:
        cfg, layer = build(name, layer_id=3, seed=2)
        init[name] = {k: v.detach().clone() for k, v in layer.state_dict().items()}
        init[name + '.meta'] = torch.tensor([3, 2])
    torch.save(init, os.path.join(HERE, 'init_small.pt'))

    # -- router ------------------------------------------------------------
    route = {}
    for bank_count, sel in ((16, 4), (256, 8), (2048, 8), (12, 3)):
        j = sum(__import__('bdm.config', fromlist=['x']).near_square_factors(bank_count))
        tie_free = torch.randn(2, 64, j, dtype=torch.float64).float()
        bf = torch.randn(2, 64, j).to(torch.bfloat16)
        for tag, scores in (('f32', tie_free), ('bf16', bf)):
            w, i = product_key_route(scores, bank_count=bank_count, selected_banks=sel)
            wb, ib = product_key_route(scores, bank_count=bank_count, selected_banks=sel, batch_factors=True)
            route[f'{bank_count}.{sel}.{tag}'] = dict(scores=scores, weights=w, indices=i,
                                                      weights_batched=wb, indices_batched=ib)
    torch.save(route, os.path.join(HERE, 'route_small.pt'))

    # -- dispatch + packed recurrence ----------------------------------------
    batch, time, s, v, j, kw, kr = 2, 24, 8, 16, 12, 3, 3
    gen = torch.Generator().manual_seed(7)

    def routes(k):
        scores = torch.randn(batch, time, j, generator=gen)
        idx = torch.argsort(scores, dim=-1)[..., :k]
        wts = torch.softmax(torch.randn(batch, time, k, generator=gen), -1)
        return idx, wts

    wi, ww = routes(kw)
    ri, rw = routes(kr)
    q = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(batch, time, s, generator=gen), dim=-1)
    vv = torch.randn(batch, time, v, generator=gen)
    g = -torch.rand(batch, time, s, generator=gen) * 0.5
    b = torch.rand(batch, time, s, generator=gen)
    w = torch.rand(batch, time, v, generator=gen)
    state = torch.randn(j, s, v, generator=gen) * 0.1
    dispatch = {}
    packed = {}
    for dtype_name, dtype in (('f32', torch.float32), ('bf16', torch.bfloat16)):
        cast = [t.to(dtype) for t in (q, k, vv)] + [g] + [t.to(dtype) for t in (b, w)]
        for routed in (False, True):
            ev = pack_bank_events(*cast, wi, ww.to(dtype), ri, rw.to(dtype), bank_count=j, routed_decay=routed)
            key = f'{dtype_name}.routed{int(routed)}'
            dispatch[key] = dict(cu_seqlens=ev.cu_seqlens, token_indices=ev.token_indices,
                                 sequence_indices=ev.sequence_indices, read_events=ev.read_events,
                                 q=ev.q, k=ev.k, v=ev.v, g=ev.g, b=ev.b, w=ev.w)
            initial = state.unsqueeze(0).expand(batch, -1, -1, -1).reshape(batch * j, 1, s, v).float()
            for sd_name, sd in (('f32', torch.float32), ('bf16', torch.bfloat16)):
                out = reference_packed_gdn2(q=ev.q, k=ev.k, v=ev.v, g=ev.g, b=ev.b, w=ev.w, scale=s ** -0.5,
                                            initial_state=initial, cu_seqlens=ev.cu_seqlens, state_dtype=sd,
                                            state_interval=16)
                packed[f'{key}.state_{sd_name}'] = out
    dispatch['inputs'] = dict(wi=wi, ww=ww, ri=ri, rw=rw, q=q, k=k, v=vv, g=g, b=b, w=w, state=state,
                              bank_count=torch.tensor(j))
    torch.save(dispatch, os.path.join(HERE, 'dispatch_small.pt'))
    torch.save(packed, os.path.join(HERE, 'packed_small.pt'))

    # -- serial oracle ---------------------------------------------------------
    serial = {}
    for routed in (False, True):
        out, final = serial_banked_gdn2(q, k, vv, g, b, w, state.unsqueeze(0).expand(batch, -1, -1, -1),
                                        wi, ww, ri, rw, scale=s ** -0.5, routed_decay=routed)
        serial[f'routed{int(routed)}'] = dict(out=out, final=final)
    torch.save(serial, os.path.join(HERE, 'serial_small.pt'))

    # -- whole layer (backend='reference') ---------------------------------------
    layer_out = {}
    for name in configs:
        cfg, layer = build(name, layer_id=1, seed=5)
        x = torch.randn(2, 20, cfg.dim, generator=gen)
        dy = torch.randn(2, 20, cfg.dim, generator=gen)
        layer.zero_grad()
        out = layer(x)
        (out * dy).sum().backward()
        grads = {n: p.grad.detach().clone() for n, p in layer.named_parameters() if p.grad is not None}
        with torch.no_grad():
            bf_layer = build(name, layer_id=1, seed=5)[1].to(torch.bfloat16)
            out_bf = bf_layer(x.to(torch.bfloat16))
        layer_out[name] = dict(x=x, dy=dy, out=out.detach(), grads=grads, out_bf16=out_bf)
    torch.save(layer_out, os.path.join(HERE, 'layer_small.pt'))
    print('wrote fixtures to', HERE)


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference/implementation')
