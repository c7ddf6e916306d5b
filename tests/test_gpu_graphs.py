"""Graph-captured decode (GraphDecoder) against the eager layer step, and the
routed prefill hot path captured in one graph against its eager step.

Every replay's output and the cache after it must equal the eager step's
bit for bit: the graph runs the same kernels in the same order.  Between
replays the test runs unrelated eager device work and synchronizes, so a
captured node that only works on the first replay would show here.
"""

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize('cache_dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_graph_decoder_matches_eager_steps(device, cache_dtype):
    from bdm_amd import BSDMConfig, BankedDeltaMemory, GraphDecoder
    cfg = BSDMConfig(dim=128, bank_count=64, bank_size=8, selected_banks=4, value_width=256, num_heads=4)
    layer = BankedDeltaMemory(cfg, layer_id=1, seed=3).to(device=device, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(21)
    batch, prefix, steps = 6, 24, 8
    x = torch.randn(batch, prefix, cfg.dim, generator=gen).to(torch.bfloat16).to(device)
    tokens = torch.randn(steps, batch, 1, cfg.dim, generator=gen).to(torch.bfloat16).to(device)
    announce('graph decoder', cache_dtype)
    with torch.no_grad():
        _, state = layer.prefill(x, state_dtype=cache_dtype)
        eager_state = state.clone()
        graph_state = state.clone()
        decoder = GraphDecoder(layer, graph_state)
        assert torch.equal(graph_state, state)  # building the graph leaves the cache untouched
        noise = torch.randn(1 << 20, device=device)
        for i in range(steps):
            want, _ = layer.step(tokens[i], eager_state)
            got = decoder.step(tokens[i])
            torch.cuda.synchronize()
            assert torch.equal(got, want), i
            assert torch.equal(graph_state, eager_state), i
            noise = (noise * 1.0001 + 1).sum() + noise  # unrelated eager work between replays
            torch.cuda.synchronize()


def test_graph_decoder_rejects_bad_input(device):
    from bdm_amd import BSDMConfig, BankedDeltaMemory, GraphDecoder
    cfg = BSDMConfig(dim=64, bank_count=16, bank_size=8, selected_banks=4, value_width=128, num_heads=2)
    layer = BankedDeltaMemory(cfg, layer_id=0, seed=0).to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        state = layer.create_state(2)
        decoder = GraphDecoder(layer, state)
        with pytest.raises(ValueError):
            decoder.step(torch.zeros(3, 1, cfg.dim, device=device, dtype=torch.bfloat16))


@pytest.mark.parametrize('interval', [16, 0], ids=['rounding', 'prefill'])
def test_hot_path_graph_replays_equal_eager(device, interval):
    """The routed hot path (router pair, dispatch, bdm_forward with its segment
    ranking, recurrence and combine) captured in one HIP graph: three replays,
    with eager steps between them, equal the eager step's y and final state
    bit for bit (no memset nodes, no host synchronisation inside)."""
    from _inputs import controllers, initial_state
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(21)
    batch, time, heads, s, v, j, kk = 2, 1024, 8, 8, 128, 256, 8
    scores_w = torch.randn(batch, time, 32, generator=gen).to(torch.bfloat16).to(device)
    scores_r = torch.randn(batch, time, 32, generator=gen).to(torch.bfloat16).to(device)
    q, k, v_, g, b, w = (t.to(device) for t in controllers(batch, time, heads, s, v, gen))
    state = initial_state(j, heads, s, v, gen, scale=0.05).to(device)
    final = torch.empty(batch, j, heads, s, v, device=device, dtype=torch.bfloat16)

    def step():
        (ww, wi), (rw, ri) = ops.router_select_pair(scores_w, scores_r, bank_count=j, selected_banks=kk)
        meta = ops.dispatch_build(wi, ri, j)
        return ops.routed_forward(q, k, v_, g, b, w, wi, ww, ri, rw, state, meta, bank_count=j, scale=s ** -0.5,
                                  routed_decay=True, round_interval=interval, final_state=final)

    announce('hot path graph', interval)
    with torch.no_grad():
        y_eager = step().clone()
        torch.cuda.synchronize()
        f_eager = final.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_graph = step()
        for _ in range(3):
            final.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y_graph, y_eager)
            assert torch.equal(final, f_eager)
            step()
            torch.cuda.synchronize()
