"""Graph-captured decode: a layer's whole single-token step (controllers,
both routes, the decode kernel and the output interface) recorded once in a
HIP graph and replayed per token.

The reference decodes eagerly (implementation/bdm/inference.py:161-194).  Here
one step is a few dozen small kernels, so launching them from the host costs
more than running them; replaying a captured graph removes that cost.  The
graph owns a static input buffer and a static output buffer and advances the
cache tensor it was built with in place.
"""

from __future__ import annotations

import torch
from torch import Tensor


class GraphDecoder:
    """Replays ``layer.step`` from a HIP graph.

    ``state`` is the decode cache (``layer.create_state`` or ``layer.prefill``
    output): the graph reads and writes it in place, so it must stay alive and
    keep its storage.  ``step(x)`` copies ``x`` [batch, 1, dim] into the static
    input, replays, and returns the static output: the returned tensor is
    overwritten by the next ``step`` (clone it to keep it).
    """

    def __init__(self, layer, state: Tensor, *, warmup: int = 2) -> None:
        if not state.is_cuda:
            raise ValueError('GraphDecoder needs a cache on a ROCm device')
        self.layer = layer
        self.state = state
        batch = state.shape[0]
        param = next(layer.parameters())
        self.input = torch.zeros(batch, 1, layer.hidden_size, device=state.device, dtype=param.dtype)
        device = state.device
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.no_grad():
            # warm the allocator and the libraries on the capture stream, on a
            # scratch copy of the cache so the real one is untouched
            scratch = state.clone()
            with torch.cuda.stream(side):
                for _ in range(warmup):
                    layer.step(self.input, scratch)
            torch.cuda.current_stream(device).wait_stream(side)
            torch.cuda.synchronize(device)
            del scratch
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(self.graph, stream=side):
                    self.output, _ = layer.step(self.input, state)
            torch.cuda.current_stream(device).wait_stream(side)

    def step(self, x: Tensor) -> Tensor:
        if tuple(x.shape) != tuple(self.input.shape):
            raise ValueError(f'x must be {tuple(self.input.shape)}')
        self.input.copy_(x)
        self.graph.replay()
        return self.output


class LanguageModelGraphDecoder:
    """Replays a whole ``BDMLanguageModel.step`` (embedding, every block's
    norms, memory-layer step and feed-forward, final norm and the vocabulary
    head) from one HIP graph.

    The reference times this loop eagerly under torch.compile
    (reproduction/experiments/perf_inference_case.py:140-160); here the ~250
    kernels of one token are recorded once.  ``caches`` (one per layer, from
    ``model.prefill``) are advanced in place by every replay.  ``step(tokens)``
    copies ``tokens`` [batch, 1] into the static input, replays, and returns
    the static logits [batch, 1, vocab], overwritten by the next call.
    """

    def __init__(self, model, caches, *, warmup: int = 2) -> None:
        if not caches or any(c is None or not c.is_cuda for c in caches):
            raise ValueError('LanguageModelGraphDecoder needs the per-layer caches on a ROCm device')
        self.model = model
        self.caches = list(caches)
        device = self.caches[0].device
        batch = self.caches[0].shape[0]
        self.input = torch.zeros(batch, 1, device=device, dtype=torch.long)
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.no_grad():
            scratch = [c.clone() for c in self.caches]
            with torch.cuda.stream(side):
                for _ in range(warmup):
                    model.step(self.input, scratch)
            torch.cuda.current_stream(device).wait_stream(side)
            torch.cuda.synchronize(device)
            del scratch
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                with torch.cuda.graph(self.graph, stream=side):
                    self.output, _ = model.step(self.input, self.caches)
            torch.cuda.current_stream(device).wait_stream(side)

    def step(self, tokens: Tensor) -> Tensor:
        if tuple(tokens.shape) != tuple(self.input.shape):
            raise ValueError(f'tokens must be {tuple(self.input.shape)}')
        self.input.copy_(tokens)
        self.graph.replay()
        return self.output
