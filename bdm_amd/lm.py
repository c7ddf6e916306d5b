"""The language-model shell around the BDM layer.

``BDMLanguageModel`` keeps the reference shell's configuration, module tree,
parameter names and seeded initialisation (implementation/bdm/model.py:143-216,
_shell.py:10-118), so state dicts interchange with the reference and
``forward(tokens, target=None)`` returns the same logits or loss.  Its
``prefill``/``step`` pair follows the reference's whole-model inference
harness (reproduction/experiments/perf_inference_case.py:15-56): each block
runs ``attention.prefill``/``attention.step`` on its own bank cache and the
head projects only the last position.

Under no_grad the shell's elementwise work runs in ``libbdm_hip.so``
(``bdm_rms_norm``, ``bdm_swiglu``) and the feed-forward's two input
projections are one GEMM over their concatenated weights.  With autograd on a
ROCm device RMSNorm runs as ``bdm_rms_norm`` forward and
``bdm_rms_norm_backward`` and the feed-forward's SwiGLU as
``bdm_swiglu_pair`` and ``bdm_swiglu_backward``; the other modules run as the
reference writes them.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .config import BDMConfig
from .model import BankedDeltaMemory

Tensor = torch.Tensor


@dataclass(frozen=True)
class LanguageModelConfig:
    """Shape of the whole language model around the memory layers: the field
    names, defaults and record format of model.py:143-161, so a reference
    record loads unchanged."""
    memory: BDMConfig = field(default_factory=BDMConfig)
    vocab_size: int = 192
    layers: int = 8
    ffn_multiple_of: int = 256
    seed: int = 0
    recompute_ffn: bool = True
    compact_replay: bool | None = None

    def __post_init__(self):
        sizes = {'vocab_size': self.vocab_size, 'layers': self.layers, 'ffn_multiple_of': self.ffn_multiple_of}
        bad = [name for name, value in sizes.items() if value <= 0]
        if bad or self.seed < 0:
            raise ValueError(f'language model needs positive {", ".join(bad) or "sizes"} and a seed >= 0')
        if not (self.compact_replay is None or isinstance(self.compact_replay, bool)):
            raise ValueError(f'compact_replay takes None or a bool, not {self.compact_replay!r}')

    def record(self):
        """Plain-dict form, the memory config nested as its own record."""
        out = asdict(self)
        out['memory'] = self.memory.record()
        return out


class _RMSNormFunction(torch.autograd.Function):
    """RMSNorm with HIP forward and backward kernels: one pass each instead
    of the ~14 FP32 elementwise kernels autograd runs for the torch chain."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        ctx.save_for_backward(x, weight)
        ctx.eps = eps
        return ops.rms_norm(x, weight, eps)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        grad_x, grad_weight = ops.rms_norm_backward(x, grad_out.contiguous(), weight, ctx.eps)
        return grad_x, grad_weight, None


class _SwiGLUFunction(torch.autograd.Function):
    """F.silu(a) * b with HIP forward and backward kernels (one pass each
    instead of silu, the product and their three backward kernels)."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return ops.swiglu_pair(a, b)

    @staticmethod
    def backward(ctx, grad_out):
        a, b = ctx.saved_tensors
        return ops.swiglu_backward(a, b, grad_out)


def _rms_norm_trainable(x: Tensor, weight: Tensor) -> bool:
    return ops.rms_norm_supported(x) and x.shape[-1] <= 4096 and weight.dtype in (torch.bfloat16, torch.float32)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight in FP32, cast back (_shell.py:10-35).
    On a ROCm device the norm and, under autograd, its gradients run in HIP
    kernels; elsewhere the torch chain of the reference."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        if not torch.is_grad_enabled() and ops.rms_norm_supported(x):
            return ops.rms_norm(x, self.weight, self.eps)
        if _rms_norm_trainable(x, self.weight):
            return _RMSNormFunction.apply(x.contiguous(), self.weight, self.eps)
        xf = x.float()
        output = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + self.eps)
        return (output * self.weight.float()).type_as(x)

    def add_norm(self, x: Tensor, residual: Tensor):
        """(residual + x, its norm): a block's residual add followed by the
        next normalization, one kernel under no_grad."""
        if not torch.is_grad_enabled() and ops.rms_norm_supported(x):
            return ops.rms_norm(x, self.weight, self.eps, residual=residual)
        total = residual + x
        return total, self(total)

    def reset_parameters(self):
        nn.init.ones_(self.weight)


class FeedForward(nn.Module):
    """SwiGLU w2(silu(w1 x) * w3 x) with the reference's hidden width rule
    (_shell.py:37-118)."""

    def __init__(self, dim: int, hidden_dim: int, multiple_of: int, ffn_dim_multiplier: float | None,
                 mp_size: int = 1, recompute_activations: bool = False):
        super().__init__()
        hidden_dim = int(2 * hidden_dim / 3)
        if ffn_dim_multiplier is not None:
            hidden_dim = int(ffn_dim_multiplier * hidden_dim)
        hidden_dim = multiple_of * ((hidden_dim + multiple_of - 1) // multiple_of)
        if hidden_dim % mp_size:
            raise ValueError('hidden width must divide over mp_size')
        self.dim, self.hidden_dim = dim, hidden_dim
        self.recompute_activations = recompute_activations
        self.w1 = nn.Linear(dim, hidden_dim, bias=False)
        self.w3 = nn.Linear(dim, hidden_dim, bias=False)
        self.w2 = nn.Linear(hidden_dim, dim, bias=False)
        self._fused_cache = None

    def _fused_input_weight(self) -> Tensor:
        key = tuple((p.data_ptr(), p._version, p.dtype) for p in (self.w1.weight, self.w3.weight))
        if self._fused_cache is None or self._fused_cache[0] != key:
            self._fused_cache = (key, torch.cat([self.w1.weight, self.w3.weight], 0).contiguous())
        return self._fused_cache[1]

    def forward(self, x: Tensor) -> Tensor:
        if not torch.is_grad_enabled() and x.is_cuda and self.hidden_dim % 8 == 0:
            gated = ops.swiglu(ops.linear(x, self._fused_input_weight()), self.hidden_dim)
            return ops.linear(gated, self.w2.weight)
        if (self.recompute_activations and torch.is_grad_enabled() and x.is_cuda and x.dtype == torch.bfloat16
                and x.numel() // self.dim >= 1024):
            return torch.utils.checkpoint.checkpoint(self._forward, x, use_reentrant=False,
                                                     preserve_rng_state=False)
        return self._forward(x)

    def _forward(self, x: Tensor) -> Tensor:
        x1, x3 = self.w1(x), self.w3(x)
        if x1.is_cuda and x1.dtype in (torch.bfloat16, torch.float32):
            return self.w2(_SwiGLUFunction.apply(x1, x3))
        return self.w2(F.silu(x1) * x3)

    def reset_parameters(self, init_std=None, factor=1.0):
        in_std = init_std or self.dim ** -0.5
        out_std = (init_std or self.hidden_dim ** -0.5) / factor
        for w in (self.w1, self.w3):
            nn.init.trunc_normal_(w.weight, mean=0.0, std=in_std, a=-3 * in_std, b=3 * in_std)
        nn.init.trunc_normal_(self.w2.weight, mean=0.0, std=out_std, a=-3 * out_std, b=3 * out_std)


class BDMBlock(nn.Module):
    """Pre-norm residual block: memory layer then SwiGLU (model.py:164-176)."""

    def __init__(self, config: LanguageModelConfig, index: int, backend: str):
        super().__init__()
        dim = config.memory.dim
        self.attention = BankedDeltaMemory(config.memory, layer_id=index, seed=config.seed, backend=backend,
                                           compact_replay=config.compact_replay)
        self.feed_forward = FeedForward(dim, 4 * dim, config.ffn_multiple_of, None,
                                        recompute_activations=config.recompute_ffn)
        self.attention_norm = RMSNorm(dim, eps=config.memory.norm_eps)
        self.ffn_norm = RMSNorm(dim, eps=config.memory.norm_eps)

    def forward(self, hidden: Tensor) -> Tensor:
        hidden = hidden + self.attention(self.attention_norm(hidden))
        return hidden + self.feed_forward(self.ffn_norm(hidden))


class BDMLanguageModel(nn.Module):
    """Token embedding, a stack of BDMBlocks, a final RMSNorm and an untied
    vocabulary head (model.py:179-216).  Module names and the seeded
    initialisation follow the reference, so state dicts interchange bit for
    bit; the memory layers run on the HIP path."""

    def __init__(self, config: LanguageModelConfig, *, backend='hip'):
        super().__init__()
        self.config = config
        self.dim = config.memory.dim
        self.layers = nn.ModuleList([BDMBlock(config, i, backend) for i in range(config.layers)])
        self.tok_embeddings = nn.Embedding(config.vocab_size, self.dim)
        self.norm = RMSNorm(self.dim, eps=config.memory.norm_eps)
        self.output = nn.Linear(self.dim, config.vocab_size, bias=False)
        self._seeded_init()

    def _seeded_init(self) -> None:
        """Every parameter from a seed derived from config.seed (offsets 100
        for the embedding and the head, 6000 + i for memory layer i, 1000 + i
        for feed-forward i), each draw under its own forked RNG so the
        caller's generator state is untouched."""
        root = self.config.seed * 100_000
        bound = self.dim ** -.5

        def seeded(offset, fill):
            with torch.random.fork_rng(devices=[]):
                torch.manual_seed(root + offset)
                fill()

        def fill_ends():
            for weight in (self.tok_embeddings.weight, self.output.weight):
                nn.init.trunc_normal_(weight, mean=0, std=bound, a=-3 * bound, b=3 * bound)

        seeded(100, fill_ends)
        for index, block in enumerate(self.layers):
            block.attention.init_weights(initialization_seed=root + 6000 + index)
            seeded(1000 + index, block.feed_forward.reset_parameters)

    def _hidden(self, tokens: Tensor) -> Tensor:
        hidden = self.tok_embeddings(tokens)
        for block in self.layers:
            hidden = block(hidden)
        return hidden

    def forward(self, tokens: Tensor, target: Tensor | None = None):
        logits = self.output(self.norm(self._hidden(tokens)))
        if target is not None:
            return F.cross_entropy(logits.float().flatten(0, -2), target.flatten())
        return logits

    # -- stateful inference (perf_inference_case.py:15-56) ---------------------------
    def empty_cache(self) -> list:
        return [None] * len(self.layers)

    def prefill(self, tokens: Tensor, caches: list | None = None):
        """Run a prompt through every block, each prefilling its bank cache
        ([B, J, H, S, v] per layer); returns (logits of the last position
        [B, 1, vocab], caches).  No autograd."""
        if torch.is_grad_enabled():
            raise RuntimeError('Stateful inference requires no_grad or inference_mode')
        caches = list(caches) if caches is not None else self.empty_cache()
        if len(caches) != len(self.layers):
            raise ValueError('one cache per layer is required')
        return self._run(tokens, caches, decode=False)

    def step(self, tokens: Tensor, caches: list):
        """One decode position ([B, 1] tokens) against prefilled caches,
        advanced in place; returns (logits [B, 1, vocab], caches)."""
        if torch.is_grad_enabled():
            raise RuntimeError('Stateful inference requires no_grad or inference_mode')
        if tokens.ndim != 2 or tokens.shape[1] != 1:
            raise ValueError('step takes [batch, 1] tokens')
        if len(caches) != len(self.layers) or any(c is None for c in caches):
            raise ValueError('step needs the caches returned by prefill')
        return self._run(tokens, list(caches), decode=True)

    def _fused_decode_supported(self, hidden: Tensor) -> bool:
        ffn = self.layers[0].feed_forward
        return (hidden.shape[0] <= ops.GEMV_MAX_ROWS and ffn.hidden_dim % 8 == 0 and self.dim % 8 == 0
                and max(ffn.hidden_dim, self.dim) <= ops.GEMV_PROLOGUE_MAX_K
                and all(block.attention.step_fused_norm_supported(hidden, block.attention_norm.weight)
                        for block in self.layers))

    def _decode_fused(self, hidden: Tensor, caches: list):
        # One decode token with every one-row elementwise kernel formed inside
        # the GEMV that consumes it: the residual add + attention_norm inside
        # the memory layer's projection, the output interface inside o_proj,
        # the residual add + ffn_norm inside w1|w3, SwiGLU inside w2, and the
        # last residual add + final norm inside the vocabulary head.
        rows = hidden.shape[0]
        delta = None
        for i, block in enumerate(self.layers):
            out, hidden = block.attention.step_fused_norm(hidden, delta, block.attention_norm.weight,
                                                          block.attention_norm.eps, caches[i])
            ffn = block.feed_forward
            gate_up, hidden = ops.gemv_fused(out.reshape(rows, self.dim), ffn._fused_input_weight(), prologue='rms',
                                             residual=hidden.reshape(rows, self.dim),
                                             norm_weight=block.ffn_norm.weight, eps=block.ffn_norm.eps)
            delta = ops.gemv_fused(gate_up, ffn.w2.weight, prologue='swiglu')
            hidden = hidden.view(rows, 1, self.dim)
        logits, _ = ops.gemv_fused(delta.reshape(rows, self.dim), self.output.weight, prologue='rms',
                                   residual=hidden.reshape(rows, self.dim), norm_weight=self.norm.weight,
                                   eps=self.norm.eps)
        return logits.view(rows, 1, -1), caches

    def _run(self, tokens: Tensor, caches: list, decode: bool):
        # Each residual add is fused with the normalization that reads its
        # result: the block's ffn_norm, then the next block's attention_norm
        # (the final norm after the last block).
        hidden = self.tok_embeddings(tokens)
        if decode and self._fused_decode_supported(hidden):
            return self._decode_fused(hidden, caches)
        normed = self.layers[0].attention_norm(hidden)
        for i, block in enumerate(self.layers):
            run = block.attention.step if decode else block.attention.prefill
            out, caches[i] = run(normed, caches[i])
            hidden, normed = block.ffn_norm.add_norm(out, hidden)
            after = self.layers[i + 1].attention_norm if i + 1 < len(self.layers) else self.norm
            hidden, normed = after.add_norm(block.feed_forward(normed), hidden)
        return ops.linear(normed[:, -1:], self.output.weight), caches


BSDMLanguageModel = BDMLanguageModel
