"""Shared-residual router projections and the HIP product-key selection.

``SharedResidualRouter`` keeps the reference module's structure and parameter
names (implementation/bdm/routing.py:11-68).  ``product_key_route`` keeps the
signature and outputs of gdn2_banks.py:74-114; the selection runs in the HIP
router kernel and its backward is the softmax/gather adjoint of the reference's
autograd graph, written in torch ops on the device.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F

from . import ops
from .config import near_square_factors


class SharedResidualRouter(nn.Module):
    """Read and write score projections that share a base map: each role's
    weight and bias are the base's plus that role's own residual, so the two
    roles start equal and learn apart (parameter names of routing.py:11-35)."""

    def __init__(self, input_width: int, output_width: int) -> None:
        super().__init__()
        if min(input_width, output_width) <= 0:
            raise ValueError(f'SharedResidualRouter needs positive widths, got {input_width} -> {output_width}')
        self.base = nn.Linear(input_width, output_width)
        self.read_residual = nn.Linear(input_width, output_width)
        self.write_residual = nn.Linear(input_width, output_width)

    def read(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.base.weight + self.read_residual.weight,
                        self.base.bias + self.read_residual.bias)

    def write(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden, self.base.weight + self.write_residual.weight,
                        self.base.bias + self.write_residual.bias)

    @torch.no_grad()
    def initialize_from_independent(self, *, std: float, read_generator=None, write_generator=None) -> None:
        """Base = mean of two truncated-normal draws; residuals and biases zero
        (routing.py:37-68)."""
        if not std > 0:
            raise ValueError(f'router init std must be > 0, got {std}')
        draws = []
        for generator in (read_generator, write_generator):
            draw = torch.empty_like(self.base.weight)
            nn.init.trunc_normal_(draw, mean=0.0, std=std, a=-3.0 * std, b=3.0 * std, generator=generator)
            draws.append(draw)
        self.base.weight.copy_(0.5 * (draws[0] + draws[1]))
        self.base.bias.zero_()
        for residual in (self.read_residual, self.write_residual):
            residual.weight.zero_()
            residual.bias.zero_()


class _ProductKeyRoute(torch.autograd.Function):
    @staticmethod
    def forward(ctx, projected, bank_count, selected_banks):
        weights, indices = ops.router_select(projected, bank_count=bank_count, selected_banks=selected_banks)
        ctx.save_for_backward(weights, indices)
        ctx.factors = near_square_factors(bank_count)
        ctx.mark_non_differentiable(indices)
        return weights, indices

    @staticmethod
    def backward(ctx, grad_weights, grad_indices):
        weights, indices = ctx.saved_tensors
        j1, j2 = ctx.factors
        w = weights.float()
        dw = grad_weights.float()
        # softmax adjoint, then each selected pair sum feeds one entry of each factor
        dvals = (w * (dw - (w * dw).sum(-1, keepdim=True))).to(weights.dtype).float()
        grad = torch.zeros((*weights.shape[:-1], j1 + j2), device=weights.device, dtype=torch.float32)
        grad[..., :j1].scatter_add_(-1, torch.div(indices, j2, rounding_mode='floor'), dvals)
        grad[..., j1:].scatter_add_(-1, indices.remainder(j2), dvals)
        return grad.to(weights.dtype), None, None


def product_key_route(projected: torch.Tensor, *, bank_count: int, selected_banks: int,
                      batch_factors: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact top-k product-key routing (gdn2_banks.py:74-114).

    ``batch_factors`` is accepted for signature compatibility: the reference
    uses it to share one top-k launch between factors (gdn2_banks.py:93-102);
    its selection is identical and the HIP kernel always treats both factors
    in one launch."""
    del batch_factors
    if projected.ndim != 3:
        raise ValueError('projected routes must be [batch, time, key_width]')
    return _ProductKeyRoute.apply(projected, bank_count, selected_banks)
