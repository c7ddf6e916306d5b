"""Bank occupancy: the Elastic-SDM final-union regularizer over banks.

``bank_occupancy`` keeps the signature and returns of the reference's
``bank_occupancy`` (reproduction/experiments/elastic_bank_regularizer.py:10-25):
``(hard - soft.detach() + soft, hard, soft)`` per sequence, where ``hard`` is
the fraction of banks written at least once and ``soft`` the mean noisy-OR
1 - prod(1 - p).  The per-(sequence, bank) sums come from the HIP kernel over
a write-only dispatch (no [batch, time, J] tensor and no atomics); the
gradient is the noisy-OR's, d soft / d p = -exp(total) * d total / d p / J,
written in torch ops.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import ops


class _OccupancyTotals(torch.autograd.Function):
    @staticmethod
    def forward(ctx, weights, indices, bank_count, valid):
        totals, counts = ops.bank_occupancy_totals(weights, indices, bank_count, valid)
        ctx.save_for_backward(weights, indices, valid if valid is not None else torch.empty(0))
        ctx.has_valid = valid is not None
        ctx.mark_non_differentiable(counts)
        return totals, counts

    @staticmethod
    def backward(ctx, grad_totals, _grad_counts):
        weights, indices, valid = ctx.saved_tensors
        if grad_totals is None:
            return None, None, None, None
        p = weights.float()
        batch = weights.shape[0]
        # d log1p(-clamp(p)) / dp = -1 / (1 - p) inside the clamp range, 0 outside
        inside = (p >= 0) & (p <= 1 - 1e-6)
        slope = torch.where(inside, -1.0 / (1.0 - p.clamp(0, 1 - 1e-6)), torch.zeros_like(p))
        if ctx.has_valid:
            slope = slope * valid[..., None].to(slope.dtype)
        upstream = torch.gather(grad_totals, 1, indices.reshape(batch, -1)).reshape(indices.shape)
        return (upstream * slope).to(weights.dtype), None, None, None


def bank_occupancy(weights: Tensor, indices: Tensor, banks: int, valid: Tensor | None = None):
    """(straight-through value, hard, soft) per sequence
    (elastic_bank_regularizer.py:10-25); weights [B, T, K] route weights,
    indices [B, T, K] int64 banks, valid [B, T] or None."""
    totals, counts = _OccupancyTotals.apply(weights, indices, banks, valid)
    soft = -torch.expm1(totals).mean(-1)
    hard = (counts > 0).float().mean(-1)
    return hard.detach() - soft.detach() + soft, hard, soft
