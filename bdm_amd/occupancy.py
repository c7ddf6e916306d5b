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


# ---------------------------------------------------------------------------
# copy-on-write state accounting (APPENDIX.md:511-584; the byte arithmetic is
# the one scripts/verify_results.py:190-235 checks)
#
# A bank holds private state from its first write on; an unwritten bank reads
# the layer's shared initial state.  The state a request holds after n
# positions is therefore its written banks times the bytes of one bank.

def written_banks(indices: Tensor, banks: int, prefixes, valid: Tensor | None = None) -> Tensor:
    """Written banks after each prefix: [B, len(prefixes)] int32, where entry
    (b, i) counts the banks that sequence b writes within its first
    ``prefixes[i]`` positions (valid tokens only).  indices [B, T, K] int64
    write routes.  One pass over the write-only dispatch finds each bank's
    first write; the curve counts first writes below each prefix end."""
    _, _, first = ops.bank_occupancy_totals(None, indices, banks, valid, first_write=True)
    return ops.written_bank_curve(first, prefixes)


def state_value_bytes(written, bank_size: int, width: int, element_bytes: int = 2):
    """Copy-on-write state bytes of ``written`` banks (a count, or the sum of
    counts over layers): written * bank_size * width * element_bytes
    (verify_results.py:207)."""
    return written * bank_size * width * element_bytes


def dense_state_bytes(layers: int, memory_rows: int, width: int, element_bytes: int = 2) -> int:
    """Fully allocated state: L * N * D * b (verify_results.py:194)."""
    return layers * memory_rows * width * element_bytes


def cow_worst_case_bytes(memory_rows: int, accessed_rows: int, history: int, layers: int, width: int,
                         element_bytes: int = 2) -> int:
    """Copy-on-write ceiling after ``history`` positions: each position writes
    at most ``accessed_rows`` = selected_banks * bank_size new rows, capped at
    the N rows of a layer: min(N, K * n) * L * D * b (verify_results.py:220)."""
    return min(memory_rows, accessed_rows * history) * layers * width * element_bytes


def attention_kv_bytes(history: int, layers: int, width: int, element_bytes: int = 2) -> int:
    """The attention KV cache compared against: 2 * n * L * D * b
    (verify_results.py:218)."""
    return 2 * history * layers * width * element_bytes
