"""The routed bank operator: the drop-in for the reference's ``bank_training``.

``bank_training(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, *,
compact_replay=None, state_dtype=torch.float32) -> raw`` keeps the argument
order, meaning and return of ``routed_update.bank_training``
(implementation/bdm/routed_update.py:52-53); ``role_bank_training`` is the
same operator without routed decay (role_bank_kernel.py:258-259).  Both accept
the reference's per-head layout (q [B,T,S], state [J,S,v]) and a multi-head
layout (q [B,T,H,S], state [J,H,S,v]) that runs every head on one dispatch.
"""

from __future__ import annotations

import torch

from . import ops
from .config import replay_interval


def _round_interval(bank_size: int, state_dtype: torch.dtype) -> int:
    if state_dtype == torch.bfloat16:
        return replay_interval(bank_size)
    if state_dtype == torch.float32:
        return 0
    raise ValueError('state_dtype must be torch.float32 or torch.bfloat16')


class RoutedUpdate(torch.autograd.Function):
    """Autograd type of the routed path (routed_update.py:16-53).

    Forward: one shared dispatch, then the fused recurrence + ordered combine.
    """

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay, state_dtype,
                routed_decay):
        meta = ops.dispatch_build(wi, ri, bank_count)
        interval = _round_interval(q.shape[-1], state_dtype)
        raw = ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, state, meta, bank_count=bank_count,
                                 scale=scale, routed_decay=routed_decay, round_interval=interval)
        ctx.mark_non_differentiable(wi, ri)
        if q.ndim == 3:
            raw = raw.view(q.shape[0], q.shape[1], v.shape[-1])
        return raw

    @staticmethod
    def backward(ctx, grad_output):
        raise NotImplementedError('the HIP backward of the routed bank path is not built yet')


def bank_training(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, *, compact_replay=None,
                  state_dtype=torch.float32):
    """Routed-decay bank operator (routed_update.py:52-53)."""
    if compact_replay is not None and type(compact_replay) is not bool:
        raise ValueError('compact_replay must be None, True, or False')
    return RoutedUpdate.apply(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay,
                              state_dtype, True)


def role_bank_training(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, *, compact_replay=None,
                       state_dtype=torch.float32):
    """Bank operator without routed decay (role_bank_kernel.py:258-259)."""
    if compact_replay is not None and type(compact_replay) is not bool:
        raise ValueError('compact_replay must be None, True, or False')
    return RoutedUpdate.apply(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay,
                              state_dtype, False)
