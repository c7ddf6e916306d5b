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

import dataclasses

import torch

from . import ops
from .config import replay_interval


def _round_interval(bank_size: int, state_dtype: torch.dtype, compact_replay, ctrl_dtype: torch.dtype) -> int:
    """Events between the BF16 roundings of the state (0: never rounded).

    The reference rounds a BF16 training state at every replay checkpoint,
    ``chunk = min(16, max(4, 128 // next_pow2(S)))`` events apart, and an
    explicit ``compact_replay=True`` with BF16 controllers shortens the chunk
    to ``min(8, chunk)`` (role_bank_kernel.py:153-165, 181-193).  With an FP32
    state the chunk only spaces the checkpoints, which never changes results."""
    if state_dtype == torch.bfloat16:
        chunk = replay_interval(bank_size)
        if compact_replay is True and ctrl_dtype == torch.bfloat16:
            chunk = min(8, chunk)
        return chunk
    if state_dtype == torch.float32:
        return 0
    raise ValueError('state_dtype must be torch.float32 or torch.bfloat16')


class RoutedUpdate(torch.autograd.Function):
    """Autograd type of the routed path (routed_update.py:16-53).

    Forward: one shared dispatch for every head, then the fused recurrence +
    ordered combine; when a gradient is needed the forward also stores the
    state at every replay boundary (BF16 when the training state is BF16,
    role_bank_kernel.py:59-66).  Backward: exact chunk replay and reverse
    adjoint, then the token-level VJP; returns gradients for
    (q, k, v, g, b, w, ww, rw, state) and None for wi, ri and the options
    (routed_update.py:49).
    """

    @staticmethod
    def forward(ctx, q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay, state_dtype,
                routed_decay):
        interval = _round_interval(q.shape[-1], state_dtype, compact_replay, q.dtype)
        meta = ops.dispatch_build(wi, ri, bank_count)
        x = ops.prepare_routed(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count=bank_count)
        wants_grad = any(ctx.needs_input_grad[i] for i in (0, 1, 2, 3, 4, 5, 7, 9, 10))
        snapshots, snap_interval = None, 0
        if wants_grad:
            snap_interval = interval or replay_interval(q.shape[-1])
            snapshots = ops.snapshot_buffer(x, snap_interval, torch.bfloat16 if interval else torch.float32)
        raw = ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, state, meta, bank_count=bank_count,
                                 scale=scale, routed_decay=routed_decay, round_interval=interval,
                                 snapshots=snapshots, snapshot_interval=snap_interval, prepared=x)
        if wants_grad:
            # the validated operands themselves, so the backward needs no second
            # pass of checks and copies; the callers' shapes and dtypes for the
            # gradients
            ctx.save_for_backward(x.q, x.k, x.g, x.b, x.v, x.w, x.ww, x.rw, x.ri, x.initial, meta.order,
                                  meta.cu_seqlens, snapshots)
            ctx.geometry = {f.name: getattr(x, f.name) for f in dataclasses.fields(x)
                            if not isinstance(getattr(x, f.name), torch.Tensor)}
            ctx.likes = [(t.shape, t.dtype) for t in (q, k, v, g, b, w, ww, rw, state)]
            ctx.options = (bank_count, scale, routed_decay, interval, snap_interval)
        if q.ndim == 3:
            raw = raw.view(q.shape[0], q.shape[1], v.shape[-1])
        return raw

    @staticmethod
    def backward(ctx, grad_output):
        xq, xk, xg, xb, xv, xw, xww, xrw, xri, xinit, order, cu, snapshots = ctx.saved_tensors
        bank_count, scale, routed_decay, interval, snap_interval = ctx.options
        meta = ops.Dispatch(order, None, None, cu, None)
        x = ops.RoutedInputs(q=xq, k=xk, g=xg, b=xb, v=xv, w=xw, ww=xww, rw=xrw, ri=xri, initial=xinit,
                             **ctx.geometry)
        grads = ops.routed_backward(x, meta, grad_output.contiguous(), snapshots, bank_count=bank_count,
                                    scale=scale, routed_decay=routed_decay, round_interval=interval,
                                    snapshot_interval=snap_interval)
        (q_like, k_like, v_like, g_like, b_like, w_like, ww_like, rw_like, state_like) = ctx.likes
        shape = lambda t, like: t.reshape(like[0]).to(like[1])  # noqa: E731
        dq, dk, dv, dg, db, dw = (shape(t, like) for t, like in ((grads.q, q_like), (grads.k, k_like),
                                                                  (grads.v, v_like), (grads.g, g_like),
                                                                  (grads.b, b_like), (grads.w, w_like)))
        # role_bank_kernel.py:256 / routed_update.py:48: round to the state dtype,
        # then sum the per-sequence adjoints over the batch
        ds = grads.initial.to(state_like[1])
        if x.initial_stride == 0:
            ds = ds.sum(0)
        ds = ds.reshape(state_like[0])
        return (dq, dk, dv, dg, db, dw, None, grads.ww.to(ww_like[1]), None, grads.rw.to(rw_like[1]), ds,
                None, None, None, None, None)


def _options(compact_slot, dtype_slot, compact_replay, state_dtype):
    """Resolve the two optional positions after ``scale``.

    The reference's autograd functions take ``(..., bank_count, scale,
    compact_replay, state_dtype)`` (routed_update.py:18, role_bank_kernel.py:233),
    and the injection point ``heads.forward_heads`` calls its
    ``training_function`` with ``None, None`` in those two positions and
    ``compact_replay=`` as a keyword (heads.py:38-39).  A ``None`` slot defers to
    the keyword; a slot and a keyword that both say something must agree."""
    if compact_slot is not None:
        if compact_replay is not None and compact_replay is not compact_slot:
            raise ValueError(f'compact_replay given twice: {compact_slot!r} by position, {compact_replay!r} by name')
        compact_replay = compact_slot
    if compact_replay is not None and type(compact_replay) is not bool:
        raise ValueError(f'compact_replay takes None or a bool, not {compact_replay!r}')
    if dtype_slot is not None:
        state_dtype = dtype_slot
    if state_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f'state_dtype must be torch.float32 or torch.bfloat16, not {state_dtype!r}')
    return compact_replay, state_dtype


def bank_training(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_slot=None, dtype_slot=None,
                  *, compact_replay=None, state_dtype=torch.float32):
    """Routed-decay bank operator (routed_update.py:52-53).

    Also the ``training_function`` of ``heads.forward_heads`` (heads.py:37-39):
    the two positions after ``scale`` take ``None`` (or the compact-replay flag
    and state dtype, as the reference's autograd function orders them)."""
    compact_replay, state_dtype = _options(compact_slot, dtype_slot, compact_replay, state_dtype)
    return RoutedUpdate.apply(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay,
                              state_dtype, True)


def role_bank_training(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_slot=None,
                       dtype_slot=None, *, compact_replay=None, state_dtype=torch.float32):
    """Bank operator without routed decay (role_bank_kernel.py:258-259); the
    same argument positions as ``bank_training``."""
    compact_replay, state_dtype = _options(compact_slot, dtype_slot, compact_replay, state_dtype)
    return RoutedUpdate.apply(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, scale, compact_replay,
                              state_dtype, False)
