"""Seeded synthetic inputs shared by the parity tests (CPU tensors)."""

from __future__ import annotations

import math

import torch

from oracle import bdm_oracle as O


def routes(batch, time, bank_count, selected, gen, dtype=torch.bfloat16, zipf: float = 0.0):
    """Router outputs from random factor scores (optionally Zipf-biased per factor)."""
    j1, j2 = O.near_square_factors(bank_count)
    scores = torch.randn(batch, time, j1 + j2, generator=gen)
    if zipf:
        for lo, n in ((0, j1), (j1, j2)):
            perm = torch.randperm(n, generator=gen)
            scores[..., lo:lo + n] -= zipf * torch.log1p(perm.float())
    scores = scores.to(dtype)
    weights, indices = O.product_key_route(scores, bank_count=bank_count, selected_banks=selected)
    return scores, weights, indices


def controllers(batch, time, heads, s, v, gen, dtype=torch.bfloat16):
    """q,k l2-normalised; v silu-like; g <= 0 log decay (FP32); b,w in (0,1)."""
    shape = (batch, time, heads)
    q = torch.nn.functional.normalize(torch.randn(*shape, s, generator=gen), dim=-1).to(dtype)
    k = torch.nn.functional.normalize(torch.randn(*shape, s, generator=gen), dim=-1).to(dtype)
    vv = torch.nn.functional.silu(torch.randn(*shape, v, generator=gen)).to(dtype)
    g = -torch.rand(*shape, s, generator=gen) * 0.3
    b = torch.sigmoid(torch.randn(*shape, s, generator=gen)).to(dtype)
    w = torch.sigmoid(torch.randn(*shape, v, generator=gen)).to(dtype)
    return q, k, vv, g, b, w


def initial_state(bank_count, heads, s, v, gen, scale=0.1, batch=None):
    shape = (bank_count, heads, s, v) if batch is None else (batch, bank_count, heads, s, v)
    return torch.randn(*shape, generator=gen) * scale


def rel_err(ours: torch.Tensor, ref: torch.Tensor, block: int | None = None, floor: float = 0.02) -> float:
    """Worst block-relative error in FP32: the last dimension is cut into
    blocks of ``block`` elements (default: the whole last dimension, i.e. one
    block per token row or state row); each block's max |ours - ref| is
    divided by its own max |ref|, floored at ``floor`` times the tensor's
    max |ref| so that blocks of near-zero values are judged on the scale of
    the rounding noise they carry.  A wrong head, token or column block whose
    values are small next to the tensor's largest value still fails."""
    ours, ref = ours.detach().float().cpu(), ref.detach().float().cpu()
    if ours.shape != ref.shape:
        raise AssertionError(f'shape {tuple(ours.shape)} != {tuple(ref.shape)}')
    if ref.numel() == 0:
        return 0.0
    width = ref.shape[-1] if ref.ndim else 1
    block = width if block is None else block
    if width % block:
        raise ValueError('block must divide the last dimension')
    diff = (ours - ref).abs().reshape(-1, block).amax(-1)
    scale = ref.abs().reshape(-1, block).amax(-1)
    top = float(ref.abs().max())
    return float((diff / scale.clamp_min(max(floor * top, 1e-30))).max())


def global_rel_err(ours: torch.Tensor, ref: torch.Tensor) -> float:
    """max |ours - ref| / max |ref| over the whole tensor."""
    ours, ref = ours.detach().float().cpu(), ref.detach().float().cpu()
    return float((ours - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def oracle_reads(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count, *, routed_decay, state_dtype,
                 interval=None, return_final=False):
    """Oracle of the multi-head HIP forward: per head ``bank_forward`` with the
    production combine rule (ordered fold above 32 columns, FP32 index_add_ at
    or below), heads concatenated (heads.py:65-66)."""
    heads = q.shape[2]
    outs, finals = [], []
    for h in range(heads):
        sl = lambda x: x[:, :, h].contiguous()  # noqa: E731
        st = state[:, h] if state.ndim == 4 else state[:, :, h]
        res = O.bank_forward(sl(q), sl(k), sl(v), sl(g), sl(b), sl(w), wi, ww, ri, rw, st, bank_count,
                             q.shape[-1] ** -0.5, routed_decay=routed_decay, state_dtype=state_dtype,
                             interval=interval, combine='role', lockstep=True, return_final=return_final)
        if return_final:
            res, fin = res
            finals.append(fin)
        outs.append(res)
    y = torch.cat(outs, dim=-1)
    if return_final:
        return y, torch.stack(finals, dim=2)
    return y


def scale_of(s):
    return s ** -0.5 if s else math.nan


def tie_dependent_rows(scores: torch.Tensor, bank_count: int, selected: int) -> torch.Tensor:
    """Rows of router scores whose selected bank *set* depends on how ties are
    broken (gdn2_banks.py:74-114): a factor's s-th and (s+1)-th largest scores
    are equal (the candidate lists change with the tie order), or among the
    s*s pair sums, added in the score dtype, the B-th and (B+1)-th largest are
    equal.  Returns a bool mask over the leading dimensions."""
    j1, j2 = O.near_square_factors(bank_count)
    s = min(selected, j1, j2)
    first, second = scores[..., :j1], scores[..., j1:j1 + j2]
    tie = torch.zeros(scores.shape[:-1], dtype=torch.bool)
    for part, n in ((first, j1), (second, j2)):
        if s < n:
            top = torch.sort(part.float(), dim=-1, descending=True).values
            tie |= top[..., s - 1] == top[..., s]
    fv = torch.sort(first.float(), dim=-1, descending=True).values[..., :s].to(scores.dtype)
    sv = torch.sort(second.float(), dim=-1, descending=True).values[..., :s].to(scores.dtype)
    pair = (fv[..., :, None] + sv[..., None, :]).flatten(-2).float()
    if selected < pair.shape[-1]:
        top = torch.sort(pair, dim=-1, descending=True).values
        tie |= top[..., selected - 1] == top[..., selected]
    return tie
