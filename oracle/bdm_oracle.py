"""CPU restatement of the reference BDM routed-memory path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this file;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker or as the timed CPU baseline.

Every function restates one piece of the reference (p0rc314in/bdm, paths
relative to ``implementation/bdm/``) in plain PyTorch on the CPU.  Each one
names the file:line it follows.  How each is pinned (golden vectors from the
reference, closed forms, invariants, brute force) is listed in the test files
``tests/test_oracle_*.py``.

Two documented choices:

* Top-k tie order.  ``torch.topk`` returns equal values in an order that
  depends on its selection algorithm (and differs between CPU and GPU
  builds).  The oracle pins a deterministic rule: among equal values the
  lower index comes first (a stable descending sort).  On inputs without ties
  this is exactly ``torch.topk``; the tests check both facts.
* Read combine.  ``scatter_bank_outputs`` (``gdn2_banks.py:265-283``) is the
  reference CPU backend's combine; on the CPU, ``index_add_`` in BF16
  accumulates in FP32 and rounds once.  The production readout that the HIP
  path replaces (``role_bank_dispatch.py:201-216``) instead adds the read
  vectors in increasing bank order and rounds to the value dtype after every
  add.  Both are restated: ``scatter_bank_outputs`` and ``ordered_readout``.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

Tensor = torch.Tensor


# ---------------------------------------------------------------------------
# geometry (config.py:7-13, role_bank_kernel.py:153-154)

def near_square_factors(value: int) -> tuple[int, int]:
    """config.py:7-13."""
    if value <= 0:
        raise ValueError('value must be positive')
    for first in range(math.isqrt(value), 0, -1):
        if value % first == 0:
            return first, value // first
    raise AssertionError


def replay_interval(bank_size: int) -> int:
    """role_bank_kernel.py:153-154 and model.py:131."""
    return min(16, max(4, 128 // (1 << (bank_size - 1).bit_length())))


# ---------------------------------------------------------------------------
# router (gdn2_banks.py:74-114)

def topk_stable(x: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """Top-k along the last dim, descending; ties keep the lower index first."""
    values, indices = torch.sort(x, dim=-1, descending=True, stable=True)
    return values[..., :k], indices[..., :k]


def product_key_route(projected: Tensor, *, bank_count: int, selected_banks: int,
                      batch_factors: bool = False) -> tuple[Tensor, Tensor]:
    """gdn2_banks.py:74-114 with the stable tie rule.

    Returns ``(weights, indices)``: weights in the score dtype (softmax in FP32,
    then cast), indices int64 ``row * J2 + col``.  Pair sums are formed in the
    score dtype (``gdn2_banks.py:106``), so BF16 scores round each pair sum.
    """
    if projected.ndim != 3:
        raise ValueError('projected routes must be [batch, time, key_width]')
    j1, j2 = near_square_factors(bank_count)
    if projected.shape[-1] != j1 + j2:
        raise ValueError('projected route width does not match the bank table')
    if not 1 <= selected_banks <= bank_count:
        raise ValueError('selected bank count is outside the bank table')
    first, second = torch.split(projected, [j1, j2], dim=-1)
    s = min(selected_banks, j1, j2)
    if batch_factors:
        # gdn2_banks.py:93-102: one top-k over stacked factors, the shorter
        # padded with -inf.  Padding sits after every real entry, so the
        # selection equals the separate top-k below.
        if j1 == j2:
            stacked = projected.reshape(*projected.shape[:-1], 2, j1)
        else:
            stacked = torch.stack((F.pad(first, (0, j2 - j1), value=-float('inf')), second), dim=-2)
        values, indices = topk_stable(stacked, s)
        fv, sv = values.unbind(-2)
        fi, si = indices.unbind(-2)
    else:
        fv, fi = topk_stable(first, s)
        sv, si = topk_stable(second, s)
    pair = (fv.unsqueeze(-1) + sv.unsqueeze(-2)).flatten(-2)
    count = min(selected_banks, pair.shape[-1])
    values, pair_index = topk_stable(pair, count)
    row = torch.gather(fi, -1, torch.div(pair_index, s, rounding_mode='floor'))
    col = torch.gather(si, -1, pair_index.remainder(s))
    return torch.softmax(values.float(), dim=-1).to(projected.dtype), row * j2 + col


def brute_force_route(projected: Tensor, bank_count: int, selected_banks: int) -> tuple[Tensor, Tensor]:
    """Top-B over all J1*J2 pair sums in FP64 (APPENDIX.md:80-84): the exact
    selection the product-key shortcut must reproduce.  Used to pin the
    router on tie-free inputs."""
    j1, j2 = near_square_factors(bank_count)
    first, second = torch.split(projected.double(), [j1, j2], dim=-1)
    table = (first.unsqueeze(-1) + second.unsqueeze(-2)).flatten(-2)
    values, index = topk_stable(table, selected_banks)
    return torch.softmax(values, dim=-1), index


# ---------------------------------------------------------------------------
# dispatch (role_bank_dispatch.py:15-38, 143-153; gdn2_banks.py:165-185, 237-246)

@dataclass
class Dispatch:
    order: Tensor        # [E] int64: original event index at each packed slot
    inverse: Tensor      # [E] int64: packed slot of each original event
    tokens: Tensor       # [E] int64: flat token of each packed event
    cu_seqlens: Tensor   # [B*J + 1] int64
    keys: Tensor         # [E] int64 sort keys in original order


def dispatch_metadata(wi: Tensor, ri: Tensor, bank_count: int) -> Dispatch:
    """Event keys ``((b*J + bank)*T + t)*2 + is_read`` (role_bank_dispatch.py:23-24,
    gdn2_banks.py:183-184) in original order (writes ``token*KW + j``, then
    reads ``NT*KW + token*KR + j``, role_bank_dispatch.py:19-21), the sorting
    permutation (``:149``), segment bounds by lower bound of ``s*2T``
    (``:27-38``), and the inverse/token maps written by ``_pack`` (``:72-73``)."""
    batch, time, kw = wi.shape
    kr = ri.shape[-1]
    nt = batch * time
    token = torch.arange(nt, dtype=torch.long)
    t_of = token % time
    b_of = token // time
    wkey = (((b_of[:, None] * bank_count + wi.reshape(nt, kw)) * time + t_of[:, None]) * 2)
    rkey = (((b_of[:, None] * bank_count + ri.reshape(nt, kr)) * time + t_of[:, None]) * 2 + 1)
    keys = torch.cat((wkey.reshape(-1), rkey.reshape(-1)))
    sorted_keys, order = torch.sort(keys, stable=True)
    bounds = torch.arange(batch * bank_count + 1, dtype=torch.long) * (2 * time)
    cu = torch.searchsorted(sorted_keys, bounds, side='left')
    inverse = torch.empty_like(order)
    inverse[order] = torch.arange(order.numel(), dtype=torch.long)
    original_token = torch.cat((token.repeat_interleave(kw), token.repeat_interleave(kr)))
    return Dispatch(order, inverse, original_token[order], cu, keys)


@dataclass
class PackedEvents:
    q: Tensor
    k: Tensor
    v: Tensor
    g: Tensor
    b: Tensor
    w: Tensor
    is_read: Tensor
    tokens: Tensor


def pack_events(q, k, v, g, b, w, wi, ww, ri, rw, order: Tensor, *, routed_decay: bool) -> PackedEvents:
    """Route-weighted per-event fields in packed order.

    ``_pack`` (role_bank_dispatch.py:47-73) and ``pack_bank_events``
    (gdn2_banks.py:196-224): eq = q*r, eb = b*p, ew = w*p rounded once to the
    source dtype; eg = g (or g*p in FP32 with routed decay,
    routed_update.py:5-13 / gdn2_banks.py:210-211).  Fields a role does not use
    are zero.  Inputs are per head: q,k,g,b [B,T,S]; v,w [B,T,V]."""
    batch, time, s = q.shape
    nt = batch * time
    kw, kr = wi.shape[-1], ri.shape[-1]
    is_read = order >= nt * kw
    route = torch.where(is_read, order - nt * kw, order)
    token = torch.where(is_read, route // kr, route // kw)
    fq, fk, fv, fg, fb, fw = (t.reshape(nt, t.shape[-1]) for t in (q, k, v, g, b, w))
    wsel = torch.where(is_read, 0, route)
    rsel = torch.where(is_read, route, 0)
    write_weight = ww.reshape(-1)[wsel]
    read_weight = rw.reshape(-1)[rsel]
    rmask = is_read.unsqueeze(-1)
    wmask = ~rmask
    eq = torch.where(rmask, fq[token] * read_weight.unsqueeze(-1), 0).to(fq.dtype)
    eb = torch.where(wmask, fb[token] * write_weight.unsqueeze(-1), 0).to(fb.dtype)
    ew = torch.where(wmask, fw[token] * write_weight.unsqueeze(-1), 0).to(fw.dtype)
    g_tok = fg[token].float()
    if routed_decay:
        g_tok = g_tok * write_weight.float().unsqueeze(-1)
    eg = torch.where(wmask, g_tok, 0)
    return PackedEvents(eq, fk[token], fv[token], eg, eb, ew, is_read, token)


# ---------------------------------------------------------------------------
# recurrence (gdn2_banks.py:11-43, role_bank_kernel.py:32-73)

class _StoredState(torch.autograd.Function):
    """Rounded storage with a straight-through adjoint (gdn2_banks.py:11-19)."""

    @staticmethod
    def forward(ctx, value, dtype):
        return value.to(dtype).float()

    @staticmethod
    def backward(ctx, grad):
        return grad, None


def _store(value: Tensor, dtype) -> Tensor:
    return _StoredState.apply(value, dtype)


def write_update(state: Tensor, k: Tensor, g: Tensor, b: Tensor, w: Tensor, v: Tensor) -> Tensor:
    """One write on an [S, V] (or batched [..., S, V]) FP32 state.

    hd = exp(g) * M;  u = w*v - (b*k)^T hd;  M' = hd + k u^T
    (role_bank_kernel.py:40-43, gdn2_banks.py:37-41)."""
    decayed = state * g.float().exp().unsqueeze(-1)
    erase = ((b.float() * k.float()).unsqueeze(-1) * decayed).sum(-2)
    update = w.float() * v.float() - erase
    return decayed + k.float().unsqueeze(-1) * update.unsqueeze(-2)


def read_value(state: Tensor, q: Tensor, scale: float) -> Tensor:
    """z = scale * q^T M (role_bank_kernel.py:71-72, gdn2_banks.py:42)."""
    return scale * (q.float().unsqueeze(-1) * state).sum(-2)


def packed_recurrence(events: PackedEvents, initial: Tensor, cu_seqlens: Tensor, scale: float, *,
                      state_dtype=torch.float32, interval: int = 16, return_final: bool = False):
    """Per-segment sequential loop of ``reference_packed_gdn2`` (gdn2_banks.py:22-43).

    ``initial`` is [segments, S, V]; segment ``i`` runs packed events
    ``cu[i]:cu[i+1]``.  With a BF16 ``state_dtype`` the state is stored
    (rounded) at the segment start and before every event whose offset in the
    segment is a multiple of ``interval`` (gdn2_banks.py:33-36,
    role_bank_kernel.py:57-64).  Returns per-event read outputs [E, V] in the
    value dtype (write rows are zero) and, when asked, the final FP32 states.
    """
    e_total = events.v.shape[0]
    output = torch.zeros(e_total, events.v.shape[-1], dtype=torch.float32)
    finals = []
    rows = []
    for sequence in range(cu_seqlens.numel() - 1):
        start, end = int(cu_seqlens[sequence]), int(cu_seqlens[sequence + 1])
        state = _store(initial[sequence], state_dtype)
        for e in range(start, end):
            if state_dtype == torch.bfloat16 and (e - start) % interval == 0:
                state = _store(state, state_dtype)
            if bool(events.is_read[e]):
                rows.append((e, read_value(state, events.q[e], scale)))
            else:
                state = write_update(state, events.k[e], events.g[e], events.b[e], events.w[e], events.v[e])
        finals.append(state)
    if rows:
        index = torch.tensor([r[0] for r in rows], dtype=torch.long)
        output = output.index_put((index,), torch.stack([r[1] for r in rows]))
    out = output.to(events.v.dtype)
    if return_final:
        return out, torch.stack(finals) if finals else initial.float()
    return out


def lockstep_recurrence(events: PackedEvents, initial: Tensor, cu_seqlens: Tensor, scale: float, *,
                        state_dtype=torch.float32, interval: int = 16, return_final: bool = False):
    """The same recurrence as ``packed_recurrence`` with all segments advanced
    together: step ``p`` applies the ``p``-th event of every segment that has
    one.  Each segment sees the identical sequence of operations; only the
    Python loop is reorganised, which makes larger parity cases affordable.
    Its agreement with ``packed_recurrence`` is itself a test."""
    lengths = cu_seqlens[1:] - cu_seqlens[:-1]
    nseg = lengths.numel()
    state = _store(initial.float(), state_dtype) if nseg else initial.float()
    e_total = events.v.shape[0]
    output = torch.zeros(e_total, events.v.shape[-1], dtype=torch.float32)
    max_len = int(lengths.max()) if nseg else 0
    starts = cu_seqlens[:-1]
    for p in range(max_len):
        live = (lengths > p).nonzero().squeeze(-1)
        e = starts[live] + p
        if state_dtype == torch.bfloat16 and p % interval == 0:
            state = state.clone()
            state[live] = _store(state[live], state_dtype)
        reading = events.is_read[e]
        wl, we = live[~reading], e[~reading]
        rl, re_ = live[reading], e[reading]
        if wl.numel():
            new = write_update(state[wl], events.k[we], events.g[we], events.b[we], events.w[we], events.v[we])
            state = state.clone()
            state[wl] = new
        if rl.numel():
            output = output.index_put((re_,), read_value(state[rl], events.q[re_], scale))
    out = output.to(events.v.dtype)
    if return_final:
        return out, state
    return out


# ---------------------------------------------------------------------------
# combine (gdn2_banks.py:265-283, role_bank_dispatch.py:201-231)

def scatter_bank_outputs(event_outputs: Tensor, tokens: Tensor, nt: int) -> Tensor:
    """index_add_ of packed outputs by token (gdn2_banks.py:280-283)."""
    out = event_outputs.new_zeros(nt, event_outputs.shape[-1])
    out.index_add_(0, tokens, event_outputs)
    return out


def ordered_readout(event_outputs: Tensor, inverse: Tensor, nt: int, kw: int, kr: int) -> Tensor:
    """Production readout (role_bank_dispatch.py:201-216): each token adds its
    read vectors in increasing packed position (= increasing bank id) and
    rounds to the value dtype after every add."""
    dtype = event_outputs.dtype
    positions = inverse[nt * kw:].reshape(nt, kr)
    ranked, _ = torch.sort(positions, dim=-1)
    total = torch.zeros(nt, event_outputs.shape[-1], dtype=torch.float32)
    for j in range(kr):
        total = (total + event_outputs[ranked[:, j]].float()).to(dtype).float()
    return total.to(dtype)


# ---------------------------------------------------------------------------
# literal bank oracle (gdn2_banks.py:286-348)

def serial_banked_gdn2(q, k, v, g, b, w, initial_state, wi, ww, ri, rw, *, scale=None,
                       routed_decay=False) -> tuple[Tensor, Tensor]:
    """Token-by-token dense-bank equations with no packing and no rounding.

    initial_state [B, J, S, V].  For each token: the KW writes in route order,
    each on the bank state left by the previous one, then the KR reads of the
    post-write states weighted by r (gdn2_banks.py:314-347)."""
    batch, time, s = q.shape
    state = initial_state.float().clone()
    scale = s ** -0.5 if scale is None else scale
    rows = torch.arange(batch)
    outputs = []
    for t in range(time):
        for j in range(wi.shape[-1]):
            bank = wi[:, t, j]
            p = ww[:, t, j].float().unsqueeze(-1)
            log_decay = g[:, t].float() * (p if routed_decay else 1.0)
            new = write_update(state[rows, bank], k[:, t], log_decay, b[:, t].float() * p,
                               w[:, t].float() * p, v[:, t])
            state = state.clone()
            state[rows, bank] = new
        y = torch.zeros(batch, v.shape[-1])
        for j in range(ri.shape[-1]):
            bank = ri[:, t, j]
            reading = (q[:, t].float().unsqueeze(-1) * state[rows, bank]).sum(-2)
            y = y + scale * rw[:, t, j].float().unsqueeze(-1) * reading
        outputs.append(y)
    return torch.stack(outputs, dim=1).to(v.dtype), state


# ---------------------------------------------------------------------------
# the routed bank operator (routed_update.py:16-53 / heads.py:25-66 with backend='reference')

def bank_forward(q, k, v, g, b, w, wi, ww, ri, rw, state, bank_count: int, scale: float, *,
                 routed_decay: bool, state_dtype=torch.float32, interval: int | None = None,
                 combine: str = 'ordered', lockstep: bool = True, return_final: bool = False):
    """One head of the routed path: dispatch, pack, recurrence, combine.

    q,k,g,b [B,T,S]; v,w [B,T,V]; wi,ri int64 [B,T,K]; ww,rw [B,T,K];
    ``state`` [J,S,V] shared by the batch or [B,J,S,V] per sequence.
    ``combine='ordered'`` is the per-add rounded fold of the production
    readout, ``'index_add'`` the CPU reference backend's FP32 sum, and
    ``'role'`` the production rule by head width: ordered above 32 columns,
    index_add_ at or below (role_bank_dispatch.py:222-226).  Differentiable
    through torch autograd."""
    batch, time, s = q.shape
    nt = batch * time
    meta = dispatch_metadata(wi, ri, bank_count)
    ev = pack_events(q, k, v, g, b, w, wi, ww, ri, rw, meta.order, routed_decay=routed_decay)
    if state.ndim == 3:
        initial = state.unsqueeze(0).expand(batch, -1, -1, -1)
    else:
        initial = state
    initial = initial.reshape(batch * bank_count, s, v.shape[-1]).float()
    interval = replay_interval(s) if interval is None else interval
    run = lockstep_recurrence if lockstep else packed_recurrence
    out, final = run(ev, initial, meta.cu_seqlens, scale, state_dtype=state_dtype, interval=interval,
                     return_final=True)
    if combine == 'role':
        combine = 'ordered' if v.shape[-1] > 32 else 'index_add'
    if combine == 'ordered':
        raw = ordered_readout(out, meta.inverse, nt, wi.shape[-1], ri.shape[-1])
    else:
        raw = scatter_bank_outputs(out, meta.tokens, nt)
    raw = raw.reshape(batch, time, -1)
    if return_final:
        return raw, final.reshape(batch, bank_count, s, v.shape[-1])
    return raw


# ---------------------------------------------------------------------------
# initialisation (_parameters.py:69-177, routing.py:37-68)

def bank_occupancy(weights: Tensor, indices: Tensor, banks: int, valid: Tensor | None = None):
    """Elastic-SDM final-union occupancy over banks
    (reproduction/experiments/elastic_bank_regularizer.py:10-25).

    Per sequence: ``hard`` = fraction of banks written at least once (valid
    tokens only); ``soft`` = mean over banks of the noisy OR
    1 - prod(1 - p) = -expm1(sum log1p(-p)), p clamped to [0, 1 - 1e-6];
    returns ``(hard - soft.detach() + soft, hard, soft)`` (straight-through).
    The token axis is collapsed before the scatter, as the reference does."""
    batch = weights.shape[0]
    addresses = indices.reshape(batch, -1)
    event_mask = torch.ones_like(indices, dtype=torch.int32)
    if valid is not None:
        event_mask = valid[..., None].expand_as(indices).to(torch.int32)
    log_survival = torch.log1p(-weights.float().clamp(0, 1 - 1e-6)) * event_mask
    totals = torch.zeros(batch, banks, dtype=torch.float32)
    totals = totals.scatter_add(1, addresses, log_survival.reshape(batch, -1))
    soft = -torch.expm1(totals).mean(-1)
    counts = torch.zeros(batch, banks, dtype=torch.int32)
    counts.scatter_add_(1, addresses, event_mask.reshape(batch, -1))
    hard = (counts > 0).float().mean(-1)
    return hard.detach() - soft.detach() + soft, hard, soft


def role_generator(layer_id: int, role: str, seed: int) -> torch.Generator:
    """Seed ``(seed XOR blake2b_8('bank_sparse_gdn2.{layer}.{role}')) mod 2^63``
    (_parameters.py:69-84)."""
    key = f'bank_sparse_gdn2.{layer_id}.{role}'.encode()
    digest = int.from_bytes(hashlib.blake2b(key, digest_size=8).digest(), byteorder='little')
    generator = torch.Generator(device='cpu')
    generator.manual_seed((seed ^ digest) % (1 << 63))
    return generator


class OracleRouter(nn.Module):
    """Shared base plus read/write residuals (routing.py:11-35)."""

    def __init__(self, width_in: int, width_out: int):
        super().__init__()
        self.base = nn.Linear(width_in, width_out)
        self.read_residual = nn.Linear(width_in, width_out)
        self.write_residual = nn.Linear(width_in, width_out)

    def read(self, hidden):
        return F.linear(hidden, self.base.weight + self.read_residual.weight,
                        self.base.bias + self.read_residual.bias)

    def write(self, hidden):
        return F.linear(hidden, self.base.weight + self.write_residual.weight,
                        self.base.bias + self.write_residual.bias)


class OracleBankedDeltaMemory(nn.Module):
    """CPU equation model of ``BankedDeltaMemory(backend='reference')``
    (model.py:24-140, heads.py:11-66, _parameters.py:40-232) with identical
    parameter names and shapes, so state dicts interchange with the HIP module."""

    def __init__(self, config, *, layer_id: int = 0, seed: int = 0):
        super().__init__()
        self.config = config
        d, j, s, h = config.dim, config.bank_count, config.bank_size, config.num_heads
        self.layer_id = layer_id
        self.initialization_seed = seed * 100_000 + 6000 + layer_id
        self.bank_count, self.bank_size, self.num_heads = j, s, h
        self.value_width = config.value_width
        self.head_value_width = config.value_width // h
        self.hidden_size = d
        key_width = h * s
        route_width = sum(near_square_factors(j))
        self.q_proj = nn.Linear(d, key_width, bias=False)
        self.k_proj = nn.Linear(d, key_width, bias=False)
        self.v_proj = nn.Linear(d, config.value_width, bias=False)
        self.shared_router = OracleRouter(d, route_width)
        self.f_proj = nn.Sequential(nn.Linear(d, self.head_value_width, bias=False),
                                    nn.Linear(self.head_value_width, key_width, bias=False))
        self.b_proj = nn.Linear(d, key_width, bias=False)
        self.w_proj = nn.Linear(d, config.value_width, bias=False)
        self.A_log = nn.Parameter(torch.empty(h, dtype=torch.float32))
        self.dt_bias = nn.Parameter(torch.empty(key_width, dtype=torch.float32))
        rows, cols = near_square_factors(config.logical_rows)
        self.register_parameter('initial_state', None)
        self.initial_row_factor = nn.Parameter(torch.zeros(rows, self.head_value_width))
        self.initial_column_factor = nn.Parameter(torch.zeros(cols, self.head_value_width))
        self.output_gate = nn.Linear(d, config.value_width, bias=True)
        self.output_norm_weight = nn.Parameter(torch.ones(config.value_width))
        if config.output_normalization == 'layer':
            self.output_norm_bias = nn.Parameter(torch.zeros(config.value_width))
        self.o_proj = nn.Linear(config.value_width, d, bias=config.output_bias)
        self.init_weights(self.initialization_seed)

    @torch.no_grad()
    def init_weights(self, seed: int):
        """_parameters.py:86-177 and routing.py:37-68."""
        gen = lambda role: role_generator(self.layer_id, role, seed)  # noqa: E731
        for name, module in self.named_modules():
            if isinstance(module, nn.Linear) and not name.startswith('shared_router.'):
                nn.init.xavier_uniform_(module.weight, gain=2 ** -2.5, generator=gen(f'{name}.weight'))
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
        std = self.hidden_size ** -0.5
        draws = []
        for role in ('read_router.weight', 'write_router.weight'):
            draw = torch.empty_like(self.shared_router.base.weight)
            nn.init.trunc_normal_(draw, mean=0.0, std=std, a=-3 * std, b=3 * std, generator=gen(role))
            draws.append(draw)
        router = self.shared_router
        router.base.weight.copy_(0.5 * (draws[0] + draws[1]))
        for lin in (router.base, router.read_residual, router.write_residual):
            lin.bias.zero_()
        router.read_residual.weight.zero_()
        router.write_residual.weight.zero_()
        self.A_log.uniform_(1.0, 16.0, generator=gen('decay_rate')).log_()
        log_dt = torch.empty_like(self.dt_bias).uniform_(math.log(0.001), math.log(0.1),
                                                         generator=gen('time_step'))
        dt = log_dt.exp().clamp_min(1e-4)
        self.dt_bias.copy_(dt + torch.log(-torch.expm1(-dt)))
        for role, factor in (('initial_state.row', self.initial_row_factor),
                             ('initial_state.column', self.initial_column_factor)):
            nn.init.trunc_normal_(factor, mean=0.0, std=std, a=-3 * std, b=3 * std, generator=gen(role))
            factor.mul_(1 / math.sqrt(2))
        self.output_norm_weight.fill_(1.0)
        if hasattr(self, 'output_norm_bias'):
            self.output_norm_bias.zero_()

    def materialize_initial_state(self) -> Tensor:
        """M0[j,h,s] = U[n // Q] + Z[n % Q] with n = (j*H + h)*S + s
        (_parameters.py:48-51, README.md:128-134).  Shape [J, H, S, v]."""
        return (self.initial_row_factor[:, None, :] + self.initial_column_factor[None, :, :]).reshape(
            self.bank_count, self.num_heads, self.bank_size, self.head_value_width)

    def normalize_qk(self, x: Tensor) -> Tensor:
        """_parameters.py:214-220 (CPU formula of the 'nvidia' mode)."""
        if self.config.qk_normalization == 'nvidia':
            xf = x.float()
            return (xf * torch.rsqrt(xf.square().sum(-1, keepdim=True) + 1e-6)).to(x.dtype)
        return F.normalize(x.float(), dim=-1).to(x.dtype)

    def controllers(self, hidden: Tensor):
        """heads.py:11-22: per-head q,k,g,b [B,T,H,S] and v,w [B,T,H,v]."""
        shape = (*hidden.shape[:-1], self.num_heads)
        q = self.normalize_qk(F.silu(self.q_proj(hidden)).reshape(*shape, self.bank_size))
        k = self.normalize_qk(F.silu(self.k_proj(hidden)).reshape(*shape, self.bank_size))
        v = F.silu(self.v_proj(hidden)).reshape(*shape, self.head_value_width)
        g = -self.A_log.float().exp()[:, None] * F.softplus(
            (self.f_proj(hidden).float() + self.dt_bias.float()).reshape(*shape, self.bank_size))
        b = self.b_proj(hidden).sigmoid().reshape(*shape, self.bank_size)
        w = self.w_proj(hidden).sigmoid().reshape(*shape, self.head_value_width)
        return q, k, v, g, b, w

    def routes(self, hidden: Tensor):
        j, sel = self.bank_count, self.config.selected_banks
        rw, ri = product_key_route(self.shared_router.read(hidden), bank_count=j, selected_banks=sel)
        ww, wi = product_key_route(self.shared_router.write(hidden), bank_count=j, selected_banks=sel)
        return ww, wi, rw, ri

    def project_output(self, hidden: Tensor, raw: Tensor) -> Tensor:
        """_parameters.py:222-232."""
        if self.config.output_normalization == 'layer':
            normalized = F.layer_norm(raw, (self.value_width,), self.output_norm_weight,
                                      self.output_norm_bias, self.config.norm_eps)
            return self.o_proj(normalized * torch.sigmoid(self.output_gate(hidden)).to(raw.dtype))
        variance = raw.float().square().mean(dim=-1, keepdim=True)
        normalized = raw * torch.rsqrt(variance + self.config.norm_eps).to(raw.dtype)
        normalized = normalized * self.output_norm_weight.to(raw.dtype)
        return self.o_proj(normalized * torch.sigmoid(self.output_gate(hidden)).to(raw.dtype))

    def bank_reads(self, hidden: Tensor, *, combine: str = 'role', lockstep: bool = True,
                   state=None, state_dtype=None, return_final: bool = False):
        """Concatenated per-head reads [B,T,V] (heads.py:25-66)."""
        q, k, v, g, b, w = self.controllers(hidden)
        ww, wi, rw, ri = self.routes(hidden)
        initial = self.materialize_initial_state() if state is None else state
        dtype = getattr(torch, self.config.training_state_dtype) if state_dtype is None else state_dtype
        reads, finals = [], []
        for head in range(self.num_heads):
            sl = lambda x: x[..., head, :].contiguous()  # noqa: E731
            st = initial[:, head] if initial.ndim == 4 else initial[:, :, head]
            out = bank_forward(sl(q), sl(k), sl(v), sl(g), sl(b), sl(w), wi, ww, ri, rw, st,
                               self.bank_count, self.bank_size ** -0.5,
                               routed_decay=self.config.routed_decay, state_dtype=dtype,
                               combine=combine, lockstep=lockstep, return_final=return_final)
            if return_final:
                out, fin = out
                finals.append(fin)
            reads.append(out)
        raw = torch.cat(reads, dim=-1)
        if return_final:
            return raw, torch.stack(finals, dim=2)
        return raw

    def forward(self, hidden: Tensor, *, combine: str = 'index_add', lockstep: bool = True) -> Tensor:
        """model.py:88-140 with backend='reference'."""
        return self.project_output(hidden, self.bank_reads(hidden, combine=combine, lockstep=lockstep))

    # -- stateful inference restated from inference.py for any head count ---------

    def create_state(self, batch: int, dtype=torch.bfloat16) -> Tensor:
        """inference.py:100-107 and product_routed_update.py:10-21: factors
        added in parameter dtype, then stored in ``dtype``.  [B, J, H, S, v]."""
        initial = (self.initial_row_factor[:, None, :] + self.initial_column_factor[None, :, :])
        initial = initial.to(self.initial_row_factor.dtype).float().to(dtype)
        initial = initial.reshape(self.bank_count, self.num_heads, self.bank_size, self.head_value_width)
        return initial.unsqueeze(0).repeat(batch, 1, 1, 1, 1)

    @torch.no_grad()
    def prefill(self, hidden: Tensor, state: Tensor | None = None, *, state_dtype=None):
        """inference.py:110-158: FP32 recurrence with no interior rounding,
        final state stored in the cache dtype."""
        cache_dtype = state_dtype or (state.dtype if state is not None else torch.bfloat16)
        if state is None:
            work = torch.float32 if self.initial_row_factor.dtype != cache_dtype else cache_dtype
            state = self.create_state(hidden.shape[0], work)
        raw, final = self.bank_reads(hidden, state=state.float(), state_dtype=torch.float32,
                                     return_final=True)
        state = final.to(state.dtype).to(cache_dtype)
        return self.project_output(hidden, raw), state

    @torch.no_grad()
    def step(self, hidden: Tensor, state: Tensor):
        """inference.py:161-194: writes first (state stored after each update),
        then reads of the updated banks combined in increasing bank id with a
        rounding after every add.  ``state`` [B,J,H,S,v] is updated in place."""
        batch = hidden.shape[0]
        q, k, v, g, b, w = self.controllers(hidden)
        ww, wi, rw, ri = self.routes(hidden)
        scale = self.bank_size ** -0.5
        rows = torch.arange(batch)
        heads = []
        for head in range(self.num_heads):
            qh, kh, vh, gh, bh, wh = (x[:, 0, head] for x in (q, k, v, g, b, w))
            for j in range(wi.shape[-1]):
                bank = wi[:, 0, j]
                p = ww[:, 0, j]
                eg = gh.float() * p.float()[:, None] if self.config.routed_decay else gh.float()
                eb = (bh * p[:, None]).to(bh.dtype)
                ew = (wh * p[:, None]).to(wh.dtype)
                cur = state[rows, bank, head].float()
                new = write_update(cur, kh, eg, eb, ew, vh)
                state[rows, bank, head] = new.to(state.dtype)
            values = []
            for j in range(ri.shape[-1]):
                bank = ri[:, 0, j]
                eq = (qh * rw[:, 0, j][:, None]).to(qh.dtype)
                values.append(read_value(state[rows, bank, head].float(), eq, scale).to(vh.dtype))
            ranks = torch.argsort(ri[:, 0], dim=-1, stable=True)
            total = torch.zeros(batch, vh.shape[-1])
            for j in range(ri.shape[-1]):
                pick = torch.stack(values, dim=1)[rows, ranks[:, j]]
                total = (total + pick.float()).to(vh.dtype).float()
            heads.append(total.to(vh.dtype))
        raw = torch.cat(heads, dim=-1).unsqueeze(1)
        return self.project_output(hidden, raw), state


def first_write_positions(indices: Tensor, banks: int, valid: Tensor | None = None) -> Tensor:
    """Per (sequence, bank): the first position that writes the bank, valid
    tokens only, or 2**31 - 1 when none does.  The copy-on-write state of the
    reference's memory study holds exactly the banks whose first write came
    before the measured prefix (APPENDIX.md:511-584)."""
    batch, time, _ = indices.shape
    pos = torch.arange(time).view(1, time, 1).expand_as(indices)
    if valid is not None:
        pos = torch.where(valid[..., None].bool(), pos, torch.full_like(pos, 2**31 - 1))
    first = torch.full((batch, banks), 2**31 - 1, dtype=torch.int64)
    first.scatter_reduce_(1, indices.reshape(batch, -1), pos.reshape(batch, -1), reduce='amin')
    return first.to(torch.int32)


def written_bank_curve(indices: Tensor, banks: int, prefixes, valid: Tensor | None = None) -> Tensor:
    """[B, P] int32: distinct banks written within the first prefixes[i]
    positions of each sequence (valid tokens only)."""
    first = first_write_positions(indices, banks, valid).to(torch.int64)
    ends = torch.as_tensor(prefixes, dtype=torch.int64).view(1, 1, -1)
    return (first[..., None] < ends).sum(1).to(torch.int32)


# ---------------------------------------------------------------------------
# language-model shell (model.py:143-216, _shell.py:10-118)

class OracleRMSNorm(nn.Module):
    """_shell.py:10-35: FP32 x * rsqrt(mean(x^2) + eps) * weight, cast back."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        out = x.float() * torch.rsqrt((x.float() * x.float()).mean(-1, keepdim=True) + self.eps)
        return (out * self.weight.float()).type_as(x)


class OracleFeedForward(nn.Module):
    """_shell.py:37-118: hidden = multiple_of * ceil(int(2 * 4d / 3) / multiple_of),
    w2(silu(w1 x) * w3 x), truncated-normal init with stds d^-1/2 and hidden^-1/2."""

    def __init__(self, dim: int, multiple_of: int):
        super().__init__()
        hidden = int(2 * (4 * dim) / 3)
        hidden = multiple_of * ((hidden + multiple_of - 1) // multiple_of)
        self.dim, self.hidden_dim = dim, hidden
        self.w1 = nn.Linear(dim, hidden, bias=False)
        self.w3 = nn.Linear(dim, hidden, bias=False)
        self.w2 = nn.Linear(hidden, dim, bias=False)

    @torch.no_grad()
    def reset(self):
        s_in, s_out = self.dim ** -0.5, self.hidden_dim ** -0.5
        for w in (self.w1, self.w3):
            nn.init.trunc_normal_(w.weight, mean=0.0, std=s_in, a=-3 * s_in, b=3 * s_in)
        nn.init.trunc_normal_(self.w2.weight, mean=0.0, std=s_out, a=-3 * s_out, b=3 * s_out)

    def forward(self, x: Tensor) -> Tensor:
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class OracleBlock(nn.Module):
    def __init__(self, memory, index: int, seed: int, multiple_of: int):
        super().__init__()
        self.attention = OracleBankedDeltaMemory(memory, layer_id=index, seed=seed)
        self.feed_forward = OracleFeedForward(memory.dim, multiple_of)
        self.attention_norm = OracleRMSNorm(memory.dim, memory.norm_eps)
        self.ffn_norm = OracleRMSNorm(memory.dim, memory.norm_eps)


class OracleLanguageModel(nn.Module):
    """BDMLanguageModel (model.py:179-216): embeddings, pre-norm blocks of
    memory layer + SwiGLU, final RMSNorm, untied head.  Seeds: embeddings and
    head from manual_seed(100000 s + 100) in that order, block i's
    feed-forward from manual_seed(100000 s + 1000 + i), the memory layers from
    their role generators."""

    def __init__(self, memory, *, vocab_size: int, layers: int, multiple_of: int = 256, seed: int = 0):
        super().__init__()
        d = memory.dim
        self.layers = nn.ModuleList([OracleBlock(memory, i, seed, multiple_of) for i in range(layers)])
        self.tok_embeddings = nn.Embedding(vocab_size, d)
        self.norm = OracleRMSNorm(d, memory.norm_eps)
        self.output = nn.Linear(d, vocab_size, bias=False)
        base, std = seed * 100_000, d ** -0.5
        with torch.no_grad(), torch.random.fork_rng(devices=[]):
            torch.manual_seed(base + 100)
            for p in (self.tok_embeddings.weight, self.output.weight):
                nn.init.trunc_normal_(p, mean=0, std=std, a=-3 * std, b=3 * std)
        for i, block in enumerate(self.layers):
            with torch.random.fork_rng(devices=[]):
                torch.manual_seed(base + 1000 + i)
                block.feed_forward.reset()

    def forward(self, tokens: Tensor, target: Tensor | None = None):
        hidden = self.tok_embeddings(tokens)
        for block in self.layers:
            hidden = hidden + block.attention(block.attention_norm(hidden))
            hidden = hidden + block.feed_forward(block.ffn_norm(hidden))
        logits = self.output(self.norm(hidden))
        if target is not None:
            return F.cross_entropy(logits.float().flatten(0, -2), target.flatten())
        return logits

    def prefill(self, tokens: Tensor, caches=None):
        """perf_inference_case.py:26-56: per-block attention.prefill on its own
        cache; logits of the last position."""
        caches = list(caches) if caches is not None else [None] * len(self.layers)
        hidden = self.tok_embeddings(tokens)
        for i, block in enumerate(self.layers):
            out, caches[i] = block.attention.prefill(block.attention_norm(hidden), caches[i])
            hidden = hidden + out
            hidden = hidden + block.feed_forward(block.ffn_norm(hidden))
        return self.output(self.norm(hidden[:, -1:])), caches

    def step(self, tokens: Tensor, caches):
        caches = list(caches)
        hidden = self.tok_embeddings(tokens)
        for i, block in enumerate(self.layers):
            out, caches[i] = block.attention.step(block.attention_norm(hidden), caches[i])
            hidden = hidden + out
            hidden = hidden + block.feed_forward(block.ffn_norm(hidden))
        return self.output(self.norm(hidden)), caches
