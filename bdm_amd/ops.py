"""Torch-facing wrappers of the HIP entry points.

Each wrapper validates shapes and dtypes the way the reference does before a
launch (ValueError for bad shapes/dtypes/devices), allocates outputs and the
workspace with torch on the input's device, and enqueues the kernels on the
current stream without synchronising.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib
from .config import near_square_factors

Tensor = torch.Tensor


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.BDM_BF16
    if dtype == torch.float32:
        return _lib.BDM_F32
    raise ValueError(f'unsupported dtype {dtype}; expected bfloat16 or float32')


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError('the HIP path requires tensors on a ROCm device')
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError('all tensors must be on the same device')
    return device


def _aligned(t: Tensor) -> Tensor:
    """Contiguous, 16-byte aligned view (copies only when needed)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _ptr(t: Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _addr(t: Tensor | None):
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# router

def router_select(projected: Tensor, *, bank_count: int, selected_banks: int) -> tuple[Tensor, Tensor]:
    """Product-key routing of ``projected`` [..., J1+J2] (gdn2_banks.py:74-114).

    Returns ``(weights, indices)``: weights in the score dtype, int64 indices,
    both [..., C] with C = min(B, min(B, J1, J2)^2)."""
    if projected.ndim < 1:
        raise ValueError('projected routes must have a factor dimension')
    j1, j2 = near_square_factors(bank_count)
    if projected.shape[-1] != j1 + j2:
        raise ValueError('projected route width does not match the bank table')
    if not 1 <= selected_banks <= bank_count:
        raise ValueError('selected bank count is outside the bank table')
    _require_gpu(projected)
    row_stride = _row_stride(projected)
    scores = projected if row_stride else _aligned(projected)
    row_stride = row_stride or scores.shape[-1]
    s = min(selected_banks, j1, j2)
    count = min(selected_banks, s * s)
    rows = scores.numel() // scores.shape[-1]
    weights = torch.empty((*scores.shape[:-1], count), device=scores.device, dtype=scores.dtype)
    indices = torch.empty((*scores.shape[:-1], count), device=scores.device, dtype=torch.int64)
    _lib.check(_lib.library().bdm_router_select(
        _ptr(scores), _dtype_code(scores.dtype), rows, row_stride, j1, j2, selected_banks,
        _ptr(weights), _ptr(indices), _stream(scores.device)), 'bdm_router_select')
    return weights, indices


def router_select_pair(first: Tensor, second: Tensor, *, bank_count: int,
                       selected_banks: int) -> tuple[tuple[Tensor, Tensor], tuple[Tensor, Tensor]]:
    """``router_select`` of two score tensors of one shape and dtype (a layer's
    write and read roles) in one launch: ``((w1, i1), (w2, i2))``."""
    if first.shape != second.shape or first.dtype != second.dtype:
        return (router_select(first, bank_count=bank_count, selected_banks=selected_banks),
                router_select(second, bank_count=bank_count, selected_banks=selected_banks))
    if first.ndim < 1:
        raise ValueError('projected routes must have a factor dimension')
    j1, j2 = near_square_factors(bank_count)
    if first.shape[-1] != j1 + j2:
        raise ValueError('projected route width does not match the bank table')
    if not 1 <= selected_banks <= bank_count:
        raise ValueError('selected bank count is outside the bank table')
    _require_gpu(first, second)
    views = []
    for t in (first, second):
        stride = _row_stride(t)
        scores = t if stride else _aligned(t)
        views.append((scores, stride or scores.shape[-1]))
    s = min(selected_banks, j1, j2)
    count = min(selected_banks, s * s)
    lead = first.shape[:-1]
    rows = first.numel() // first.shape[-1]
    device = first.device
    outs = [(torch.empty((*lead, count), device=device, dtype=first.dtype),
             torch.empty((*lead, count), device=device, dtype=torch.int64)) for _ in range(2)]
    _lib.check(_lib.library().bdm_router_select_pair(
        _ptr(views[0][0]), views[0][1], _ptr(views[1][0]), views[1][1], _dtype_code(first.dtype), rows, j1, j2,
        selected_banks, _ptr(outs[0][0]), _ptr(outs[0][1]), _ptr(outs[1][0]), _ptr(outs[1][1]),
        _stream(device)), 'bdm_router_select_pair')
    return outs[0], outs[1]


def _row_stride(t: Tensor) -> int:
    """Row stride of a view whose rows are contiguous and evenly spaced from a
    16-byte aligned start (a column slice of a wider matrix), else 0."""
    if t.ndim < 1 or t.numel() == 0 or t.stride(-1) != 1 or t.data_ptr() % 16:
        return 0
    if t.ndim == 1:
        return t.shape[-1]
    stride = t.stride(-2)
    expect = stride
    for d in range(t.ndim - 2, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            return 0
        expect *= t.shape[d]
    return stride if stride >= t.shape[-1] else 0


# ---------------------------------------------------------------------------
# dispatch

# Route validation on the product path: off by default, because reading the
# status word synchronises the host with the device once per dispatch.
_validate_routes = os.environ.get('BDM_VALIDATE_ROUTES', '0') not in ('', '0')


def set_route_validation(enabled: bool) -> None:
    """When enabled, every ``dispatch_build`` (and so every forward, prefill
    and training call) reads the route flags the dispatch kernels raise and
    raises ValueError for a bank index outside [0, bank_count) or a bank
    selected twice by one token in one role.  Disabled, malformed routes are
    not reported: out-of-range indices are clamped to a valid bank and the
    results are undefined.  ``BDM_VALIDATE_ROUTES=1`` enables it at import."""
    global _validate_routes
    _validate_routes = bool(enabled)


def route_validation() -> bool:
    return _validate_routes


@dataclass
class Dispatch:
    """Packed-event metadata (role_bank_dispatch.py:135-140).  inverse and
    tokens are None where they were not asked for (route_dispatch); the
    recurrence and its backward read order and cu_seqlens only."""
    order: Tensor
    inverse: Tensor | None
    tokens: Tensor | None
    cu_seqlens: Tensor
    status: Tensor  # int32 on device: bdm_route_flags raised while building
    segment_order: Tensor | None = None  # the forward's longest-first order, when the dispatch ranked it

    def check_routes(self) -> None:
        """Synchronise and raise ValueError if the routes were malformed."""
        flags = int(self.status.item())
        if flags & _lib.BDM_ROUTE_OUT_OF_RANGE:
            raise ValueError('bank indices outside [0, bank_count)')
        if flags & _lib.BDM_ROUTE_DUPLICATE:
            raise ValueError('a token selected the same bank twice in one role')


def dispatch_build(write_indices: Tensor, read_indices: Tensor, bank_count: int) -> Dispatch:
    """Stable bucketing of write/read events into (batch, bank) segments."""
    if write_indices.ndim != 3 or read_indices.ndim != 3 or write_indices.shape[:2] != read_indices.shape[:2]:
        raise ValueError('route indices must be [batch, time, selected] with matching batch and time')
    if write_indices.dtype != torch.long or read_indices.dtype != torch.long:
        raise ValueError('bank indices must be int64')
    device = _require_gpu(write_indices, read_indices)
    batch, time, kw = write_indices.shape
    kr = read_indices.shape[-1]
    wi, ri = _aligned(write_indices), _aligned(read_indices)
    events = batch * time * (kw + kr)
    lib = _lib.library()
    order = torch.empty(events, device=device, dtype=torch.int64)
    inverse = torch.empty(events, device=device, dtype=torch.int64)
    tokens = torch.empty(events, device=device, dtype=torch.int64)
    cu = torch.empty(batch * bank_count + 1, device=device, dtype=torch.int64)
    status = torch.empty(1, device=device, dtype=torch.int32)  # cleared and set by the dispatch itself
    ws_bytes = lib.bdm_dispatch_workspace_size_ex(batch, time, bank_count, kw, kr)
    workspace = torch.empty(max(int(ws_bytes), 1), device=device, dtype=torch.uint8)
    _lib.check(lib.bdm_dispatch_build(
        _ptr(wi), _ptr(ri), batch, time, kw, kr, bank_count, _ptr(order), _ptr(inverse), _ptr(tokens), _ptr(cu),
        _ptr(status), _ptr(workspace), ws_bytes, _stream(device)), 'bdm_dispatch_build')
    meta = Dispatch(order, inverse, tokens, cu, status)
    if _validate_routes:
        meta.check_routes()
    return meta


def route_dispatch(write_scores: Tensor, read_scores: Tensor, *, bank_count: int, selected_banks: int,
                   maps: bool = False) -> tuple[tuple[Tensor, Tensor], tuple[Tensor, Tensor], Dispatch]:
    """Both routers and the dispatch of one step in one call
    (bdm_route_dispatch): ``router_select_pair`` of the [batch, time, J1 + J2]
    write and read scores, then ``dispatch_build`` on those routes, with the
    tile counting done by the routing launch and the forward's longest-first
    segment order ranked in the same call.  ``maps``: also build inverse and
    tokens.  Returns
    ``((ww, wi), (rw, ri), dispatch)``."""
    if write_scores.ndim != 3 or write_scores.shape != read_scores.shape or write_scores.dtype != read_scores.dtype:
        raise ValueError('route scores must be two [batch, time, J1 + J2] tensors of one shape and dtype')
    j1, j2 = near_square_factors(bank_count)
    if write_scores.shape[-1] != j1 + j2:
        raise ValueError('projected route width does not match the bank table')
    s = min(selected_banks, j1, j2)
    if not 1 <= selected_banks <= s * s:
        raise ValueError('selected bank count is outside what the product key can select')
    device = _require_gpu(write_scores, read_scores)
    views = []
    for t in (write_scores, read_scores):
        stride = _row_stride(t)
        scores = t if stride else _aligned(t)
        views.append((scores, stride or scores.shape[-1]))
    batch, time = write_scores.shape[:2]
    k = selected_banks
    events = batch * time * 2 * k
    ww, rw = (torch.empty(batch, time, k, device=device, dtype=write_scores.dtype) for _ in range(2))
    wi, ri = (torch.empty(batch, time, k, device=device, dtype=torch.int64) for _ in range(2))
    order = torch.empty(events, device=device, dtype=torch.int64)
    inverse = torch.empty(events, device=device, dtype=torch.int64) if maps else None
    tokens = torch.empty(events, device=device, dtype=torch.int64) if maps else None
    cu = torch.empty(batch * bank_count + 1, device=device, dtype=torch.int64)
    status = torch.empty(1, device=device, dtype=torch.int32)
    seg_order = torch.empty(batch * bank_count, device=device, dtype=torch.int32)
    args = _lib.RouteDispatchArgs()
    args.write_scores, args.write_stride = _ptr(views[0][0]), views[0][1]
    args.read_scores, args.read_stride = _ptr(views[1][0]), views[1][1]
    args.score_dtype = _dtype_code(write_scores.dtype)
    args.batch, args.time = batch, time
    args.factor_first, args.factor_second, args.selected = j1, j2, k
    args.write_weights, args.write_indices = _ptr(ww), _ptr(wi)
    args.read_weights, args.read_indices = _ptr(rw), _ptr(ri)
    args.order, args.cu_seqlens, args.status = _ptr(order), _ptr(cu), _ptr(status)
    args.inverse = _ptr(inverse) if maps else None
    args.tokens = _ptr(tokens) if maps else None
    args.segment_order = _ptr(seg_order)
    lib = _lib.library()
    ws_bytes = lib.bdm_route_dispatch_workspace_size(ctypes.byref(args))
    workspace = torch.empty(max(int(ws_bytes), 1), device=device, dtype=torch.uint8)
    _lib.check(lib.bdm_route_dispatch(ctypes.byref(args), _ptr(workspace), ws_bytes, _stream(device)),
               'bdm_route_dispatch')
    meta = Dispatch(order, inverse, tokens, cu, status, seg_order)
    if _validate_routes:
        meta.check_routes()
    return (ww, wi), (rw, ri), meta


# ---------------------------------------------------------------------------
# forward recurrence + combine

def _as_heads(t: Tensor, name: str) -> Tensor:
    if t.ndim == 3:
        return t.unsqueeze(2)
    if t.ndim == 4:
        return t
    raise ValueError(f'{name} must be [batch, time, width] or [batch, time, heads, width]')


@dataclass
class RoutedInputs:
    """Validated, contiguous, 16-byte aligned operands of the routed recurrence
    with their geometry (shared by the forward and the backward)."""
    q: Tensor
    k: Tensor
    g: Tensor
    b: Tensor
    v: Tensor
    w: Tensor
    ww: Tensor
    rw: Tensor
    ri: Tensor
    initial: Tensor
    initial_stride: int
    batch: int
    time: int
    heads: int
    bank_size: int
    width: int
    write_banks: int
    read_banks: int
    per_head_layout: bool
    dtype: torch.dtype
    device: torch.device


def prepare_routed(q, k, v, g, b, w, wi, ww, ri, rw, initial: Tensor, *, bank_count: int) -> RoutedInputs:
    """Shape/dtype validation of the routed operator's operands
    (role_bank_dispatch.py:156-166 and routed_update.py:18-22 assert the same)."""
    q4, k4, g4, b4 = (_as_heads(t, n) for t, n in ((q, 'q'), (k, 'k'), (g, 'g'), (b, 'b')))
    v4, w4 = _as_heads(v, 'v'), _as_heads(w, 'w')
    if not (q4.shape == k4.shape == g4.shape == b4.shape):
        raise ValueError('q, k, g, and b must share [batch,time,heads,bank_size]')
    if v4.shape != w4.shape or v4.shape[:3] != q4.shape[:3]:
        raise ValueError('v and w must share [batch,time,heads,value_width] with the keys')
    batch, time, heads, s = q4.shape
    width = v4.shape[-1]
    if wi.shape[:2] != (batch, time) or ri.shape[:2] != (batch, time):
        raise ValueError('routes disagree with controller batch or time')
    if wi.shape != ww.shape or ri.shape != rw.shape:
        raise ValueError('route indices and weights must align')
    dtype = q4.dtype
    for t in (k4, b4, v4, w4, ww, rw):
        if t.dtype != dtype:
            raise ValueError('q, k, b, v, w and the route weights must share one dtype')
    device = _require_gpu(q4, k4, g4, b4, v4, w4, wi, ww, ri, rw, initial)
    per_head_layout = q.ndim == 4
    shared_dims = 4 if per_head_layout else 3
    if initial.ndim == shared_dims:
        init_stride = 0
    elif initial.ndim == shared_dims + 1:
        if initial.shape[0] != batch:
            raise ValueError('per-sequence initial state must lead with the batch dimension')
        init_stride = initial[0].numel()
    else:
        raise ValueError('initial state has the wrong rank')
    expect = (bank_count, heads, s, width) if per_head_layout else (bank_count, s, width)
    if tuple(initial.shape[-len(expect):]) != expect:
        raise ValueError(f'initial state must end in {expect}, got {tuple(initial.shape)}')
    if initial.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError('initial state must be FP32 or BF16')
    return RoutedInputs(
        q=_aligned(q4), k=_aligned(k4), g=_aligned(g4.float()), b=_aligned(b4), v=_aligned(v4), w=_aligned(w4),
        ww=_aligned(ww), rw=_aligned(rw), ri=_aligned(ri), initial=_aligned(initial), initial_stride=init_stride,
        batch=batch, time=time, heads=heads, bank_size=s, width=width, write_banks=wi.shape[-1],
        read_banks=ri.shape[-1], per_head_layout=per_head_layout, dtype=dtype, device=device)


def snapshot_buffer(x: RoutedInputs, interval: int, dtype: torch.dtype) -> Tensor:
    """Snapshot storage for a forward with backward: [E // interval, H, S, v]."""
    events = x.batch * x.time * (x.write_banks + x.read_banks)
    rows = int(_lib.library().bdm_snapshot_rows(events, interval))
    return torch.empty((max(rows, 1), x.heads, x.bank_size, x.width), device=x.device, dtype=dtype)


def routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, initial: Tensor, meta: Dispatch, *, bank_count: int,
                   scale: float, routed_decay: bool, round_interval: int = 0,
                   final_state: Tensor | None = None, snapshots: Tensor | None = None,
                   snapshot_interval: int = 0, prepared: RoutedInputs | None = None,
                   phase_events=None, workspace: Tensor | None = None) -> Tensor:
    """Bank recurrence and ordered read combine for every head.

    q,k,g,b: [B,T,S] or [B,T,H,S];  v,w: [B,T,v] or [B,T,H,v];
    initial: [J,S,v] / [J,H,S,v] shared by the batch, or [B,J,S,v] /
    [B,J,H,S,v] per sequence (4-D is read as per-head when q is 4-D);
    final_state: optional [B,J,H,S,v] (or [B,J,S,v]) output, may alias initial;
    snapshots: optional buffer from ``snapshot_buffer`` for the backward;
    phase_events: optional three torch.cuda.Event (timing enabled) recorded on
    the current stream before the recurrence, before the combine and after it;
    workspace: optional uint8 device tensor of at least
    bdm_forward_workspace_size bytes (allocated per call otherwise); its
    contents on entry do not matter.
    Returns y [B, T, H*v] in the controller dtype."""
    x = prepared or prepare_routed(q, k, v, g, b, w, wi, ww, ri, rw, initial, bank_count=bank_count)
    _require_gpu(meta.order, final_state, snapshots)
    if final_state is not None:
        if final_state.numel() != x.batch * bank_count * x.heads * x.bank_size * x.width \
                or not final_state.is_contiguous():
            raise ValueError('final_state must be a contiguous [batch, J, H, S, v] tensor')
        if final_state.data_ptr() % 16:
            raise ValueError('final_state must be 16-byte aligned')
    output = torch.empty((x.batch, x.time, x.heads * x.width), device=x.device, dtype=x.dtype)
    args = _lib.ForwardArgs()
    args.q, args.k, args.g, args.b, args.v, args.w = (t.data_ptr() for t in (x.q, x.k, x.g, x.b, x.v, x.w))
    args.write_weights, args.read_weights, args.read_indices = x.ww.data_ptr(), x.rw.data_ptr(), x.ri.data_ptr()
    args.order, args.cu_seqlens = meta.order.data_ptr(), meta.cu_seqlens.data_ptr()
    args.initial = x.initial.data_ptr()
    args.final_state = final_state.data_ptr() if final_state is not None else None
    args.output = output.data_ptr()
    args.initial_batch_stride = x.initial_stride
    args.batch, args.time = x.batch, x.time
    args.heads, args.bank_size, args.head_width, args.bank_count = x.heads, x.bank_size, x.width, bank_count
    args.write_banks, args.read_banks = x.write_banks, x.read_banks
    args.ctrl_dtype = _dtype_code(x.dtype)
    args.initial_dtype = _dtype_code(x.initial.dtype)
    args.final_dtype = _dtype_code(final_state.dtype) if final_state is not None else 0
    args.routed_decay = int(bool(routed_decay))
    args.round_interval = int(round_interval)
    args.scale = float(scale)
    if snapshots is not None:
        args.snapshots = snapshots.data_ptr()
        args.snapshot_interval = int(snapshot_interval)
        args.snapshot_dtype = _dtype_code(snapshots.dtype)
    if meta.segment_order is not None:
        if meta.segment_order.numel() != x.batch * bank_count:
            raise ValueError('the dispatch was built for another geometry')
        args.segment_order = meta.segment_order.data_ptr()
    if phase_events is not None:
        for i, ev in enumerate(phase_events):
            if ev.cuda_event == 0:  # torch creates the HIP event on first use
                ev.record()
            args.phase_events[i] = ev.cuda_event
    lib = _lib.library()
    ws_bytes = lib.bdm_forward_workspace_size(ctypes.byref(args))
    if workspace is None:
        workspace = torch.empty(max(int(ws_bytes), 1), device=x.device, dtype=torch.uint8)
    elif workspace.dtype != torch.uint8 or workspace.device != x.device or workspace.numel() < ws_bytes \
            or not workspace.is_contiguous():
        raise ValueError(f'workspace must be a contiguous uint8 tensor of at least {ws_bytes} bytes on {x.device}')
    _lib.check(lib.bdm_forward(ctypes.byref(args), _ptr(workspace), ws_bytes, _stream(x.device)), 'bdm_forward')
    return output


@dataclass
class RoutedGrads:
    q: Tensor
    k: Tensor
    v: Tensor
    g: Tensor
    b: Tensor
    w: Tensor
    ww: Tensor
    rw: Tensor
    initial: Tensor  # FP32 [B, J, H, S, v] adjoint of each sequence's initial state


def routed_backward(x: RoutedInputs, meta: Dispatch, grad_output: Tensor, snapshots: Tensor, *, bank_count: int,
                    scale: float, routed_decay: bool, round_interval: int, snapshot_interval: int) -> RoutedGrads:
    """Gradients of ``routed_forward`` (RoutedUpdate.backward, routed_update.py:31-49)."""
    if grad_output.shape != (x.batch, x.time, x.heads * x.width):
        grad_output = grad_output.reshape(x.batch, x.time, x.heads * x.width)
    dy = _aligned(grad_output.to(x.dtype))
    ctrl = (x.batch, x.time, x.heads, x.bank_size)
    vals = (x.batch, x.time, x.heads, x.width)
    empty = lambda shape, dtype=x.dtype: torch.empty(shape, device=x.device, dtype=dtype)  # noqa: E731
    out = RoutedGrads(q=empty(ctrl), k=empty(ctrl), v=empty(vals), g=empty(ctrl, torch.float32), b=empty(ctrl),
                      w=empty(vals), ww=empty(x.ww.shape), rw=empty(x.rw.shape),
                      initial=empty((x.batch, bank_count, x.heads, x.bank_size, x.width), torch.float32))
    args = _lib.BackwardArgs()
    args.q, args.k, args.g, args.b, args.v, args.w = (t.data_ptr() for t in (x.q, x.k, x.g, x.b, x.v, x.w))
    args.write_weights, args.read_weights = x.ww.data_ptr(), x.rw.data_ptr()
    args.order, args.cu_seqlens = meta.order.data_ptr(), meta.cu_seqlens.data_ptr()
    args.initial, args.snapshots, args.grad_output = x.initial.data_ptr(), snapshots.data_ptr(), dy.data_ptr()
    args.grad_q, args.grad_k, args.grad_g = out.q.data_ptr(), out.k.data_ptr(), out.g.data_ptr()
    args.grad_b, args.grad_v, args.grad_w = out.b.data_ptr(), out.v.data_ptr(), out.w.data_ptr()
    args.grad_write_weights, args.grad_read_weights = out.ww.data_ptr(), out.rw.data_ptr()
    args.grad_initial = out.initial.data_ptr()
    args.initial_batch_stride = x.initial_stride
    args.batch, args.time = x.batch, x.time
    args.heads, args.bank_size, args.head_width, args.bank_count = x.heads, x.bank_size, x.width, bank_count
    args.write_banks, args.read_banks = x.write_banks, x.read_banks
    args.ctrl_dtype = _dtype_code(x.dtype)
    args.initial_dtype = _dtype_code(x.initial.dtype)
    args.snapshot_dtype = _dtype_code(snapshots.dtype)
    args.routed_decay = int(bool(routed_decay))
    args.round_interval = int(round_interval)
    args.snapshot_interval = int(snapshot_interval)
    args.scale = float(scale)
    lib = _lib.library()
    ws_bytes = lib.bdm_backward_workspace_size(ctypes.byref(args))
    workspace = torch.empty(max(int(ws_bytes), 1), device=x.device, dtype=torch.uint8)
    _lib.check(lib.bdm_backward(ctypes.byref(args), _ptr(workspace), ws_bytes, _stream(x.device)), 'bdm_backward')
    return out


# ---------------------------------------------------------------------------
# decode

def decode_step(q, k, v, g, b, w, wi, ww, ri, rw, state: Tensor, *, bank_count: int, scale: float,
                routed_decay: bool) -> Tensor:
    """One token per sequence against ``state`` [B,J,H,S,v] (updated in place).

    q,k,g,b: [B,H,S]; v,w: [B,H,v]; wi,ww: [B,KW]; ri,rw: [B,KR].
    Returns y [B, H*v]."""
    if q.ndim != 3 or v.ndim != 3:
        raise ValueError('decode controllers must be [batch, heads, width]')
    batch, heads, s = q.shape
    width = v.shape[-1]
    if state.shape != (batch, bank_count, heads, s, width) or not state.is_contiguous():
        raise ValueError('state must be a contiguous [batch, banks, heads, bank_size, head_width] tensor')
    if state.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError('state must be FP32 or BF16')
    device = _require_gpu(q, k, v, g, b, w, wi, ww, ri, rw, state)
    dtype = q.dtype
    qc, kc, bc, vc, wc = (_aligned(t) for t in (q, k, b, v, w))
    gc = _aligned(g.float())
    wwc, rwc, wic, ric = (_aligned(t) for t in (ww, rw, wi, ri))
    output = torch.empty((batch, heads * width), device=device, dtype=dtype)
    args = _lib.DecodeArgs()
    args.q, args.k, args.b, args.g, args.v, args.w = (t.data_ptr() for t in (qc, kc, bc, gc, vc, wc))
    args.write_weights, args.read_weights = wwc.data_ptr(), rwc.data_ptr()
    args.write_indices, args.read_indices = wic.data_ptr(), ric.data_ptr()
    args.state, args.output = state.data_ptr(), output.data_ptr()
    args.batch = batch
    args.heads, args.bank_size, args.head_width, args.bank_count = heads, s, width, bank_count
    args.write_banks, args.read_banks = wi.shape[-1], ri.shape[-1]
    args.ctrl_dtype = _dtype_code(dtype)
    args.state_dtype = _dtype_code(state.dtype)
    args.routed_decay = int(bool(routed_decay))
    args.scale = float(scale)
    _lib.check(_lib.library().bdm_decode(ctypes.byref(args), _stream(device)), 'bdm_decode')
    return output


def _decode_fused_args(proj, f, columns, a_log, dt_bias, state, heads, bank_size, head_width, bank_count,
                       selected_banks, qk_norm, routed_decay, scale, f_weight=None):
    j1, j2 = near_square_factors(bank_count)
    args = _lib.DecodeFusedArgs()
    args.batch, args.proj_stride = proj.shape[0], proj.stride(0)
    args.f_stride = f.stride(0) if f is not None else 0
    if f_weight is not None:
        args.f_col, args.f_width = columns['f'], f_weight.shape[1]
    args.q_col, args.k_col, args.v_col = columns['q'], columns['k'], columns['v']
    args.b_col, args.w_col, args.read_col, args.write_col = columns['b'], columns['w'], columns['read'], columns['write']
    args.heads, args.bank_size, args.head_width = heads, bank_size, head_width
    args.factor_first, args.factor_second, args.selected_banks = j1, j2, selected_banks
    args.ctrl_dtype, args.param_dtype = _dtype_code(proj.dtype), _dtype_code(a_log.dtype)
    args.state_dtype = _dtype_code(state.dtype)
    args.qk_norm = 1 if qk_norm == 'nvidia' else 0
    args.routed_decay = int(bool(routed_decay))
    args.scale = float(scale)
    return args


def _f_weight_ok(proj, f_weight, heads, bank_size):
    return (f_weight.dtype == proj.dtype and f_weight.ndim == 2 and f_weight.is_contiguous()
            and f_weight.shape[0] == heads * bank_size and f_weight.data_ptr() % 16 == 0)


def decode_fused_supported(proj: Tensor, f: Tensor | None, columns: dict, a_log: Tensor, dt_bias: Tensor,
                           state: Tensor, *, heads: int, bank_size: int, head_width: int, bank_count: int,
                           selected_banks: int, f_weight: Tensor | None = None) -> bool:
    """Whether ``decode_fused`` takes this geometry (BF16 controllers, S = 8,
    8 banks per role from J1, J2 <= 64, aligned slices, spans of 48..128, of
    64..128 when f is formed in the launch from ``f_weight``)."""
    if not (proj.is_cuda and proj.ndim == 2 and proj.stride(-1) == 1 and proj.dtype == torch.bfloat16):
        return False
    if f_weight is None:
        if f is None or f.ndim != 2 or f.stride(-1) != 1 or f.dtype != proj.dtype or f.data_ptr() % 16:
            return False
    elif not _f_weight_ok(proj, f_weight, heads, bank_size):
        return False
    if a_log.dtype != dt_bias.dtype or a_log.dtype not in (torch.bfloat16, torch.float32):
        return False
    if state.dtype not in (torch.bfloat16, torch.float32):
        return False
    if any(t.data_ptr() % 16 for t in (proj, state)) or not state.is_contiguous():
        return False
    args = _decode_fused_args(proj, f if f_weight is None else None, columns, a_log, dt_bias, state, heads, bank_size,
                              head_width, bank_count, selected_banks, 'nvidia', True, 1.0, f_weight)
    args.f_weight = f_weight.data_ptr() if f_weight is not None else None
    return bool(_lib.library().bdm_decode_fused_supported(ctypes.byref(args)))


def decode_fused(proj: Tensor, f: Tensor | None, columns: dict, a_log: Tensor, dt_bias: Tensor, state: Tensor, *,
                 heads: int, bank_size: int, head_width: int, bank_count: int, selected_banks: int, qk_norm: str,
                 routed_decay: bool, scale: float, f_weight: Tensor | None = None,
                 f_out: Tensor | None = None) -> Tensor:
    """One decode step from the projection outputs in one launch: the
    controller epilogue (``controller_epilogue``), both routes
    (``router_select_pair``) and ``decode_step``, with identical results.

    proj: [B, P] the fused projection row of each sequence's token (q, k, v,
    b, w and the read/write route scores at ``columns``); f: [B, H*S] the
    f_proj output; state: [B, J, H, S, v], updated in place.  Returns y
    [B, H*v].

    With ``f_weight`` (f_proj's second factor, [H*S, F]) f is formed in the
    launch from proj's f_proj first-factor slice at ``columns['f']`` (F
    columns) and ``f`` is ignored: FP32 dot products in a fixed order, rounded
    to the projection dtype.  ``f_out`` [B, H*S], when given, receives it."""
    _require_gpu(proj, a_log, dt_bias, state)
    batch = proj.shape[0]
    if state.shape != (batch, bank_count, heads, bank_size, head_width) or not state.is_contiguous():
        raise ValueError('state must be a contiguous [batch, banks, heads, bank_size, head_width] tensor')
    if f_weight is not None:
        _require_gpu(f_weight)
        if not _f_weight_ok(proj, f_weight, heads, bank_size):
            raise ValueError('f_weight must be a contiguous, 16-byte aligned [heads*bank_size, F] matrix of '
                             'the projection dtype')
        f = None
        if f_out is not None and (f_out.shape != (batch, heads * bank_size) or f_out.dtype != proj.dtype
                                  or not f_out.is_contiguous()):
            raise ValueError('f_out must be a contiguous [batch, heads*bank_size] tensor of the projection dtype')
    elif f is None:
        raise ValueError('decode_fused needs f or f_weight')
    else:
        _require_gpu(f)
    a_log, dt_bias = _aligned(a_log.contiguous()), _aligned(dt_bias.contiguous())
    output = torch.empty((batch, heads * head_width), device=proj.device, dtype=proj.dtype)
    args = _decode_fused_args(proj, f, columns, a_log, dt_bias, state, heads, bank_size, head_width, bank_count,
                              selected_banks, qk_norm, routed_decay, scale, f_weight)
    args.proj, args.a_log, args.dt_bias = (t.data_ptr() for t in (proj, a_log, dt_bias))
    args.f = f.data_ptr() if f is not None else None
    args.f_weight = f_weight.data_ptr() if f_weight is not None else None
    args.f_out = f_out.data_ptr() if (f_weight is not None and f_out is not None) else None
    args.state, args.output = state.data_ptr(), output.data_ptr()
    _lib.check(_lib.library().bdm_decode_fused(ctypes.byref(args), _stream(proj.device)), 'bdm_decode_fused')
    return output


# ---------------------------------------------------------------------------
# inference epilogues (the controller activations and the output interface)

def controller_epilogue(proj: Tensor, f: Tensor, columns: dict, a_log: Tensor, dt_bias: Tensor, *, heads: int,
                        bank_size: int, head_width: int, qk_norm: str):
    """Controllers of heads.controllers (heads.py:11-22) from one projection
    matrix ``proj`` [N, P] (the q, k, v, b, w slices at ``columns``) and the
    f_proj output ``f`` [N, H*S]: returns q, k, b [N, H, S], v, w [N, H, v]
    in the projection dtype and g [N, H, S] FP32."""
    _require_gpu(proj, f, a_log, dt_bias)
    if proj.ndim != 2 or proj.stride(-1) != 1 or f.ndim != 2 or f.stride(-1) != 1:
        raise ValueError('proj and f must be row-major matrices')
    if a_log.dtype != dt_bias.dtype:
        raise ValueError('A_log and dt_bias must share a dtype')
    n = proj.shape[0]
    dev, dt = proj.device, proj.dtype
    q = torch.empty(n, heads, bank_size, device=dev, dtype=dt)
    k, b = torch.empty_like(q), torch.empty_like(q)
    g = torch.empty(n, heads, bank_size, device=dev, dtype=torch.float32)
    v = torch.empty(n, heads, head_width, device=dev, dtype=dt)
    w = torch.empty_like(v)
    a_log, dt_bias = a_log.contiguous(), dt_bias.contiguous()  # kept alive until the launch is enqueued
    args = _lib.ControllerArgs()
    args.proj, args.f, args.a_log, args.dt_bias = (t.data_ptr() for t in (proj, f, a_log, dt_bias))
    args.q, args.k, args.v, args.b, args.w, args.g = (t.data_ptr() for t in (q, k, v, b, w, g))
    args.tokens, args.proj_stride, args.f_stride = n, proj.stride(0), f.stride(0)
    args.q_col, args.k_col, args.v_col = columns['q'], columns['k'], columns['v']
    args.b_col, args.w_col = columns['b'], columns['w']
    args.heads, args.bank_size, args.head_width = heads, bank_size, head_width
    args.ctrl_dtype, args.param_dtype = _dtype_code(dt), _dtype_code(a_log.dtype)
    args.qk_norm = 1 if qk_norm == 'nvidia' else 0
    _lib.check(_lib.library().bdm_controller_epilogue(ctypes.byref(args), _stream(dev)), 'bdm_controller_epilogue')
    return q, k, v, g, b, w


def output_epilogue(raw: Tensor, gate: Tensor, weight: Tensor, bias: Tensor | None, *, eps: float,
                    kind: str) -> Tensor:
    """norm(raw) * sigmoid(gate) of _project_bank_output (_parameters.py:222-232),
    before o_proj: ``kind`` 'layer' (LayerNorm with weight, bias) or 'rms'."""
    _require_gpu(raw, gate, weight, bias)
    if raw.ndim != 2 or gate.ndim != 2 or gate.stride(-1) != 1 or gate.shape != raw.shape:
        raise ValueError('raw and gate must be [tokens, width] with contiguous rows')
    raw, weight = raw.contiguous(), weight.contiguous()
    bias = None if bias is None else bias.contiguous()
    out = torch.empty_like(raw)
    args = _lib.OutputArgs()
    args.raw, args.gate, args.out = raw.data_ptr(), gate.data_ptr(), out.data_ptr()
    args.norm_weight = weight.data_ptr()
    args.norm_bias = None if bias is None else bias.data_ptr()
    args.tokens, args.gate_stride, args.width = raw.shape[0], gate.stride(0), raw.shape[1]
    args.ctrl_dtype, args.param_dtype = _dtype_code(raw.dtype), _dtype_code(weight.dtype)
    args.norm_kind = 1 if kind == 'layer' else 0
    args.eps = float(eps)
    _lib.check(_lib.library().bdm_output_epilogue(ctypes.byref(args), _stream(raw.device)), 'bdm_output_epilogue')
    return out


# ---------------------------------------------------------------------------
# skinny linear maps (decode)

GEMV_MAX_ROWS = 4            # the streaming GEMV and its prologues
SKINNY_MAX_ROWS = 64         # the matrix-core tiles (BF16, no prologue)
GEMV_PROLOGUE_MAX_K = 6144


def gemv_supported(x: Tensor, weight: Tensor, bias: Tensor | None) -> bool:
    rows = x.numel() // max(x.shape[-1], 1)
    k = x.shape[-1]
    common = (x.is_cuda and weight.dtype == x.dtype and weight.ndim == 2 and weight.is_contiguous()
              and k == weight.shape[1] and weight.data_ptr() % 16 == 0
              and (bias is None or (bias.dtype == x.dtype and bias.shape == (weight.shape[0],))))
    if 1 <= rows <= GEMV_MAX_ROWS:
        return common and x.dtype in (torch.bfloat16, torch.float32) and k % 8 == 0
    return (common and rows <= SKINNY_MAX_ROWS and x.dtype == torch.bfloat16 and k % 32 == 0
            and weight.shape[0] < 2 ** 31)


def gemv(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """F.linear(x, weight, bias) for the rows of a decode step: 1 to 4 rows
    stream the weight once at HBM bandwidth, 5 to 64 BF16 rows run as
    matrix-core tiles (K % 32 == 0); FP32 accumulation, one rounding."""
    _require_gpu(x, weight, bias)
    if not gemv_supported(x, weight, bias):
        raise ValueError('gemv takes 1-4 BF16/FP32 rows (K % 8 == 0) or 5-64 BF16 rows (K % 32 == 0) and a '
                         'contiguous aligned [N, K] weight')
    lead, k = x.shape[:-1], x.shape[-1]
    rows, n = x.numel() // k, weight.shape[0]
    x2 = _aligned(x.reshape(rows, k))
    b = None if bias is None else bias.contiguous()
    y = torch.empty(rows, n, device=x.device, dtype=x.dtype)
    _lib.check(_lib.library().bdm_gemv(_ptr(x2), _ptr(weight), _ptr(b), _ptr(y), rows, n, k,
                                       _dtype_code(x.dtype), _stream(x.device)), 'bdm_gemv')
    return y.view(*lead, n)


_PROLOGUES = {'rms': _lib.GEMV_RMS, 'swiglu': _lib.GEMV_SWIGLU, 'out_layer': _lib.GEMV_OUT_LAYER,
              'out_rms': _lib.GEMV_OUT_RMS}


def gemv_fused(x: Tensor, weight: Tensor, bias: Tensor | None = None, *, prologue: str,
               residual: Tensor | None = None, norm_weight: Tensor | None = None, norm_bias: Tensor | None = None,
               gate: Tensor | None = None, eps: float = 1e-5):
    """F.linear of 1-4 rows whose input is formed inside the GEMV, bit-identical
    to running the elementwise kernel first:
      'rms'       RMSNorm(x [+ residual]) * norm_weight; with ``residual``
                  returns (y, x + residual rounded) -- the block's new hidden;
      'swiglu'    silu(a) * b of x = [rows, 2K] (a | b);
      'out_layer' / 'out_rms'  the layer's output interface: norm(x) * sigmoid(gate)."""
    _require_gpu(x, weight, bias, residual, norm_weight, norm_bias, gate)
    kind = _PROLOGUES[prologue]
    k = weight.shape[1]
    rows = x.numel() // x.shape[-1]
    if not (1 <= rows <= GEMV_MAX_ROWS) or x.dtype not in (torch.bfloat16, torch.float32) or weight.dtype != x.dtype:
        raise ValueError('gemv_fused takes 1-4 BF16/FP32 rows of the weight dtype')
    if x.shape[-1] != (2 * k if prologue == 'swiglu' else k) or k % 8 or k > GEMV_PROLOGUE_MAX_K:
        raise ValueError('x does not match the weight (K % 8 == 0, K <= 6144; 2K columns for swiglu)')
    x2 = _aligned(x.reshape(rows, x.shape[-1]))
    res = None if residual is None else _aligned(residual.reshape(rows, k))
    total = None if res is None else torch.empty_like(res)
    g = None
    if gate is not None:
        g = gate.reshape(rows, -1) if gate.stride(-1) == 1 else gate.reshape(rows, -1).contiguous()
        if g.data_ptr() % 16 or g.stride(0) % 8:
            g = g.contiguous().clone()
    nw = None if norm_weight is None else _aligned(norm_weight)
    nb = None if norm_bias is None else _aligned(norm_bias)
    b = None if bias is None else bias.contiguous()
    y = torch.empty(rows, weight.shape[0], device=x.device, dtype=x.dtype)
    args = _lib.GemvArgs()
    args.x, args.weight, args.bias, args.y = _addr(x2), _addr(weight), _addr(b), _addr(y)
    args.residual, args.sum_out, args.norm_weight, args.norm_bias, args.gate = (
        _addr(res), _addr(total), _addr(nw), _addr(nb), _addr(g))
    args.rows, args.n, args.k = rows, weight.shape[0], k
    args.gate_stride = 0 if g is None else g.stride(0)
    args.dtype = _dtype_code(x.dtype)
    args.param_dtype = _dtype_code(nw.dtype) if nw is not None else _lib.BDM_F32
    args.prologue, args.eps = kind, float(eps)
    _lib.check(_lib.library().bdm_gemv_ex(ctypes.byref(args), _stream(x.device)), 'bdm_gemv_ex')
    y = y.view(*x.shape[:-1], weight.shape[0])
    if total is not None:
        return y, total.view(residual.shape)
    return y


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """Inference F.linear: the HBM-streaming GEMV (1-4 rows) or the
    matrix-core tiles (5-64 BF16 rows) for a decode step, the library GEMM
    otherwise (and under autograd)."""
    if not torch.is_grad_enabled() and gemv_supported(x, weight, bias):
        return gemv(x, weight, bias)
    return F.linear(x, weight, bias)


# ---------------------------------------------------------------------------
# language-model shell

def rms_norm_supported(x: Tensor) -> bool:
    return x.is_cuda and x.dtype in (torch.bfloat16, torch.float32) and x.shape[-1] % 8 == 0 and x.shape[-1] <= 8192


def rms_norm(x: Tensor, weight: Tensor, eps: float, residual: Tensor | None = None):
    """RMSNorm of the shell (_shell.py:29-35) in one pass: FP32 arithmetic,
    one rounding.  With ``residual``, returns (x + residual rounded, its norm),
    the block's residual add fused in; otherwise the norm of x."""
    _require_gpu(x, weight, residual)
    if not rms_norm_supported(x):
        raise ValueError('rms_norm takes BF16/FP32 rows whose width is a multiple of 8, at most 8192')
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype):
        raise ValueError('residual must match x')
    if weight.shape != (x.shape[-1],):
        raise ValueError('weight must be [width]')
    x, weight = _aligned(x), _aligned(weight)
    res = None if residual is None else _aligned(residual)
    out = torch.empty_like(x)
    total = None if res is None else torch.empty_like(x)
    width = x.shape[-1]
    _lib.check(_lib.library().bdm_rms_norm(
        _ptr(x), _ptr(res), _ptr(weight), _ptr(total), _ptr(out), x.numel() // width, width, _dtype_code(x.dtype),
        _dtype_code(weight.dtype), float(eps), _stream(x.device)), 'bdm_rms_norm')
    return out if res is None else (total, out)


def rms_norm_backward(x: Tensor, grad_out: Tensor, weight: Tensor, eps: float):
    """Gradients (grad_x, grad_weight) of ``rms_norm(x, weight, eps)``: the
    derivative of the shell's FP32 RMSNorm (_shell.py:29-35), one pass over
    the rows and a column sum for the weight.  width <= 4096."""
    _require_gpu(x, grad_out, weight)
    width = x.shape[-1]
    if not rms_norm_supported(x) or width > 4096:
        raise ValueError('rms_norm_backward takes BF16/FP32 rows whose width is a multiple of 8, at most 4096')
    if grad_out.shape != x.shape or grad_out.dtype != x.dtype or weight.shape != (width,):
        raise ValueError('grad_out must match x and weight must be [width]')
    x, grad_out, weight = _aligned(x), _aligned(grad_out), _aligned(weight)
    rows = x.numel() // width
    lib = _lib.library()
    partials = torch.empty(max(int(lib.bdm_rms_norm_backward_partials(rows)), 1) * width, device=x.device,
                           dtype=torch.float32)
    grad_x = torch.empty_like(x)
    grad_weight = torch.empty_like(weight)
    _lib.check(lib.bdm_rms_norm_backward(
        _ptr(x), _ptr(grad_out), _ptr(weight), _ptr(grad_x), _ptr(grad_weight), _ptr(partials), rows, width,
        _dtype_code(x.dtype), _dtype_code(weight.dtype), float(eps), _stream(x.device)), 'bdm_rms_norm_backward')
    return grad_x, grad_weight


def swiglu_pair(a: Tensor, b: Tensor) -> Tensor:
    """round(round(silu(a)) * b) elementwise (the shell's SwiGLU with its two
    inputs from separate GEMMs, _shell.py:86-91)."""
    _require_gpu(a, b)
    if a.shape != b.shape or a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError('swiglu_pair takes two BF16/FP32 tensors of one shape')
    a, b = a.contiguous(), b.contiguous()
    out = torch.empty_like(a)
    _lib.check(_lib.library().bdm_swiglu_pair(_ptr(a), _ptr(b), _ptr(out), a.numel(), _dtype_code(a.dtype),
                                               _stream(a.device)), 'bdm_swiglu_pair')
    return out


def swiglu_backward(a: Tensor, b: Tensor, grad_out: Tensor):
    """(grad_a, grad_b) of ``swiglu_pair(a, b)`` as autograd forms them for
    F.silu(a) * b."""
    _require_gpu(a, b, grad_out)
    if not (a.shape == b.shape == grad_out.shape) or not (a.dtype == b.dtype == grad_out.dtype):
        raise ValueError('swiglu_backward takes three tensors of one shape and dtype')
    a, b, grad_out = a.contiguous(), b.contiguous(), grad_out.contiguous()
    grad_a, grad_b = torch.empty_like(a), torch.empty_like(b)
    _lib.check(_lib.library().bdm_swiglu_backward(_ptr(a), _ptr(b), _ptr(grad_out), _ptr(grad_a), _ptr(grad_b),
                                                   a.numel(), _dtype_code(a.dtype), _stream(a.device)),
               'bdm_swiglu_backward')
    return grad_a, grad_b


def swiglu(gate_up: Tensor, hidden: int) -> Tensor:
    """silu(x1) * x3 of the shell's feed-forward (_shell.py:86-91) from the
    output [..., 2*hidden] of one GEMM with the concatenated w1 | w3 weights."""
    _require_gpu(gate_up)
    if gate_up.shape[-1] != 2 * hidden or hidden % 8:
        raise ValueError('gate_up must be [..., 2*hidden] with hidden a multiple of 8')
    gate_up = _aligned(gate_up)
    out = torch.empty(*gate_up.shape[:-1], hidden, device=gate_up.device, dtype=gate_up.dtype)
    _lib.check(_lib.library().bdm_swiglu(_ptr(gate_up), _ptr(out), gate_up.numel() // (2 * hidden), hidden,
                                         _dtype_code(gate_up.dtype), _stream(gate_up.device)), 'bdm_swiglu')
    return out


# ---------------------------------------------------------------------------
# bank occupancy

def bank_occupancy_totals(weights: Tensor, indices: Tensor, bank_count: int, valid: Tensor | None = None,
                          first_write: bool = False):
    """Per (sequence, bank): the sum of log1p(-clamp(p, 0, 1-1e-6)) over its
    writes (FP32) and their number, over the segments of a write-only dispatch
    (elastic_bank_regularizer.py:10-25).  weights [B, T, K], int64 indices
    [B, T, K] or None (totals are then 0), valid [B, T] or None.  Returns
    (totals [B, J], counts [B, J]), and with ``first_write`` also the first
    written position of each bank ([B, J] int32, 2**31 - 1 when the bank is
    never written)."""
    if indices.ndim != 3 or indices.dtype != torch.long or (weights is not None and weights.shape != indices.shape):
        raise ValueError('weights and int64 indices must both be [batch, time, selected]')
    device = _require_gpu(weights, indices, valid)
    batch, time, k = indices.shape
    meta = dispatch_build(indices, indices[..., :0], bank_count)
    w = None if weights is None else _aligned(weights)
    mask = None if valid is None else valid.reshape(batch * time).to(torch.uint8).contiguous()
    totals = torch.empty(batch, bank_count, device=device, dtype=torch.float32)
    counts = torch.empty(batch, bank_count, device=device, dtype=torch.int32)
    first = torch.empty(batch, bank_count, device=device, dtype=torch.int32) if first_write else None
    _lib.check(_lib.library().bdm_bank_occupancy(
        _ptr(w), _lib.BDM_BF16 if w is None else _dtype_code(w.dtype), _ptr(mask), _ptr(meta.order), _ptr(meta.cu_seqlens), batch, time, k,
        bank_count, _ptr(totals), _ptr(counts), _ptr(first), _stream(device)), 'bdm_bank_occupancy')
    if first_write:
        return totals, counts, first
    return totals, counts


def written_bank_curve(first_write: Tensor, prefixes) -> Tensor:
    """Banks written before each prefix end, per sequence: [B, len(prefixes)]
    int32 from the first-write positions [B, J] of ``bank_occupancy_totals``."""
    if first_write.ndim != 2 or first_write.dtype != torch.int32:
        raise ValueError('first_write must be [batch, banks] int32')
    device = _require_gpu(first_write)
    ends = torch.as_tensor(prefixes, dtype=torch.long).reshape(-1).to(device).contiguous()
    if ends.numel() == 0:
        raise ValueError('at least one prefix is needed')
    if int(ends.numel()) > 2**31 - 1:
        raise ValueError('too many prefixes')
    batch, banks = first_write.shape
    first = first_write.contiguous()
    written = torch.empty(batch, ends.numel(), device=device, dtype=torch.int32)
    _lib.check(_lib.library().bdm_written_bank_curve(
        _ptr(first), batch, banks, _ptr(ends), ends.numel(), _ptr(written), _stream(device)),
        'bdm_written_bank_curve')
    return written
