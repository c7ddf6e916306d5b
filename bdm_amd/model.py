"""The BDM layer module on the HIP path.

``BankedDeltaMemory`` keeps the reference module's constructor, parameter
names/shapes, seeded initialisation and ``forward``/``prefill``/``step``
methods (implementation/bdm/model.py:15-140, _parameters.py, heads.py,
inference.py) so state dicts and call sites interchange.  The routed-memory
path (router selection, dispatch, recurrence, combine, decode) runs in
``libbdm_hip.so``; the controller and output projections stay torch GEMMs.

``backend`` accepts ``'hip'`` and, as an alias so that reference call sites
keep working, ``'role'`` (the reference's GPU backend name).
"""

from __future__ import annotations

import hashlib
import math

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .config import BDMConfig, near_square_factors
from .routed_update import _round_interval, bank_training, role_bank_training
from .routing import SharedResidualRouter, product_key_route

Tensor = torch.Tensor


class BankedDeltaMemory(nn.Module):
    """Shared-residual product routing around dense GDN2 memory banks."""

    # Inference steps run the controller epilogue, both routes and the decode
    # kernel as one launch (``ops.decode_fused``) where the geometry allows;
    # False keeps the three separate kernels.  The fused launch also forms
    # f_proj's second factor, in another FP32 summation order than the GEMM,
    # so f may differ by one BF16 rounding and y and the cache match the
    # separate kernels within tolerance rather than bit for bit.
    fused_decode = True

    def __init__(self, config: BDMConfig, *, layer_id=0, seed=0, backend='hip', compact_replay=None):
        super().__init__()
        if backend not in ('hip', 'role'):
            raise ValueError("backend must be hip (or its alias role); the CPU equation oracle lives in oracle/")
        if min(seed, layer_id) < 0:
            raise ValueError(f'seed and layer_id must be >= 0, got seed={seed}, layer_id={layer_id}')
        if not (compact_replay is None or isinstance(compact_replay, bool)):
            raise ValueError(f'compact_replay takes None or a bool, not {compact_replay!r}')
        self.compact_replay = compact_replay
        self.config, self.backend = config, 'hip'
        self.hidden_size, self.bank_count, self.bank_size = config.dim, config.bank_count, config.bank_size
        self.value_width, self.kernel_key_width = config.value_width, config.bank_size
        self.num_heads = config.num_heads
        self.head_value_width = config.head_value_width
        key_width = config.num_heads * config.bank_size
        self.num_reads = self.num_writes = config.selected_banks
        self.layer_id, self.initialization_seed = layer_id, seed * 100_000 + 6000 + layer_id
        self.norm_eps = config.norm_eps
        self.shared_residual_router = True
        self.initial_state_mode = 'product_key'
        self.routing_mode = 'product_topk'
        route_width = sum(near_square_factors(config.bank_count))
        self.factor_route_width = self.route_projection_width = route_width
        self.q_proj = nn.Linear(config.dim, key_width, bias=False)
        self.k_proj = nn.Linear(config.dim, key_width, bias=False)
        self.v_proj = nn.Linear(config.dim, config.value_width, bias=False)
        self.shared_router = SharedResidualRouter(config.dim, route_width)
        self.read_route_proj = self.write_route_proj = None
        self.f_proj = nn.Sequential(nn.Linear(config.dim, config.head_value_width, bias=False),
                                    nn.Linear(config.head_value_width, key_width, bias=False))
        self.b_proj = nn.Linear(config.dim, key_width, bias=False)
        self.w_proj = nn.Linear(config.dim, config.value_width, bias=False)
        self.A_log = nn.Parameter(torch.empty(config.num_heads, dtype=torch.float32))
        self.dt_bias = nn.Parameter(torch.empty(key_width, dtype=torch.float32))
        self.A_log._no_weight_decay = self.dt_bias._no_weight_decay = True
        rows, columns = near_square_factors(config.logical_rows)
        self.register_parameter('initial_state', None)
        self.initial_row_factor = nn.Parameter(torch.zeros(rows, config.head_value_width))
        self.initial_column_factor = nn.Parameter(torch.zeros(columns, config.head_value_width))
        self.initial_row_factor._sdm_memory_bank = self.initial_column_factor._sdm_memory_bank = True
        self.output_gate = nn.Linear(config.dim, config.value_width, bias=True)
        self.output_norm_weight = nn.Parameter(torch.ones(config.value_width))
        if config.output_normalization == 'layer':
            self.output_norm_bias = nn.Parameter(torch.zeros(config.value_width))
        self.o_proj = nn.Linear(config.value_width, config.dim, bias=config.output_bias)
        self._fused_cache = None  # concatenated inference projection, keyed by the parameters' storage
        self.init_weights(initialization_seed=self.initialization_seed)

    # -- geometry helpers (_parameters.py:11-38) ------------------------------------
    @property
    def total_rows(self) -> int:
        return self.bank_count * self.num_heads * self.bank_size

    @property
    def touched_rows(self) -> int:
        return self.num_writes * self.num_heads * self.bank_size

    @property
    def logical_reads(self) -> int:
        return self.num_reads * self.num_heads * self.bank_size

    @property
    def logical_writes(self) -> int:
        return self.num_writes * self.num_heads * self.bank_size

    @property
    def initial_state_parameter_count(self) -> int:
        return sum(p.numel() for p in (self.initial_state, self.initial_row_factor, self.initial_column_factor)
                   if p is not None)

    def materialize_initial_state(self) -> Tensor:
        """M0 from the product factors (_parameters.py:40-67): row n = j*H*S + h*S + s
        starts at U[n // Q] + Z[n % Q].  [J, H, S, v] for H > 1, [J, S, V] for H = 1."""
        total = self.initial_row_factor[:, None, :] + self.initial_column_factor[None, :, :]
        if self.num_heads != 1:
            return total.reshape(self.bank_count, self.num_heads, self.bank_size, self.head_value_width)
        return total.reshape(self.bank_count, self.bank_size, self.value_width)

    # -- initialisation (_parameters.py:69-180) --------------------------------------
    def _role_generator(self, role: str, parameter: Tensor, initialization_seed):
        if initialization_seed is None:
            return None
        key = f'bank_sparse_gdn2.{self.layer_id}.{role}'.encode()
        digest = int.from_bytes(hashlib.blake2b(key, digest_size=8).digest(), byteorder='little')
        generator = torch.Generator(device=parameter.device)
        generator.manual_seed((initialization_seed ^ digest) % (1 << 63))
        return generator

    def init_weights(self, init_std=None, factor: float = 1.0, width_scaling=None, *,
                     initialization_seed=None) -> None:
        del width_scaling
        if initialization_seed is None:
            initialization_seed = self.initialization_seed
        if initialization_seed is not None and initialization_seed < 0:
            raise ValueError('initialization_seed must be non-negative')
        for name, module in self.named_modules():
            if isinstance(module, nn.Linear) and not name.startswith('shared_router.'):
                nn.init.xavier_uniform_(module.weight, gain=2 ** -2.5,
                                        generator=self._role_generator(f'{name}.weight', module.weight,
                                                                       initialization_seed))
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
        route_std = (init_std or self.hidden_size ** -0.5) / factor
        base = self.shared_router.base.weight
        self.shared_router.initialize_from_independent(
            std=route_std,
            read_generator=self._role_generator('read_router.weight', base, initialization_seed),
            write_generator=self._role_generator('write_router.weight', base, initialization_seed))
        with torch.no_grad():
            self.A_log.uniform_(1.0, 16.0, generator=self._role_generator('decay_rate', self.A_log,
                                                                         initialization_seed)).log_()
            log_dt = torch.empty_like(self.dt_bias).uniform_(
                math.log(0.001), math.log(0.1),
                generator=self._role_generator('time_step', self.dt_bias, initialization_seed))
            dt = log_dt.exp().clamp_min(1e-4)
            self.dt_bias.copy_(dt + torch.log(-torch.expm1(-dt)))
            for role, parameter in (('initial_state.row', self.initial_row_factor),
                                    ('initial_state.column', self.initial_column_factor)):
                std = (init_std or self.hidden_size ** -0.5) / factor
                nn.init.trunc_normal_(parameter, mean=0.0, std=std, a=-3 * std, b=3 * std,
                                      generator=self._role_generator(role, parameter, initialization_seed))
                parameter.mul_(1 / math.sqrt(2))
            self.output_norm_weight.fill_(1.0)
            if hasattr(self, 'output_norm_bias'):
                self.output_norm_bias.zero_()

    def reset_parameters(self) -> None:
        self.init_weights(initialization_seed=self.initialization_seed)

    # -- controllers, routes and output interface -----------------------------------
    def _route_projections(self, hidden: Tensor) -> tuple[Tensor, Tensor]:
        return self.shared_router.read(hidden), self.shared_router.write(hidden)

    def _route(self, projected: Tensor, selected_banks: int):
        return product_key_route(projected, bank_count=self.bank_count, selected_banks=selected_banks)

    def _route_both(self, write_routes: Tensor, read_routes: Tensor):
        """Both roles' routes, ``(ww, wi), (rw, ri)``: one launch when no
        gradient flows to the scores and the roles select equally many banks."""
        needs_grad = torch.is_grad_enabled() and (write_routes.requires_grad or read_routes.requires_grad)
        if not needs_grad and self.num_writes == self.num_reads:
            return ops.router_select_pair(write_routes, read_routes, bank_count=self.bank_count,
                                          selected_banks=self.num_writes)
        return self._route(write_routes, self.num_writes), self._route(read_routes, self.num_reads)

    def _route_and_dispatch(self, write_routes: Tensor, read_routes: Tensor):
        """Both roles' routes and the dispatch over them: one library call
        (ops.route_dispatch) when no gradient flows to the scores and the
        roles select equally many banks, else the two steps."""
        needs_grad = torch.is_grad_enabled() and (write_routes.requires_grad or read_routes.requires_grad)
        if (not needs_grad and self.num_writes == self.num_reads and write_routes.ndim == 3
                and write_routes.shape == read_routes.shape and write_routes.dtype == read_routes.dtype):
            return ops.route_dispatch(write_routes, read_routes, bank_count=self.bank_count,
                                      selected_banks=self.num_writes)
        (ww, wi), (rw, ri) = self._route_both(write_routes, read_routes)
        return (ww, wi), (rw, ri), ops.dispatch_build(wi, ri, self.bank_count)

    def _normalize_qk(self, value: Tensor) -> Tensor:
        """'nvidia': x * rsqrt(sum x^2 + 1e-6) in FP32 (the in-file formula of
        _parameters.py:219; the reference calls FLA's l2norm on GPU, which is not
        available here); 'original': F.normalize (:220)."""
        if self.config.qk_normalization == 'nvidia':
            xf = value.float()
            return (xf * torch.rsqrt(xf.square().sum(-1, keepdim=True) + 1e-6)).to(value.dtype)
        return F.normalize(value.float(), dim=-1).to(value.dtype)

    def _controllers(self, hidden: Tensor):
        """Per-head controllers (heads.py:11-22): q,k,g,b [B,T,H,S]; v,w [B,T,H,v]."""
        shape = (*hidden.shape[:-1], self.num_heads)
        q = self._normalize_qk(F.silu(self.q_proj(hidden)).reshape(*shape, self.bank_size))
        k = self._normalize_qk(F.silu(self.k_proj(hidden)).reshape(*shape, self.bank_size))
        v = F.silu(self.v_proj(hidden)).reshape(*shape, self.head_value_width)
        g = -self.A_log.float().exp()[:, None] * F.softplus(
            (self.f_proj(hidden).float() + self.dt_bias.float()).reshape(*shape, self.bank_size))
        b = self.b_proj(hidden).sigmoid().reshape(*shape, self.bank_size)
        w = self.w_proj(hidden).sigmoid().reshape(*shape, self.head_value_width)
        return q, k, v, g, b, w

    # -- fused inference path -----------------------------------------------------------
    def _fused_weights(self):
        """One weight and bias for every linear map of ``hidden`` the layer makes
        (q, k, v, the first f_proj factor, b, w, both route roles, the output
        gate), concatenated along the outputs and cached while the parameters
        keep their storage and version.  Returns (weight, bias, column offsets)."""
        router = self.shared_router
        parts = [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.f_proj[0].weight,
                 self.b_proj.weight, self.w_proj.weight]
        tracked = parts + [router.base.weight, router.base.bias, router.read_residual.weight,
                           router.read_residual.bias, router.write_residual.weight, router.write_residual.bias,
                           self.output_gate.weight, self.output_gate.bias]
        key = tuple((t.data_ptr(), t._version, t.dtype) for t in tracked)
        if self._fused_cache is None or self._fused_cache[0] != key:
            with torch.no_grad():
                read_w = router.base.weight + router.read_residual.weight
                write_w = router.base.weight + router.write_residual.weight
                weight = torch.cat(parts + [read_w, write_w, self.output_gate.weight], 0).contiguous()
                plain = sum(t.shape[0] for t in parts)
                bias = torch.cat([torch.zeros(plain, device=weight.device, dtype=weight.dtype),
                                  router.base.bias + router.read_residual.bias,
                                  router.base.bias + router.write_residual.bias, self.output_gate.bias])
            names = ('q', 'k', 'v', 'f', 'b', 'w', 'read', 'write', 'gate')
            widths = [t.shape[0] for t in parts] + [read_w.shape[0], write_w.shape[0], self.output_gate.weight.shape[0]]
            columns, at = {}, 0
            for name, width in zip(names, widths):
                columns[name] = at
                at += width
            self._fused_cache = (key, weight, bias, columns)
        return self._fused_cache[1:]

    def _fused_supported(self, hidden: Tensor) -> bool:
        return (hidden.dtype in (torch.bfloat16, torch.float32) and self.A_log.dtype == self.dt_bias.dtype
                and self.bank_size in (8, 16, 32) and self.value_width % 8 == 0 and self.value_width <= 4096
                and self.output_norm_weight.dtype in (torch.bfloat16, torch.float32))

    def _fused_controllers(self, hidden: Tensor, proj: Tensor | None = None):
        """Inference controllers, route scores and the output-gate projection from
        one projection GEMM and the controller epilogue (heads.py:11-22).
        ``proj``: the projection already computed (hidden then only gives the
        leading shape)."""
        weight, bias, cols = self._fused_weights()
        lead = hidden.shape[:-1]
        if proj is None:
            proj = ops.linear(hidden.reshape(-1, self.hidden_size), weight, bias)
        hv, rw = self.head_value_width, self.factor_route_width
        f = ops.linear(proj[:, cols['f']:cols['f'] + hv], self.f_proj[1].weight)
        q, k, v, g, b, w = ops.controller_epilogue(proj, f, cols, self.A_log, self.dt_bias, heads=self.num_heads,
                                                   bank_size=self.bank_size, head_width=hv,
                                                   qk_norm=self.config.qk_normalization)
        heads = (*lead, self.num_heads)
        controllers = (q.view(*heads, self.bank_size), k.view(*heads, self.bank_size), v.view(*heads, hv),
                       g.view(*heads, self.bank_size), b.view(*heads, self.bank_size), w.view(*heads, hv))
        read_scores = proj[:, cols['read']:cols['read'] + rw].view(*lead, rw)
        write_scores = proj[:, cols['write']:cols['write'] + rw].view(*lead, rw)
        gate = proj[:, cols['gate']:cols['gate'] + self.value_width]
        return controllers, (read_scores, write_scores), gate

    def _inference_inputs(self, hidden: Tensor):
        """The controllers and route scores prefill and step use: the fused
        projection and epilogue where the geometry allows, the torch ops
        otherwise.  Returns ((q, k, v, g, b, w), (read scores, write scores),
        the output-gate projection or None)."""
        if self._fused_supported(hidden):
            return self._fused_controllers(hidden)
        return self._controllers(hidden), self._route_projections(hidden), None

    def _inference_output(self, hidden: Tensor, gate, raw: Tensor) -> Tensor:
        return self._fused_output(gate, raw) if gate is not None else self._project_bank_output(hidden, raw)

    def _fused_output(self, gate: Tensor, raw: Tensor) -> Tensor:
        """_project_bank_output (_parameters.py:222-232) with the normalization
        and gate in one epilogue kernel, then o_proj."""
        layer = self.config.output_normalization == 'layer'
        normalized = ops.output_epilogue(raw.reshape(-1, self.value_width), gate, self.output_norm_weight,
                                         self.output_norm_bias if layer else None, eps=self.norm_eps,
                                         kind='layer' if layer else 'rms')
        return ops.linear(normalized, self.o_proj.weight, self.o_proj.bias).view(*raw.shape[:-1], -1)

    def _project_bank_output(self, hidden: Tensor, raw: Tensor) -> Tensor:
        """LN (or RMS) x sigmoid gate -> o_proj (_parameters.py:222-232)."""
        if self.config.output_normalization == 'layer':
            normalized = F.layer_norm(raw, (self.value_width,), self.output_norm_weight,
                                      self.output_norm_bias, self.norm_eps)
            return self.o_proj(normalized * torch.sigmoid(self.output_gate(hidden)).to(raw.dtype))
        variance = raw.float().square().mean(dim=-1, keepdim=True)
        normalized = raw * torch.rsqrt(variance + self.norm_eps).to(raw.dtype)
        normalized = normalized * self.output_norm_weight.to(raw.dtype)
        return self.o_proj(normalized * torch.sigmoid(self.output_gate(hidden)).to(raw.dtype))

    def _state_heads(self, state: Tensor) -> Tensor:
        return state.reshape(self.bank_count, self.num_heads, self.bank_size, self.head_value_width)

    # -- forward (model.py:88-140) ----------------------------------------------------
    def bank_reads(self, hidden: Tensor) -> Tensor:
        """The routed-memory path: concatenated head reads y [B, T, V]."""
        q, k, v, g, b, w = self._controllers(hidden)
        read_routes, write_routes = self._route_projections(hidden)
        (ww, wi), (rw, ri) = self._route_both(write_routes, read_routes)
        state = self._state_heads(self.materialize_initial_state())
        operator = bank_training if self.config.routed_decay else role_bank_training
        return operator(q, k, v, g, b, w, wi, ww, ri, rw, state, self.bank_count, self.bank_size ** -0.5,
                        compact_replay=self.compact_replay,
                        state_dtype=getattr(torch, self.config.training_state_dtype))

    def forward(self, hidden: Tensor) -> Tensor:
        if hidden.ndim != 3 or hidden.shape[-1] != self.hidden_size or hidden.shape[1] == 0:
            raise ValueError('hidden must be [batch, positive time, dim]')
        if not hidden.is_cuda:
            raise ValueError('the hip backend requires ROCm tensors; the CPU oracle lives in oracle/')
        if not torch.is_grad_enabled() and self._fused_supported(hidden):
            return self._forward_inference(hidden)
        return self._project_bank_output(hidden, self.bank_reads(hidden))

    def _forward_inference(self, hidden: Tensor) -> Tensor:
        """forward without autograd: the projections through one GEMM and the
        controller epilogue, both routes in one launch, the routed operator's
        forward (the training state and rounding policy of bank_reads, no
        snapshots) and the output interface in one epilogue before o_proj --
        about a third of the launches of the autograd path."""
        controllers, (read_routes, write_routes), gate = self._fused_controllers(hidden)
        (ww, wi), (rw, ri), meta = self._route_and_dispatch(write_routes, read_routes)
        q, k, v, g, b, w = controllers
        state = self._state_heads(self.materialize_initial_state())
        # the routed operator's forward (bank_training, routed_update.py:16-53)
        # on this dispatch: its state policy, no snapshots under no_grad
        interval = _round_interval(self.bank_size, getattr(torch, self.config.training_state_dtype),
                                   self.compact_replay, q.dtype)
        raw = ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, state, meta, bank_count=self.bank_count,
                                 scale=self.bank_size ** -0.5, routed_decay=self.config.routed_decay,
                                 round_interval=interval)
        return self._fused_output(gate, raw)

    # -- stateful inference (inference.py:88-194) -----------------------------------
    def _cache_shape(self, batch: int) -> tuple[int, ...]:
        if self.num_heads == 1:
            return (batch, self.bank_count, self.bank_size, self.value_width)
        return (batch, self.bank_count, self.num_heads, self.bank_size, self.head_value_width)

    def _validate_stateful(self, hidden: Tensor, state: Tensor | None) -> None:
        if not hidden.is_cuda:
            raise ValueError('Stateful inference requires the HIP backend on a ROCm device')
        if hidden.ndim != 3 or hidden.shape[1] == 0 or hidden.shape[-1] != self.hidden_size:
            raise ValueError('hidden must be [batch, positive time, dim]')
        if state is not None and (tuple(state.shape) != self._cache_shape(hidden.shape[0])
                                  or state.dtype not in (torch.float32, torch.bfloat16)
                                  or state.device != hidden.device or not state.is_contiguous()):
            raise ValueError('state must be contiguous FP32 or BF16 [batch, banks, (heads,) rows, values] '
                             'on the input device')

    def create_state(self, batch: int, *, dtype=torch.bfloat16) -> Tensor:
        """Initial cache: factors added in parameter dtype, stored in ``dtype``
        (inference.py:100-107, product_routed_update.py:10-21)."""
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError('cache dtype must be FP32 or BF16')
        with torch.no_grad():
            total = (self.initial_row_factor[:, None, :] + self.initial_column_factor[None, :, :])
            # the sum is in parameter dtype; widening BF16 to FP32 and back is
            # exact, so only a change of dtype converts
            initial = total if total.dtype == dtype else total.float().to(dtype)
            initial = initial.reshape(self._cache_shape(1)[1:]).unsqueeze(0)
            if batch == 1:
                return initial.contiguous()
            return initial.expand(batch, *initial.shape[1:]).contiguous()

    def prefill(self, hidden: Tensor, state: Tensor | None = None, *, state_dtype=None):
        """Process a prefix; BF16 cache storage (the default) rounds at handoff.
        Recurrence arithmetic is FP32 with no interior rounding (forward_rows.py:176-184)."""
        self._validate_stateful(hidden, state)
        if torch.is_grad_enabled():
            raise RuntimeError('Stateful inference requires no_grad or inference_mode')
        cache_dtype = state_dtype or (state.dtype if state is not None else torch.bfloat16)
        if cache_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError('cache dtype must be FP32 or BF16')
        if state is None:
            work = torch.float32 if self.initial_row_factor.dtype != cache_dtype else cache_dtype
            state = self.create_state(hidden.shape[0], dtype=work)
        elif state_dtype is not None and state_dtype != state.dtype:
            raise ValueError('state_dtype must match the supplied cache')
        (q, k, v, g, b, w), (read_routes, write_routes), gate = self._inference_inputs(hidden)
        (ww, wi), (rw, ri), meta = self._route_and_dispatch(write_routes, read_routes)
        heads_view = state.view(hidden.shape[0], self.bank_count, self.num_heads, self.bank_size,
                                self.head_value_width)
        raw = ops.routed_forward(q, k, v, g, b, w, wi, ww, ri, rw, heads_view, meta,
                                 bank_count=self.bank_count, scale=self.bank_size ** -0.5,
                                 routed_decay=self.config.routed_decay, round_interval=0,
                                 final_state=heads_view)
        if state.dtype != cache_dtype:
            state = state.to(cache_dtype)
        return self._inference_output(hidden, gate, raw), state

    def step(self, hidden: Tensor, state: Tensor):
        """Advance an existing bank state by one token (inference only)."""
        self._validate_stateful(hidden, state)
        if torch.is_grad_enabled() or hidden.shape[1] != 1:
            raise ValueError('step requires one token under no_grad/inference_mode')
        if self._fused_supported(hidden):
            weight, bias, cols = self._fused_weights()
            proj = ops.linear(hidden.reshape(-1, self.hidden_size), weight, bias)
            gate = proj[:, cols['gate']:cols['gate'] + self.value_width]
            raw = self._decode_fused(proj, state)
            if raw is None:
                controllers, scores, gate = self._fused_controllers(hidden, proj=proj)
                raw = self._decode_banks(controllers, scores, hidden.shape[0], state)
            return self._fused_output(gate, raw.unsqueeze(1)), state
        (q, k, v, g, b, w), (read_routes, write_routes), gate = self._inference_inputs(hidden)
        raw = self._decode_banks((q, k, v, g, b, w), (read_routes, write_routes), hidden.shape[0], state)
        return self._inference_output(hidden, gate, raw.unsqueeze(1)), state

    def _decode_fused(self, proj: Tensor, state: Tensor) -> Tensor | None:
        """The step's controller epilogue, routes and decode kernel in one
        launch from the fused projection ``proj`` [B, P]: the bank reads [B, V],
        or None where ``ops.decode_fused`` does not take the geometry."""
        if not self.fused_decode or self.num_reads != self.num_writes:
            return None
        _, _, cols = self._fused_weights()
        rows, hv = proj.shape[0], self.head_value_width
        heads_view = state.view(rows, self.bank_count, self.num_heads, self.bank_size, hv)
        geometry = dict(heads=self.num_heads, bank_size=self.bank_size, head_width=hv, bank_count=self.bank_count,
                        selected_banks=self.num_writes)
        options = dict(qk_norm=self.config.qk_normalization, routed_decay=self.config.routed_decay,
                       scale=self.bank_size ** -0.5)
        f_weight = self.f_proj[1].weight
        # f_proj's second factor inside the launch where it takes it (one GEMM node fewer)
        if ops.decode_fused_supported(proj, None, cols, self.A_log, self.dt_bias, heads_view, **geometry,
                                      f_weight=f_weight):
            return ops.decode_fused(proj, None, cols, self.A_log, self.dt_bias, heads_view, **geometry, **options,
                                    f_weight=f_weight)
        f = ops.linear(proj[:, cols['f']:cols['f'] + hv], f_weight)
        if not ops.decode_fused_supported(proj, f, cols, self.A_log, self.dt_bias, heads_view, **geometry):
            return None
        return ops.decode_fused(proj, f, cols, self.A_log, self.dt_bias, heads_view, **geometry, **options)

    def _decode_banks(self, controllers, scores, batch: int, state: Tensor) -> Tensor:
        """Both routes and the decode kernel of one step: the bank reads [B, V]."""
        q, k, v, g, b, w = controllers
        read_routes, write_routes = scores
        width = read_routes.shape[-1]
        if (batch == 1 and self.num_reads == self.num_writes and read_routes.stride(-1) == 1
                and write_routes.data_ptr() == read_routes.data_ptr() + width * read_routes.element_size()):
            # one token: its read and write scores are adjacent slices of the
            # projection row, so both roles route in one launch, as two rows
            pair = torch.as_strided(read_routes, (1, 2, width), (2 * width, width, 1))
            weights, indices = self._route(pair, self.num_reads)
            rw, ww = weights[:, 0:1], weights[:, 1:2]
            ri, wi = indices[:, 0:1], indices[:, 1:2]
        else:
            (ww, wi), (rw, ri) = self._route_both(write_routes, read_routes)
        heads_view = state.view(batch, self.bank_count, self.num_heads, self.bank_size, self.head_value_width)
        return ops.decode_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], b[:, 0], w[:, 0], wi[:, 0], ww[:, 0],
                               ri[:, 0], rw[:, 0], heads_view, bank_count=self.bank_count,
                               scale=self.bank_size ** -0.5, routed_decay=self.config.routed_decay)

    def step_fused_norm(self, hidden: Tensor, delta: Tensor | None, norm_weight: Tensor, norm_eps: float,
                        state: Tensor):
        """The memory sublayer of a pre-norm block for one decode token, with the
        block's residual add and RMSNorm formed inside the projection GEMV and
        the output interface inside the o_proj GEMV (``bdm_gemv_ex``):
        h = hidden + delta (delta None: h = hidden), out = step(RMSNorm(h)).
        Returns (out, h).  It matches the unfused kernels within tolerance:
        the decode launch forms f itself in another summation order, and the
        layer-norm prologue may differ from the standalone kernel by an ulp."""
        weight, bias, _ = self._fused_weights()
        rows = hidden.shape[0]
        flat = hidden.reshape(rows, self.hidden_size)
        if delta is None:
            proj = ops.gemv_fused(flat, weight, bias, prologue='rms', norm_weight=norm_weight, eps=norm_eps)
            new_hidden = hidden
        else:
            proj, total = ops.gemv_fused(delta.reshape(rows, self.hidden_size), weight, bias, prologue='rms',
                                         residual=flat, norm_weight=norm_weight, eps=norm_eps)
            new_hidden = total.view_as(hidden)
        _, _, cols = self._fused_weights()
        gate = proj[:, cols['gate']:cols['gate'] + self.value_width]
        raw = self._decode_fused(proj, state)
        if raw is None:
            controllers, scores, gate = self._fused_controllers(new_hidden, proj=proj)
            raw = self._decode_banks(controllers, scores, rows, state)
        layer = self.config.output_normalization == 'layer'
        out = ops.gemv_fused(raw, self.o_proj.weight, self.o_proj.bias,
                             prologue='out_layer' if layer else 'out_rms', norm_weight=self.output_norm_weight,
                             norm_bias=self.output_norm_bias if layer else None, gate=gate, eps=self.norm_eps)
        return out.view(rows, 1, self.hidden_size), new_hidden

    def step_fused_norm_supported(self, hidden: Tensor, norm_weight: Tensor) -> bool:
        rows = hidden.shape[0]
        return (hidden.is_cuda and hidden.dim() == 3 and hidden.shape[1] == 1 and 1 <= rows <= ops.GEMV_MAX_ROWS
                and self._fused_supported(hidden) and self.hidden_size % 8 == 0
                and max(self.hidden_size, self.value_width) <= ops.GEMV_PROLOGUE_MAX_K
                and self.o_proj.weight.dtype == hidden.dtype and self.q_proj.weight.dtype == hidden.dtype
                and norm_weight.dtype in (torch.bfloat16, torch.float32)
                and (self.o_proj.bias is None or self.o_proj.bias.dtype == hidden.dtype))
