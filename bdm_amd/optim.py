"""The shell's AdamW recipe with FP32 masters, as one fused HIP pass.

Reference: reproduction/experiments/optim.py:7-50 (``AdamW`` for the "wiki"
benchmark).  Each step there clips the BF16 gradients to norm 1.0 in place,
copies them to FP32 master gradients, runs torch's fused AdamW on the FP32
masters and copies the masters back into the BF16 weights: four passes over
every parameter.  ``MasterAdamW.step`` computes the clipping norm with torch
(the same calls, so the same BF16 coefficient) and then makes one pass
(``bdm_adamw_step``) that scales each gradient as the in-place clip would,
updates the master and both moments with torch's fused-AdamW arithmetic and
writes the rounded master into the weight.  The masters and moments live in
three flat FP32 buffers.

Differences from the reference wrapper: the gradients are left unscaled
(the reference leaves them clipped), ``step`` returns the norm as a device
tensor (the reference returns a Python float, a host synchronisation) and
does not raise on a non-finite norm (the reference's error_if_nonfinite
check also synchronises the host; test the returned norm instead), and every
parameter must have a gradient at each step.  ``state_dict`` and
``load_state_dict`` save and restore the masters, moments and step count;
``reload_masters`` re-reads the masters from the current weights.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

_ALIGN = 4  # elements: a tensor's slice of the flat buffers starts 16-byte aligned
CHUNK = 16384  # elements per workgroup


class MasterAdamW:
    """BF16 weights with FP32 masters, moments and a fused update.

    ``params``: the BF16 CUDA parameters (``network.parameters()``); a
    parameter flagged ``_no_weight_decay`` takes weight decay 0, the others
    ``weight_decay`` (the reference's two groups).  ``step(lr)`` clips to
    ``max_norm`` and applies one AdamW update with learning rate ``lr``.
    """

    def __init__(self, params, lr: float = 3e-4, betas=(0.9, 0.95), eps: float = 1e-8, weight_decay: float = 0.01,
                 max_norm: float = 1.0) -> None:
        self.params = list(params)
        if not self.params:
            raise ValueError('MasterAdamW needs parameters')
        device = self.params[0].device
        for p in self.params:
            if p.device != device or not p.is_cuda or p.dtype != torch.bfloat16 or not p.is_contiguous():
                raise ValueError('MasterAdamW takes contiguous BF16 parameters on one ROCm device')
        self.lr, self.betas, self.eps, self.max_norm = float(lr), (float(betas[0]), float(betas[1])), float(eps), \
            float(max_norm)
        self.device = device
        offsets, total = [], 0
        for p in self.params:
            offsets.append(total)
            total += (p.numel() + _ALIGN - 1) // _ALIGN * _ALIGN
        self.offsets = offsets
        self.master = torch.zeros(total, dtype=torch.float32, device=device)
        for p, off in zip(self.params, offsets):
            self.master[off:off + p.numel()].copy_(p.detach().reshape(-1))
        self.exp_avg = torch.zeros_like(self.master)
        self.exp_avg_sq = torch.zeros_like(self.master)
        self.decay = [0.0 if bool(getattr(p, '_no_weight_decay', False)) else float(weight_decay) for p in self.params]
        block_tensor, block_start = [], []
        for i, p in enumerate(self.params):
            for start in range(0, p.numel(), CHUNK):
                block_tensor.append(i)
                block_start.append(start)
        self.block_tensor = torch.tensor(block_tensor, dtype=torch.int32, device=device)
        self.block_start = torch.tensor(block_start, dtype=torch.int64, device=device)
        self.blocks = len(block_tensor)
        n = len(self.params)
        self._desc_host = (_lib.AdamwTensor * n)()
        for i, (p, off) in enumerate(zip(self.params, offsets)):
            self._desc_host[i].param = p.data_ptr()
            self._desc_host[i].offset = off
            self._desc_host[i].numel = p.numel()
            self._desc_host[i].weight_decay = self.decay[i]
        nbytes = ctypes.sizeof(self._desc_host)
        self._desc_pinned = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
        self._desc = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self._desc_copied = None  # event after the last upload of the pinned descriptors
        self._scale = torch.ones(1, dtype=torch.float32, device=device)
        self.step_count = 0

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None

    @torch.no_grad()
    def step(self, lr: float | None = None) -> Tensor:
        grads = [p.grad for p in self.params]
        if any(g is None for g in grads):
            raise ValueError('MasterAdamW.step: every parameter needs a gradient')
        for p, g in zip(self.params, grads):
            if g.dtype != torch.bfloat16 or not g.is_contiguous() or g.shape != p.shape:
                raise ValueError('MasterAdamW.step: gradients must be contiguous BF16 of the parameter shape')
        # clip_grad_norm_(params, max_norm): the same norm and BF16 coefficient
        norm = torch.nn.utils.get_total_norm(grads, 2.0)
        coef = torch.clamp(self.max_norm / (norm + 1e-6), max=1.0)
        self._scale.copy_(coef.reshape(1))
        if lr is not None:
            self.lr = float(lr)
        self.step_count += 1
        if self._desc_copied is not None:
            self._desc_copied.synchronize()  # the previous upload has left the pinned buffer
        for i, (p, g) in enumerate(zip(self.params, grads)):
            self._desc_host[i].param = p.data_ptr()  # current storage, should the parameter have moved
            self._desc_host[i].grad = g.data_ptr()
        ctypes.memmove(self._desc_pinned.data_ptr(), ctypes.addressof(self._desc_host), ctypes.sizeof(self._desc_host))
        self._desc.copy_(self._desc_pinned, non_blocking=True)
        self._desc_copied = torch.cuda.Event()
        self._desc_copied.record()
        args = _lib.AdamwArgs()
        args.tensors = self._desc.data_ptr()
        args.block_tensor = self.block_tensor.data_ptr()
        args.block_start = self.block_start.data_ptr()
        args.tensor_count, args.blocks, args.chunk = len(self.params), self.blocks, CHUNK
        args.master, args.exp_avg, args.exp_avg_sq = (self.master.data_ptr(), self.exp_avg.data_ptr(),
                                                      self.exp_avg_sq.data_ptr())
        args.grad_scale = self._scale.data_ptr()
        args.lr, args.beta1, args.beta2, args.eps = self.lr, self.betas[0], self.betas[1], self.eps
        args.step = float(self.step_count)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(_lib.library().bdm_adamw_step(ctypes.byref(args), ctypes.c_void_p(stream)), 'bdm_adamw_step')
        return norm

    def state_dict(self) -> dict:
        """The FP32 masters and both moments per parameter (CPU copies), the
        step count and the hyperparameters: what resuming needs.  The content
        is what the reference wrapper saves (reproduction/experiments/
        optim.py:52-54), but not its layout ({'optimizer': torch AdamW state,
        'masters': [...]}): the two checkpoint formats do not interchange."""
        count = len(self.params)
        return {'masters': [self.master_of(i).detach().cpu().clone() for i in range(count)],
                'exp_avg': [self.moments_of(i)[0].detach().cpu().clone() for i in range(count)],
                'exp_avg_sq': [self.moments_of(i)[1].detach().cpu().clone() for i in range(count)],
                'step': self.step_count, 'lr': self.lr, 'betas': self.betas, 'eps': self.eps,
                'max_norm': self.max_norm, 'weight_decay': list(self.decay)}

    @torch.no_grad()
    def load_state_dict(self, state: dict) -> None:
        """Restore masters, moments and the step count, with the reference's
        checks (optim.py:57-71): FP32 tensors of the parameters' shapes, and
        the same per-parameter weight decay as this optimizer's.  The
        BF16 weights are left as they are; call ``reload_masters`` first if the
        weights, not the saved masters, should win."""
        count = len(self.params)
        if 'weight_decay' in state and [float(d) for d in state['weight_decay']] != [float(d) for d in self.decay]:
            raise ValueError('Invalid optimizer checkpoint: per-parameter weight decay differs from this '
                             "optimizer's (it is fixed at construction)")
        for key in ('masters', 'exp_avg', 'exp_avg_sq'):
            saved = state[key]
            if len(saved) != count:
                raise ValueError('Invalid FP32 master checkpoint: parameter count changed')
            for p, t in zip(self.params, saved):
                if t.dtype != torch.float32 or tuple(t.shape) != tuple(p.shape):
                    raise ValueError('Invalid FP32 master checkpoint' if key == 'masters'
                                     else 'Optimizer moment precision changed')
        for i in range(count):
            self.master_of(i).copy_(state['masters'][i])
            avg, avg_sq = self.moments_of(i)
            avg.copy_(state['exp_avg'][i])
            avg_sq.copy_(state['exp_avg_sq'][i])
        self.step_count = int(state['step'])
        self.lr = float(state.get('lr', self.lr))
        self.betas = tuple(float(b) for b in state.get('betas', self.betas))
        self.eps = float(state.get('eps', self.eps))
        self.max_norm = float(state.get('max_norm', self.max_norm))

    @torch.no_grad()
    def reload_masters(self) -> None:
        """Copy the current BF16 weights into the FP32 masters (after weights
        were loaded or edited once the optimizer exists); moments are kept."""
        for i, p in enumerate(self.params):
            self.master_of(i).copy_(p.detach())

    def master_of(self, i: int) -> Tensor:
        """Parameter i's FP32 master, shaped like the parameter (a view)."""
        p = self.params[i]
        return self.master[self.offsets[i]:self.offsets[i] + p.numel()].view(p.shape)

    def moments_of(self, i: int) -> tuple[Tensor, Tensor]:
        p = self.params[i]
        sl = slice(self.offsets[i], self.offsets[i] + p.numel())
        return self.exp_avg[sl].view(p.shape), self.exp_avg_sq[sl].view(p.shape)
