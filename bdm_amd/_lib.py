"""ctypes binding of ``libbdm_hip.so`` (the C ABI declared in ``include/bdm_hip.h``).

The library is built in-tree by ``bdm_amd/csrc/Makefile``.  Loading never
falls back to anything else: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

LIBRARY_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libbdm_hip.so')

BDM_F32 = 0
BDM_BF16 = 1
BDM_ROUTE_OUT_OF_RANGE = 1
BDM_ROUTE_DUPLICATE = 2

EXPORTED_SYMBOLS = (
    'bdm_version', 'bdm_last_error_string', 'bdm_router_select', 'bdm_dispatch_workspace_size',
    'bdm_dispatch_build', 'bdm_forward_workspace_size', 'bdm_forward', 'bdm_snapshot_rows',
    'bdm_backward_workspace_size', 'bdm_backward', 'bdm_decode', 'bdm_decode_fused', 'bdm_decode_fused_supported',
    'bdm_controller_epilogue', 'bdm_output_epilogue',
    'bdm_bank_occupancy',
    'bdm_written_bank_curve',
    'bdm_rms_norm',
    'bdm_swiglu',
    'bdm_gemv',
    'bdm_gemv_ex',
    'bdm_adamw_step',
    'bdm_rms_norm_backward_partials',
    'bdm_rms_norm_backward',
    'bdm_swiglu_pair',
    'bdm_swiglu_backward',
    'bdm_dispatch_workspace_size_ex',
    'bdm_dispatch_build_static',
    'bdm_router_select_pair',
    'bdm_route_dispatch_workspace_size',
    'bdm_route_dispatch',
)

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_size_t = ctypes.c_size_t


class ForwardArgs(ctypes.Structure):
    """Mirror of ``bdm_forward_args``."""
    _fields_ = [
        ('q', _vp), ('k', _vp), ('g', _vp), ('b', _vp), ('v', _vp), ('w', _vp),
        ('write_weights', _vp), ('read_weights', _vp), ('read_indices', _vp),
        ('order', _vp), ('cu_seqlens', _vp), ('initial', _vp), ('final_state', _vp), ('output', _vp),
        ('initial_batch_stride', _i64), ('batch', _i64), ('time', _i64),
        ('heads', _i32), ('bank_size', _i32), ('head_width', _i32), ('bank_count', _i32),
        ('write_banks', _i32), ('read_banks', _i32),
        ('ctrl_dtype', _i32), ('initial_dtype', _i32), ('final_dtype', _i32),
        ('routed_decay', _i32), ('round_interval', _i32), ('scale', _f32),
        ('snapshots', _vp), ('snapshot_interval', _i32), ('snapshot_dtype', _i32),
        ('phase_events', _vp * 3),
        ('segment_order', _vp),
    ]


class RouteDispatchArgs(ctypes.Structure):
    """Mirror of ``bdm_route_dispatch_args``."""
    _fields_ = [
        ('write_scores', _vp), ('write_stride', _i64), ('read_scores', _vp), ('read_stride', _i64),
        ('score_dtype', _i32), ('batch', _i64), ('time', _i64),
        ('factor_first', _i32), ('factor_second', _i32), ('selected', _i32),
        ('write_weights', _vp), ('write_indices', _vp), ('read_weights', _vp), ('read_indices', _vp),
        ('order', _vp), ('inverse', _vp), ('tokens', _vp), ('cu_seqlens', _vp), ('status', _vp),
        ('segment_order', _vp),
    ]


class BackwardArgs(ctypes.Structure):
    """Mirror of ``bdm_backward_args``."""
    _fields_ = [
        ('q', _vp), ('k', _vp), ('g', _vp), ('b', _vp), ('v', _vp), ('w', _vp),
        ('write_weights', _vp), ('read_weights', _vp), ('order', _vp), ('cu_seqlens', _vp),
        ('initial', _vp), ('snapshots', _vp), ('grad_output', _vp),
        ('grad_q', _vp), ('grad_k', _vp), ('grad_g', _vp), ('grad_b', _vp), ('grad_v', _vp), ('grad_w', _vp),
        ('grad_write_weights', _vp), ('grad_read_weights', _vp), ('grad_initial', _vp),
        ('initial_batch_stride', _i64), ('batch', _i64), ('time', _i64),
        ('heads', _i32), ('bank_size', _i32), ('head_width', _i32), ('bank_count', _i32),
        ('write_banks', _i32), ('read_banks', _i32),
        ('ctrl_dtype', _i32), ('initial_dtype', _i32), ('snapshot_dtype', _i32), ('routed_decay', _i32),
        ('round_interval', _i32), ('snapshot_interval', _i32), ('scale', _f32),
    ]


class DecodeArgs(ctypes.Structure):
    """Mirror of ``bdm_decode_args``."""
    _fields_ = [
        ('q', _vp), ('k', _vp), ('b', _vp), ('g', _vp), ('v', _vp), ('w', _vp),
        ('write_weights', _vp), ('read_weights', _vp), ('write_indices', _vp), ('read_indices', _vp),
        ('state', _vp), ('output', _vp), ('batch', _i64),
        ('heads', _i32), ('bank_size', _i32), ('head_width', _i32), ('bank_count', _i32),
        ('write_banks', _i32), ('read_banks', _i32),
        ('ctrl_dtype', _i32), ('state_dtype', _i32), ('routed_decay', _i32), ('scale', _f32),
    ]


class DecodeFusedArgs(ctypes.Structure):
    """Mirror of ``bdm_decode_fused_args``."""
    _fields_ = [
        ('proj', _vp), ('f', _vp), ('a_log', _vp), ('dt_bias', _vp), ('state', _vp), ('output', _vp),
        ('batch', _i64), ('proj_stride', _i64), ('f_stride', _i64),
        ('q_col', _i32), ('k_col', _i32), ('v_col', _i32), ('b_col', _i32), ('w_col', _i32),
        ('read_col', _i32), ('write_col', _i32),
        ('heads', _i32), ('bank_size', _i32), ('head_width', _i32), ('factor_first', _i32),
        ('factor_second', _i32), ('selected_banks', _i32),
        ('ctrl_dtype', _i32), ('param_dtype', _i32), ('state_dtype', _i32), ('qk_norm', _i32),
        ('routed_decay', _i32), ('scale', _f32),
        ('f_weight', _vp), ('f_out', _vp), ('f_col', _i32), ('f_width', _i32),
    ]


class ControllerArgs(ctypes.Structure):
    """Mirror of ``bdm_controller_args``."""
    _fields_ = [
        ('proj', _vp), ('f', _vp), ('a_log', _vp), ('dt_bias', _vp),
        ('q', _vp), ('k', _vp), ('v', _vp), ('b', _vp), ('w', _vp), ('g', _vp),
        ('tokens', _i64), ('proj_stride', _i64), ('f_stride', _i64),
        ('q_col', _i32), ('k_col', _i32), ('v_col', _i32), ('b_col', _i32), ('w_col', _i32),
        ('heads', _i32), ('bank_size', _i32), ('head_width', _i32),
        ('ctrl_dtype', _i32), ('param_dtype', _i32), ('qk_norm', _i32),
    ]


class OutputArgs(ctypes.Structure):
    """Mirror of ``bdm_output_args``."""
    _fields_ = [
        ('raw', _vp), ('gate', _vp), ('norm_weight', _vp), ('norm_bias', _vp), ('out', _vp),
        ('tokens', _i64), ('gate_stride', _i64),
        ('width', _i32), ('ctrl_dtype', _i32), ('param_dtype', _i32), ('norm_kind', _i32), ('eps', _f32),
    ]


GEMV_PLAIN, GEMV_RMS, GEMV_SWIGLU, GEMV_OUT_LAYER, GEMV_OUT_RMS = 0, 1, 2, 3, 4


class GemvArgs(ctypes.Structure):
    """Mirror of ``bdm_gemv_args``."""
    _fields_ = [
        ('x', _vp), ('weight', _vp), ('bias', _vp), ('y', _vp), ('residual', _vp), ('sum_out', _vp),
        ('norm_weight', _vp), ('norm_bias', _vp), ('gate', _vp),
        ('rows', _i64), ('n', _i64), ('k', _i64), ('gate_stride', _i64),
        ('dtype', _i32), ('param_dtype', _i32), ('prologue', _i32), ('eps', _f32),
    ]


class AdamwTensor(ctypes.Structure):
    """Mirror of ``bdm_adamw_tensor`` (40 bytes)."""
    _fields_ = [('param', _vp), ('grad', _vp), ('offset', _i64), ('numel', _i64), ('weight_decay', ctypes.c_double)]


class AdamwArgs(ctypes.Structure):
    """Mirror of ``bdm_adamw_args``."""
    _fields_ = [
        ('tensors', _vp), ('block_tensor', _vp), ('block_start', _vp),
        ('tensor_count', _i64), ('blocks', _i64), ('chunk', _i64),
        ('master', _vp), ('exp_avg', _vp), ('exp_avg_sq', _vp), ('grad_scale', _vp),
        ('lr', ctypes.c_double), ('beta1', ctypes.c_double), ('beta2', ctypes.c_double),
        ('eps', ctypes.c_double), ('step', ctypes.c_double),
    ]


class BDMError(RuntimeError):
    """A call into libbdm_hip returned a non-zero status."""


@lru_cache(maxsize=None)
def library() -> ctypes.CDLL:
    if not os.path.exists(LIBRARY_PATH):
        raise ImportError(f'{LIBRARY_PATH} is missing; build it with `make -C bdm_amd/csrc` '
                          'or __graft_entry__.build()')
    lib = ctypes.CDLL(LIBRARY_PATH)
    lib.bdm_version.restype = _i32
    lib.bdm_last_error_string.restype = ctypes.c_char_p
    lib.bdm_router_select.argtypes = [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp]
    lib.bdm_router_select.restype = _i32
    lib.bdm_dispatch_workspace_size.argtypes = [_i64, _i64, _i32]
    lib.bdm_dispatch_workspace_size.restype = _size_t
    lib.bdm_dispatch_build.argtypes = [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _size_t, _vp]
    lib.bdm_dispatch_build.restype = _i32
    lib.bdm_router_select_pair.argtypes = [_vp, _i64, _vp, _i64, _i32, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                           _vp]
    lib.bdm_router_select_pair.restype = _i32
    lib.bdm_dispatch_build_static.argtypes = [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.bdm_dispatch_build_static.restype = _i32
    lib.bdm_forward_workspace_size.argtypes = [ctypes.POINTER(ForwardArgs)]
    lib.bdm_forward_workspace_size.restype = _size_t
    lib.bdm_forward.argtypes = [ctypes.POINTER(ForwardArgs), _vp, _size_t, _vp]
    lib.bdm_forward.restype = _i32
    lib.bdm_snapshot_rows.argtypes = [_i64, _i32]
    lib.bdm_snapshot_rows.restype = _i64
    lib.bdm_backward_workspace_size.argtypes = [ctypes.POINTER(BackwardArgs)]
    lib.bdm_backward_workspace_size.restype = _size_t
    lib.bdm_backward.argtypes = [ctypes.POINTER(BackwardArgs), _vp, _size_t, _vp]
    lib.bdm_backward.restype = _i32
    lib.bdm_decode.argtypes = [ctypes.POINTER(DecodeArgs), _vp]
    lib.bdm_decode.restype = _i32
    lib.bdm_decode_fused.argtypes = [ctypes.POINTER(DecodeFusedArgs), _vp]
    lib.bdm_decode_fused.restype = _i32
    lib.bdm_decode_fused_supported.argtypes = [ctypes.POINTER(DecodeFusedArgs)]
    lib.bdm_decode_fused_supported.restype = _i32
    lib.bdm_controller_epilogue.argtypes = [ctypes.POINTER(ControllerArgs), _vp]
    lib.bdm_controller_epilogue.restype = _i32
    lib.bdm_output_epilogue.argtypes = [ctypes.POINTER(OutputArgs), _vp]
    lib.bdm_output_epilogue.restype = _i32
    lib.bdm_bank_occupancy.argtypes = [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp]
    lib.bdm_bank_occupancy.restype = _i32
    lib.bdm_written_bank_curve.argtypes = [_vp, _i64, _i32, _vp, _i32, _vp, _vp]
    lib.bdm_written_bank_curve.restype = _i32
    lib.bdm_rms_norm.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _f32, _vp]
    lib.bdm_rms_norm.restype = _i32
    lib.bdm_swiglu.argtypes = [_vp, _vp, _i64, _i32, _i32, _vp]
    lib.bdm_swiglu.restype = _i32
    lib.bdm_gemv.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp]
    lib.bdm_gemv.restype = _i32
    lib.bdm_gemv_ex.argtypes = [_vp, _vp]
    lib.bdm_gemv_ex.restype = _i32
    lib.bdm_adamw_step.argtypes = [_vp, _vp]
    lib.bdm_adamw_step.restype = _i32
    lib.bdm_rms_norm_backward_partials.argtypes = [_i64]
    lib.bdm_rms_norm_backward_partials.restype = _i64
    lib.bdm_rms_norm_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _f32, _vp]
    lib.bdm_rms_norm_backward.restype = _i32
    lib.bdm_swiglu_pair.argtypes = [_vp, _vp, _vp, _i64, _i32, _vp]
    lib.bdm_swiglu_pair.restype = _i32
    lib.bdm_swiglu_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp]
    lib.bdm_swiglu_backward.restype = _i32
    lib.bdm_dispatch_workspace_size_ex.argtypes = [_i64, _i64, _i32, _i32, _i32]
    lib.bdm_dispatch_workspace_size_ex.restype = _size_t
    lib.bdm_route_dispatch_workspace_size.argtypes = [ctypes.POINTER(RouteDispatchArgs)]
    lib.bdm_route_dispatch_workspace_size.restype = _size_t
    lib.bdm_route_dispatch.argtypes = [ctypes.POINTER(RouteDispatchArgs), _vp, _size_t, _vp]
    lib.bdm_route_dispatch.restype = _i32
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        message = library().bdm_last_error_string().decode(errors='replace')
        if status in (-1,):
            raise ValueError(f'{what}: {message}')
        if status in (-2,):
            raise NotImplementedError(f'{what}: {message}')
        raise BDMError(f'{what} failed ({status}): {message}')
