"""The C-ABI library: it loads, exports every declared symbol and rejects bad
arguments before touching a device.  Runs without a GPU."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, 'include', 'bdm_hip.h')


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(bdm_[a-z_]+)\s*\(', text)))


@pytest.fixture(scope='module')
def lib():
    from bdm_amd import _lib
    return _lib.library()


def test_header_declares_the_expected_entry_points():
    from bdm_amd import _lib
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.bdm_version() >= 1


def test_workspace_sizes(lib):
    # (tiles of 32 tokens + one row of segment totals) x banks x int32 per batch
    assert lib.bdm_dispatch_workspace_size(8, 4096, 256) == 8 * (128 + 1) * 256 * 4
    assert lib.bdm_dispatch_workspace_size(0, 4096, 256) == 0
    from bdm_amd import _lib
    args = _lib.ForwardArgs()
    args.batch, args.time, args.heads, args.head_width, args.read_banks = 2, 10, 3, 16, 4
    args.bank_size, args.write_banks = 4, 4
    args.ctrl_dtype = _lib.BDM_BF16
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # read rows: BF16, H*v per read event, row token*KR + j
    rows = r256(2 * 10 * 4 * 3 * 16 * 2)
    assert lib.bdm_forward_workspace_size(ctypes.byref(args)) == rows
    # S = 8 under the prefill policy (no rounding, no snapshots) adds the
    # piece list of cut segments: at most 2 * (E // 512) + 1 pieces, with
    # their FP32 start states [H, 8, v] and transitions [H, 8, 8]
    args.bank_size, args.head_width, args.round_interval = 8, 128, 0
    rows = r256(2 * 10 * 4 * 3 * 128 * 2)
    pieces = 2 * ((2 * 10 * 8) // 512) + 1
    extra = r256(pieces * 16) + 256 + r256(pieces * 3 * 8 * 128 * 4) + r256(pieces * 3 * 64 * 4)
    assert lib.bdm_forward_workspace_size(ctypes.byref(args)) == rows + extra
    args.round_interval = 16  # the training policy rounds inside the recurrence: no pieces
    assert lib.bdm_forward_workspace_size(ctypes.byref(args)) == rows


def test_invalid_arguments_are_rejected_without_a_launch(lib):
    from bdm_amd import _lib
    rc = lib.bdm_router_select(None, _lib.BDM_BF16, 4, 3, 16, 16, 8, None, None, None)
    assert rc == -1 and b'bad geometry' in lib.bdm_last_error_string()
    rc = lib.bdm_router_select(None, _lib.BDM_BF16, 4, 32, 16, 16, 20, None, None, None)
    assert rc == -2
    # more than 8192 banks take the radix-sort path: accepted geometry, then the null operands
    rc = lib.bdm_dispatch_build(None, None, 1, 8, 2, 2, 16384, None, None, None, None, None, None, 0, None)
    assert rc == -1 and b'null pointer' in lib.bdm_last_error_string()
    rc = lib.bdm_forward(None, None, 0, None)
    assert rc == -1
    args = _lib.ForwardArgs()
    args.batch, args.time, args.heads, args.bank_size, args.head_width = 1, 4, 1, 64, 16
    args.bank_count, args.write_banks, args.read_banks = 4, 1, 1
    assert lib.bdm_forward(ctypes.byref(args), None, 0, None) == -2
    dargs = _lib.DecodeArgs()
    assert lib.bdm_decode(ctypes.byref(dargs), None) == -1
    rargs = _lib.RouteDispatchArgs()
    assert lib.bdm_route_dispatch(None, None, 0, None) == -1
    assert lib.bdm_route_dispatch(ctypes.byref(rargs), None, 0, None) == -1
    rargs.batch, rargs.time, rargs.factor_first, rargs.factor_second, rargs.selected = 2, 64, 16, 16, 8
    rc = lib.bdm_route_dispatch(ctypes.byref(rargs), None, 0, None)
    assert rc == -1 and b'null pointer' in lib.bdm_last_error_string()


def test_python_errors_mirror_the_reference():
    import torch
    from bdm_amd import BSDMConfig, BankedDeltaMemory, ops
    with pytest.raises(ValueError):
        BankedDeltaMemory(BSDMConfig(dim=32, bank_count=16, bank_size=8, selected_banks=4, value_width=16),
                          backend='reference')
    with pytest.raises(ValueError):
        ops.router_select(torch.zeros(2, 7), bank_count=16, selected_banks=4)
    with pytest.raises(ValueError):
        ops.dispatch_build(torch.zeros(1, 2, 3, dtype=torch.int32), torch.zeros(1, 2, 3, dtype=torch.int32), 16)
    layer = BankedDeltaMemory(BSDMConfig(dim=32, bank_count=16, bank_size=8, selected_banks=4, value_width=16))
    with pytest.raises(ValueError):
        layer(torch.zeros(1, 0, 32))
    with pytest.raises(ValueError):
        layer(torch.zeros(1, 3, 32))  # CPU tensors: the HIP path never falls back


def test_backward_rejects_bad_arguments(lib):
    from bdm_amd import _lib
    assert lib.bdm_backward(None, None, 0, None) == -1
    args = _lib.BackwardArgs()
    args.batch, args.time, args.heads, args.bank_size, args.head_width = 1, 4, 1, 8, 16
    args.bank_count, args.write_banks, args.read_banks = 4, 1, 1
    args.ctrl_dtype = args.initial_dtype = args.snapshot_dtype = _lib.BDM_BF16
    args.round_interval, args.snapshot_interval = 16, 16
    assert lib.bdm_backward(ctypes.byref(args), None, 0, None) == -1  # null operands
    assert b'null pointer' in lib.bdm_last_error_string()
    args.round_interval, args.snapshot_interval = 16, 8
    assert lib.bdm_backward(ctypes.byref(args), None, 0, None) == -1
    args.round_interval, args.snapshot_interval = 0, 16
    assert lib.bdm_backward(ctypes.byref(args), None, 0, None) == -1  # BF16 snapshots of an unrounded state
    # du (NT*KW*H*v FP32) + U/X/P (3*NT*KW*H*S) + dq (NT*KR*H*S), each 256-byte aligned, and for
    # S = 8 with replay interval 16 the per-event meta (E x 16 bytes)
    args.snapshot_dtype = _lib.BDM_F32
    size = lib.bdm_backward_workspace_size(ctypes.byref(args))
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert size == up(4 * 16 * 4) + up(3 * 4 * 8 * 4) + up(4 * 8 * 4) + up(4 * 2 * 16)
    args.snapshot_interval = 8
    size = lib.bdm_backward_workspace_size(ctypes.byref(args))
    assert size == up(4 * 16 * 4) + up(3 * 4 * 8 * 4) + up(4 * 8 * 4)
    assert lib.bdm_snapshot_rows(1000, 16) == 62 and lib.bdm_snapshot_rows(0, 16) == 0


def test_struct_layouts_match_the_header(tmp_path):
    """sizeof/offsetof of every argument struct, compiled from the header with
    gcc, equal the ctypes mirrors the Python layer passes."""
    import shutil
    import subprocess
    from bdm_amd import _lib
    gcc = shutil.which('gcc')
    if gcc is None:
        pytest.skip('no host C compiler')
    mirrors = {'bdm_forward_args': _lib.ForwardArgs, 'bdm_backward_args': _lib.BackwardArgs,
               'bdm_decode_args': _lib.DecodeArgs, 'bdm_decode_fused_args': _lib.DecodeFusedArgs,
               'bdm_controller_args': _lib.ControllerArgs,
               'bdm_output_args': _lib.OutputArgs, 'bdm_gemv_args': _lib.GemvArgs,
               'bdm_adamw_tensor': _lib.AdamwTensor, 'bdm_adamw_args': _lib.AdamwArgs,
               'bdm_route_dispatch_args': _lib.RouteDispatchArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void) {']
    for struct, mirror in mirrors.items():
        lines.append(f'printf("{struct} size %zu\\n", sizeof({struct}));')
        for field, _ in mirror._fields_:
            lines.append(f'printf("{struct} {field} %zu\\n", offsetof({struct}, {field}));')
    lines.append('return 0; }')
    src = tmp_path / 'layout.c'
    src.write_text('\n'.join(lines))
    exe = tmp_path / 'layout'
    subprocess.run([gcc, str(src), '-o', str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split('\n')
    got = {tuple(line.split()[:2]): int(line.split()[2]) for line in out if line}
    for struct, mirror in mirrors.items():
        assert got[(struct, 'size')] == ctypes.sizeof(mirror), struct
        for field, _ in mirror._fields_:
            assert got[(struct, field)] == getattr(mirror, field).offset, (struct, field)


def test_dispatch_workspace_sizes(lib):
    """The LDS-mask path's bucket counts up to 8192 banks; above that only the
    sort path's size (keys, values, sort scratch) is defined."""
    assert lib.bdm_dispatch_workspace_size(2, 64, 256) == 2 * (2 + 1) * 256 * 4
    assert lib.bdm_dispatch_workspace_size_ex(2, 64, 256, 8, 8) == lib.bdm_dispatch_workspace_size(2, 64, 256)
    assert lib.bdm_dispatch_workspace_size(1, 64, 16384) == 0
    events = 64 * 16
    assert lib.bdm_dispatch_workspace_size_ex(1, 64, 16384, 8, 8) >= events * (2 * 8 + 2 * 4)


def test_adamw_rejects_bad_arguments(lib):
    from bdm_amd import _lib
    assert lib.bdm_adamw_step(None, None) == -1
    args = _lib.AdamwArgs()
    args.blocks, args.chunk, args.tensor_count, args.step = 1, 6, 1, 1.0  # chunk not a multiple of 4
    assert lib.bdm_adamw_step(ctypes.byref(args), None) == -1
    assert b'block table' in lib.bdm_last_error_string()
    args.chunk = 8
    assert lib.bdm_adamw_step(ctypes.byref(args), None) == -1
    assert b'null pointer' in lib.bdm_last_error_string()
    args.blocks = 0
    assert lib.bdm_adamw_step(ctypes.byref(args), None) == 0  # nothing to update: no launch


def test_epilogues_reject_bad_arguments(lib):
    from bdm_amd import _lib
    assert lib.bdm_controller_epilogue(None, None) == -1
    args = _lib.ControllerArgs()
    args.tokens, args.heads, args.bank_size, args.head_width = 4, 2, 8, 64
    args.proj_stride, args.f_stride = 100, 16
    args.ctrl_dtype = args.param_dtype = _lib.BDM_BF16
    args.q_col, args.k_col, args.b_col, args.v_col, args.w_col = 0, 16, 32, 48, 60  # w runs past the row
    assert lib.bdm_controller_epilogue(ctypes.byref(args), None) == -1
    assert b'outside the projection row' in lib.bdm_last_error_string()
    args.proj_stride = 300
    assert lib.bdm_controller_epilogue(ctypes.byref(args), None) == -1  # null operands
    args.bank_size = 12
    args.proj_stride = 400
    assert lib.bdm_controller_epilogue(ctypes.byref(args), None) == -1  # null checked before the S template
    out = _lib.OutputArgs()
    out.tokens, out.width, out.gate_stride = 4, 100, 100  # width not a multiple of 8
    out.ctrl_dtype = out.param_dtype = _lib.BDM_BF16
    assert lib.bdm_output_epilogue(ctypes.byref(out), None) == -1
    out.width, out.gate_stride, out.norm_kind = 128, 128, 2
    assert lib.bdm_output_epilogue(ctypes.byref(out), None) == -1
