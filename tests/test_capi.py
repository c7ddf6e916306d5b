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
    # tiles of 32 tokens x banks x int32 per batch
    assert lib.bdm_dispatch_workspace_size(8, 4096, 256) == 8 * 128 * 256 * 4
    assert lib.bdm_dispatch_workspace_size(0, 4096, 256) == 0
    from bdm_amd import _lib
    args = _lib.ForwardArgs()
    args.batch, args.time, args.heads, args.head_width, args.read_banks = 2, 10, 3, 16, 4
    args.ctrl_dtype = _lib.BDM_BF16
    assert lib.bdm_forward_workspace_size(ctypes.byref(args)) == (2 * 10 * 4 * 3 * 16 * 2 + 255) // 256 * 256


def test_invalid_arguments_are_rejected_without_a_launch(lib):
    from bdm_amd import _lib
    rc = lib.bdm_router_select(None, _lib.BDM_BF16, 4, 3, 16, 16, 8, None, None, None)
    assert rc == -1 and b'bad geometry' in lib.bdm_last_error_string()
    rc = lib.bdm_router_select(None, _lib.BDM_BF16, 4, 32, 16, 16, 20, None, None, None)
    assert rc == -2
    rc = lib.bdm_dispatch_build(None, None, 1, 8, 2, 2, 16384, None, None, None, None, None, None, 0, None)
    assert rc == -2 and b'bank_count' in lib.bdm_last_error_string()
    rc = lib.bdm_forward(None, None, 0, None)
    assert rc == -1
    args = _lib.ForwardArgs()
    args.batch, args.time, args.heads, args.bank_size, args.head_width = 1, 4, 1, 64, 16
    args.bank_count, args.write_banks, args.read_banks = 4, 1, 1
    assert lib.bdm_forward(ctypes.byref(args), None, 0, None) == -2
    dargs = _lib.DecodeArgs()
    assert lib.bdm_decode(ctypes.byref(dargs), None) == -1


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
