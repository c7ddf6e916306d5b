"""The allocation-free dispatch, bdm_dispatch_build_static, through the C ABI.

It must give the outputs of bdm_dispatch_build (same permutation, inverse,
tokens, segment bounds and route flags) bit for bit, on consecutive calls that
share its static scratch (the second call smaller than the first), and reject
geometries its fixed scratch cannot hold with an error and a message.
"""

import ctypes
import sys

import pytest
import torch

from _inputs import routes

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


def _outputs(batch, time, kw, kr, bank_count, device):
    events = batch * time * (kw + kr)
    return dict(order=torch.full((events,), -7, device=device, dtype=torch.int64),
                inverse=torch.full((events,), -7, device=device, dtype=torch.int64),
                tokens=torch.full((events,), -7, device=device, dtype=torch.int64),
                cu=torch.full((batch * bank_count + 1,), -7, device=device, dtype=torch.int64),
                status=torch.full((1,), 12345, device=device, dtype=torch.int32))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dispatch_with_workspace(wi, ri, bank_count):
    from bdm_amd import _lib
    lib = _lib.library()
    batch, time, kw = wi.shape
    kr = ri.shape[-1]
    out = _outputs(batch, time, kw, kr, bank_count, wi.device)
    ws = int(lib.bdm_dispatch_workspace_size_ex(batch, time, bank_count, kw, kr))
    workspace = torch.empty(max(ws, 1), device=wi.device, dtype=torch.uint8)
    rc = lib.bdm_dispatch_build(_ptr(wi), _ptr(ri), batch, time, kw, kr, bank_count, _ptr(out['order']),
                                _ptr(out['inverse']), _ptr(out['tokens']), _ptr(out['cu']), _ptr(out['status']),
                                _ptr(workspace), ws, _stream(wi.device))
    assert rc == 0, lib.bdm_last_error_string()
    return out


def dispatch_static(wi, ri, bank_count):
    from bdm_amd import _lib
    lib = _lib.library()
    batch, time, kw = wi.shape
    kr = ri.shape[-1]
    out = _outputs(batch, time, kw, kr, bank_count, wi.device)
    rc = lib.bdm_dispatch_build_static(_ptr(wi), _ptr(ri), batch, time, kw, kr, bank_count, _ptr(out['order']),
                                       _ptr(out['inverse']), _ptr(out['tokens']), _ptr(out['cu']),
                                       _ptr(out['status']), _stream(wi.device))
    return rc, out


def _case(batch, time, bank_count, kk, seed, device, bad=False):
    gen = torch.Generator().manual_seed(seed)
    _, _, wi = routes(batch, time, bank_count, kk, gen)
    _, _, ri = routes(batch, time, bank_count, kk, gen)
    if bad:  # a repeated bank and an out-of-range one: both route flags
        wi[0, 1, 1] = wi[0, 1, 0]
        ri[0, 2, 0] = bank_count + 3
    return wi.to(device), ri.to(device)


def test_static_dispatch_under_graph_capture(device):
    """Captured in a HIP graph (the callers it is for), and first called
    there when this file runs alone: each replay, after new routes are copied
    into the captured inputs and with eager work in between, equals the
    workspace dispatch of those routes bit for bit."""
    from bdm_amd import _lib
    lib = _lib.library()
    batch, time, bank_count, kk = 8, 4096, 256, 8
    wi, ri = _case(batch, time, bank_count, kk, 11, device)
    out = _outputs(batch, time, kk, kk, bank_count, device)
    torch.cuda.synchronize()
    announce('static dispatch under graph capture')
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.bdm_dispatch_build_static(_ptr(wi), _ptr(ri), batch, time, kk, kk, bank_count, _ptr(out['order']),
                                           _ptr(out['inverse']), _ptr(out['tokens']), _ptr(out['cu']),
                                           _ptr(out['status']), _stream(device))
    assert rc == 0, lib.bdm_last_error_string()
    for replay, seed in enumerate((12, 13, 14)):
        new_wi, new_ri = _case(batch, time, bank_count, kk, seed, device)
        wi.copy_(new_wi)
        ri.copy_(new_ri)
        for t in out.values():
            t.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        want = dispatch_with_workspace(new_wi, new_ri, bank_count)
        torch.cuda.synchronize()
        for key in ('order', 'inverse', 'tokens', 'cu', 'status'):
            assert torch.equal(out[key], want[key]), (replay, key)
    del graph


def test_static_dispatch_matches_the_workspace_dispatch(device):
    # the C2 geometry, then a smaller one on the same (reused) static scratch,
    # then malformed routes, then the C2 geometry again
    for name, seed, (batch, time, bank_count, kk, bad) in (('C2', 1, (8, 4096, 256, 8, False)),
                                                             ('smaller', 2, (2, 300, 64, 4, False)),
                                                             ('bad routes', 3, (1, 40, 16, 4, True)),
                                                             ('C2 again', 4, (8, 4096, 256, 8, False))):
        announce('static dispatch', name)
        wi, ri = _case(batch, time, bank_count, kk, seed, device, bad)
        rc, got = dispatch_static(wi, ri, bank_count)
        from bdm_amd import _lib
        assert rc == 0, _lib.library().bdm_last_error_string()
        want = dispatch_with_workspace(wi, ri, bank_count)
        torch.cuda.synchronize()
        for key in ('order', 'inverse', 'tokens', 'cu', 'status'):
            assert torch.equal(got[key], want[key]), (name, key)
        if bad:
            assert int(got['status'].item()) == 3  # out of range | duplicate
        else:
            assert int(got['status'].item()) == 0


def test_static_dispatch_rejects_what_its_scratch_cannot_hold(device):
    from bdm_amd import _lib
    lib = _lib.library()
    announce('static dispatch limits')
    # more banks than the LDS-mask path: the radix sort needs a workspace
    wi, ri = _case(1, 8, 9000, 4, 1, device)
    rc, _ = dispatch_static(wi, ri, 9000)
    assert rc == -2 and b'radix-sort' in lib.bdm_last_error_string()  # BDM_ERR_UNSUPPORTED
    # per-tile counts beyond the static buffer: batch 8 x 2049 tiles x 256 banks x 4 B > 16 MiB
    wi = torch.zeros(8, 65536, 1, dtype=torch.int64, device=device)
    ri = torch.zeros(8, 65536, 1, dtype=torch.int64, device=device)
    rc, _ = dispatch_static(wi, ri, 256)
    assert rc == -2 and b'static buffer' in lib.bdm_last_error_string()
    torch.cuda.synchronize()
