"""bank_occupancy on the GPU against the oracle restatement of
elastic_bank_regularizer.py:10-25 (pinned in test_oracle_invariants.py).

hard must be exact (it is a count); soft and the gradient agree to FP32
summation order (the GPU sums a bank's writes with a wave reduction, the
oracle in token order).  Two runs are bit-identical (no atomics)."""

import sys

import pytest
import torch

from _inputs import rel_err, routes
from oracle import bdm_oracle as O

pytestmark = pytest.mark.gpu


def announce(*what):
    print('CASE', *what, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize('masked', [False, True], ids=['all', 'valid'])
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32], ids=['bf16', 'f32'])
def test_bank_occupancy_matches_oracle(device, masked, dtype):
    from bdm_amd import bank_occupancy
    gen = torch.Generator().manual_seed(17)
    batch, time, banks, k = 3, 300, 256, 8
    _, weights, indices = routes(batch, time, banks, k, gen, dtype=dtype)
    weights = (weights.float() * 3).clamp(0, 1).to(dtype)  # some weights at the clamp
    valid = torch.rand(batch, time, generator=gen) < 0.6 if masked else None
    announce('occupancy', dtype, masked)
    ref_value, ref_hard, ref_soft = O.bank_occupancy(weights.detach().clone().float(), indices, banks, valid)
    wd = weights.detach().clone().to(device).requires_grad_(True)
    value, hard, soft = bank_occupancy(wd, indices.to(device), banks, None if valid is None else valid.to(device))
    (value * torch.arange(1, batch + 1, device=device)).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(hard.cpu(), ref_hard)
    assert rel_err(soft, ref_soft) < 1e-5 and rel_err(value, ref_value) < 1e-5
    wr = weights.detach().clone().float().requires_grad_(True)
    rv, _, _ = O.bank_occupancy(wr, indices, banks, valid)
    (rv * torch.arange(1, batch + 1)).sum().backward()
    assert rel_err(wd.grad, wr.grad) < (1e-2 if dtype == torch.bfloat16 else 1e-4)


def test_bank_occupancy_is_deterministic(device):
    from bdm_amd import ops
    gen = torch.Generator().manual_seed(18)
    _, weights, indices = routes(2, 2000, 2048, 8, gen)
    announce('occupancy determinism')
    runs = [ops.bank_occupancy_totals(weights.to(device), indices.to(device), 2048) for _ in range(2)]
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize('masked', [False, True], ids=['all', 'valid'])
def test_written_banks_match_oracle(device, masked):
    """First-write positions and the written-bank curve (the copy-on-write
    state count) equal the oracle exactly, prefixes past the end included."""
    from bdm_amd import ops, written_banks
    gen = torch.Generator().manual_seed(19)
    batch, time, banks, k = 3, 300, 256, 8
    _, weights, indices = routes(batch, time, banks, k, gen)
    valid = torch.rand(batch, time, generator=gen) < 0.5 if masked else None
    prefixes = [0, 1, 7, 150, 299, 300, 1000]
    announce('written banks', masked)
    vd = None if valid is None else valid.to(device)
    _, counts, first = ops.bank_occupancy_totals(weights.to(device), indices.to(device), banks, vd, first_write=True)
    curve = written_banks(indices.to(device), banks, prefixes, vd)
    torch.cuda.synchronize()
    assert torch.equal(first.cpu(), O.first_write_positions(indices, banks, valid))
    assert torch.equal(curve.cpu(), O.written_bank_curve(indices, banks, prefixes, valid))
    assert torch.equal(curve[:, -1].cpu(), (counts > 0).sum(1).int().cpu())


def test_written_banks_memory_study_shape(device):
    """The reference memory study's geometry (J = 2048, K = 8, 16k positions)
    at its measured prefixes: exact against the oracle, K banks after one
    token, never above min(J, K t)."""
    from bdm_amd import written_banks
    gen = torch.Generator().manual_seed(20)
    batch, time, banks, k = 4, 16384, 2048, 8
    _, _, indices = routes(batch, time, banks, k, gen)
    prefixes = [1, 8, 32, 128, 512, 1008, 1024, 4096, 16368, 16384]
    announce('written banks 16k')
    curve = written_banks(indices.to(device), banks, prefixes).cpu()
    assert torch.equal(curve, O.written_bank_curve(indices, banks, prefixes))
    assert torch.all(curve[:, 0] == k)
    for i, t in enumerate(prefixes):
        assert torch.all(curve[:, i] <= min(banks, k * t))
