"""Copy-on-write state accounting against the reference's published memory
measurements (data/trained-bsdm-memory.json, sliced into
tests/golden/cow_memory.json by make_cow_golden.py).

The identities are the ones scripts/verify_results.py:190-235 asserts for
that file; here they pin ``bdm_amd.occupancy``'s byte functions: dense state,
the copy-on-write ceiling min(N, K n) L D b, the attention KV comparison
2 n L D b, and the bytes and fractions of measured written-bank counts."""

import json
import os

import pytest

from conftest import ROOT

GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'cow_memory.json')


@pytest.fixture(scope='module')
def data():
    with open(GOLDEN) as f:
        return json.load(f)


def close(a, b):
    return a == pytest.approx(b, rel=1e-6, abs=1e-6)


def test_request_bytes(data):
    from bdm_amd import occupancy as occ
    c, eb = data['configuration'], data['element_bytes']
    dense = occ.dense_state_bytes(c['layers'], c['memory_rows'], c['width'], eb)
    assert dense == 32 * 2**20
    assert data['accessed_rows'] == c['selected_banks'] * c['bank_size']
    for p in data['requests'] + data['prefixes']:
        h = p['history_positions']
        assert p['dense_sdm_bsdm_bytes'] == dense
        assert p['attention_kv_bytes'] == occ.attention_kv_bytes(h, c['layers'], c['width'], eb)
        assert p['cow_worst_case_bytes'] == occ.cow_worst_case_bytes(
            c['memory_rows'], data['accessed_rows'], h, c['layers'], c['width'], eb)
        # measured copy-on-write bytes never exceed the ceiling
        assert p['cow_bytes'] <= p['cow_worst_case_bytes'] and p['elastic_cow_bytes'] <= p['cow_worst_case_bytes']
    for p in data['requests']:
        assert p['history_positions'] == p['request_positions'] - 16


def test_measured_banks_to_bytes(data):
    from bdm_amd import occupancy as occ
    c, eb = data['configuration'], data['element_bytes']
    assert len(data['rows']) == 4
    for row in data['rows']:
        banks = row['written_banks_by_request_and_layer']
        assert len(banks) == 64 and all(len(x) == c['layers'] for x in banks)
        assert all(c['selected_banks'] <= b <= c['bank_count'] for x in banks for b in x)
        mean = sum(map(sum, banks)) / len(banks)
        assert close(row['bank_fraction'], mean / (c['layers'] * c['bank_count']))
        assert close(row['bank_value_bytes'], occ.state_value_bytes(mean, c['bank_size'], c['width'], eb))
        for p in row['prefixes']:
            fraction = sum(p['per_layer_bank_fraction']) / c['layers']
            assert close(p['bank_fraction'], fraction)
            banks_held = fraction * c['layers'] * c['bank_count']
            assert close(p['bank_value_bytes'], occ.state_value_bytes(banks_held, c['bank_size'], c['width'], eb))


def test_first_token_writes_k_banks(data):
    """The first position of every request and layer holds exactly the K
    distinct banks its write route selects."""
    c = data['configuration']
    for row in data['rows']:
        first = next(p for p in row['prefixes'] if p['tokens'] == 1)
        for f in first['per_layer_bank_fraction']:
            assert close(f, c['selected_banks'] / c['bank_count'])
