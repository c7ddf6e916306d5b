"""Writes ``cow_memory.json``: a small slice of the reference's published
copy-on-write memory measurements (data/trained-bsdm-memory.json), kept as the
known answers for the state-byte arithmetic of ``bdm_amd.occupancy``.

The source is a JSON data file, read with ``json``; nothing of the reference
is imported or run.  Kept: the configuration numbers the arithmetic uses,
every per-request byte record, every nested-prefix byte record, and for two
test-split rows of each arm the per-request, per-layer written-bank counts
with the fractions and bytes derived from them.

Usage:  python tests/golden/make_cow_golden.py [/root/reference/data/trained-bsdm-memory.json]
"""

from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CONFIG_KEYS = ('layers', 'width', 'bank_count', 'bank_size', 'selected_banks', 'memory_rows')


def main(source: str) -> None:
    with open(source) as f:
        data = json.load(f)
    out = {
        'configuration': {k: data['configuration'][k] for k in CONFIG_KEYS},
        'accessed_rows': data['accessed_rows'],
        'element_bytes': data['element_bytes'],
        'requests': data['requests'],
        'prefixes': data['prefixes'],
        'rows': [],
    }
    for arm in data['arms']:
        for row in arm['splits']['test'][:2]:
            out['rows'].append({
                'elastic_coefficient': arm['elastic_coefficient'],
                'id': row['id'],
                'sequence_length': row['sequence_length'],
                'bank_fraction': row['bank_fraction'],
                'bank_value_bytes': row['bank_value_bytes'],
                'written_banks_by_request_and_layer': row['written_banks_by_request_and_layer'],
                'prefixes': row['prefixes'],
            })
    with open(os.path.join(HERE, 'cow_memory.json'), 'w') as f:
        json.dump(out, f, separators=(',', ':'))


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference/data/trained-bsdm-memory.json')
