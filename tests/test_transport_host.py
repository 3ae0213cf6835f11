"""Host side of the recall transport (no GPU): liblazyrecall_recall.so loads and exports every
symbol include/lazyrecall_recall.h declares, with the loader's table matching the header; the
ring refuses a bad configuration before touching HIP; the eviction batch order (distinct slots
in (layer, head, position) order, as the reference packs them, transport.py:141-167) equals a
plain restatement with Python sets and sorted()."""

import re
from pathlib import Path

import numpy as np
import pytest

from code_for_iclr27_amd import transport

HEADER = Path(__file__).resolve().parents[1] / "include" / "lazyrecall_recall.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lrr_\w+)\s*\(", text, re.M)))


def test_ring_library_exports_header():
    library = transport.load()
    assert declared_symbols() == sorted(transport.SIGNATURES)
    for name in declared_symbols():
        assert hasattr(library, name), name


def test_ring_refuses_bad_configuration_without_hip():
    library = transport.load()
    assert not library.lrr_create(0, 8, 128, 4, 2, 64, 32, 1024, 2, 0, *([None] * 10))
    assert "Invalid recall configuration" in library.lrr_last_error().decode()
    assert not library.lrr_create(2, 2, 128, 4, 2, 64, 4, 1024, 2, 0, *([None] * 10))
    assert "Invalid recall configuration" in library.lrr_last_error().decode()  # results < L*H*topk
    assert not library.lrr_create(2, 2, 128, 4, 2, 64, 16, 1024, 2, 0, *([None] * 10))
    assert "Invalid recall staging buffers" in library.lrr_last_error().decode()


def test_configuration_checks_match_reference():
    with pytest.raises(ValueError, match="Invalid recall configuration"):
        transport.RecallTransport(2, 3, 8, 64)
    with pytest.raises(ValueError, match="Invalid recall configuration"):
        transport.RecallTransport(2, 2, 8, 64, topk=0)


@pytest.mark.parametrize("seed", range(5))
def test_batch_order_and_dedup(seed):
    rng = np.random.default_rng(seed)
    removals = {}
    for _ in range(rng.integers(1, 12)):
        key = (int(rng.integers(0, 6)), int(rng.integers(0, 4)))
        values = rng.integers(0, 50, rng.integers(0, 9)).tolist()
        removals[key] = values if seed % 2 else np.asarray(values, np.int64)
    expect = [(layer, head, position) for (layer, head) in sorted(removals)
              for position in sorted(set(int(p) for p in removals[(layer, head)]))]
    got = transport.RecallTransport._batch(removals)
    assert got.shape == (len(expect), 3)
    assert [tuple(int(v) for v in row) for row in got] == expect
    assert transport.RecallTransport._batch({}).shape == (0, 3)
