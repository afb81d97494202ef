"""Level choice of the shared-prefix cascade (host logic, no GPU): the dynamic program
against brute force over every set of at most three boundaries, and the levels a batch
of page tables yields."""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PagedBatchCache, PagedKVCache, _PrefixCascade as PC


def _cost(shared, bounds):
    total, prev = 0.0, 0
    for b in bounds:
        c = sum(1 for s in shared if s >= b)
        if c < PC.MIN_GROUP:
            return float("inf")
        total += -(-c // 64) * (b - prev) * PC.US_PER_BLOCK_PAGE + PC.US_PER_LEVEL
        prev = b
    edges = [0, *bounds]
    for s in shared:
        total += (s - max(e for e in edges if e <= s)) * PC.US_PER_PAGE_READ
    return total


@pytest.mark.parametrize("seed", range(12))
def test_boundaries_are_optimal(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(2, 200))
    top = int(rng.integers(1, 24))
    shared = [int(x) for x in rng.integers(0, top + 1, rows)]
    got = PC._boundaries(shared)
    cand = sorted({s for s in shared if s > 0})
    options = [()] + [c for k in range(1, PC.MAX_LEVELS + 1) for c in itertools.combinations(cand, k)]
    best = min(_cost(shared, c) for c in options)
    assert got == sorted(got) and len(got) <= PC.MAX_LEVELS
    assert _cost(shared, got) == pytest.approx(best)


def test_boundaries_edge_cases():
    assert PC._boundaries([]) == []
    assert PC._boundaries([0, 0, 0]) == []
    assert PC._boundaries([40]) == []            # one row shares with nobody
    # three rows reading 40 pages each cost about what one padded 64-row level does; six
    # rows make the level pay off
    assert PC._boundaries([40] * 6) == [40]


def test_levels_from_page_tables():
    config = Qwen3Config(context_length=8192, n_layers=1)
    pool = KVPagePool(config, 200, device="cpu")
    prefix = pool.acquire(30)
    caches = []
    specs = [(30, 7800 + 10 * i) for i in range(8)] + [(12, 3300 + 100 * i) for i in range(6)] + [(0, 900)]
    for n_shared, length in specs:
        cache = PagedKVCache(pool, 8192)
        cache.pages.extend(prefix[:n_shared])
        cache.pages.extend(pool.acquire(-(-length // 256) - n_shared))
        cache.length = length
        caches.append(cache)
    batch = PagedBatchCache(caches, device_metadata=False, prefix_cascade=False)
    levels = PC.levels(batch, [1] * len(caches))
    assert [(first, end) for _, first, end, _ in levels] == [(0, 12), (12, 30)]
    assert levels[0][3] == list(range(14)) and levels[1][3] == list(range(8))
    assert all(ref in range(8) for ref, _, _, _ in levels)
    # a chunk row (more than one query) never joins a level; the unshared row never does
    q_lens = [1] * len(caches)
    q_lens[2] = 5
    assert all(2 not in rows and 14 not in rows for _, _, _, rows in PC.levels(batch, q_lens))
