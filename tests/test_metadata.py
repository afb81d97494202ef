"""Tick metadata: the oracle against the reference's known answers and a brute-force
walk of the page tables; the host path of the paged-cache classes against the oracle."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedBatchCache, PagedKVCache
from oracle import metadata


def brute_force(lengths, counts, tables, page_size, tails):
    """Token-by-token: lay every table out as its flat list of (page, offset) slots in
    logical order, then read slot `pos`; rows are numbered by walking the batch."""
    cu_q, cu_k, used, positions, slots, logits = [0], [0], [], [], [], []
    row = 0
    for b, (length, count) in enumerate(zip(lengths, counts)):
        flat = []
        for page in tables[b]:
            for offset in range(page_size):
                flat.append(page * page_size + offset)
        for i in range(count):
            positions.append(length + i)
            slots.append(flat[length + i])
            row += 1
        for j in range(tails[b]):
            logits.append(row - tails[b] + j)
        cu_q.append(row)
        used.append(length + count)
        cu_k.append(cu_k[-1] + length + count)
    return cu_q, cu_k, used, positions, slots, logits


def test_reference_known_answers():
    # test_paged_attention.py:97-113: lengths 3 and 7, one decode token each.
    m = metadata.tick_metadata([3, 7], [1, 1], [[0], [1]], 256)
    assert m["seqused_k"].tolist() == [4, 8]
    assert m["cu_seq_q"].tolist() == [0, 1, 2]
    assert m["cu_seq_k"].tolist() == [0, 4, 12]
    assert m["write_slots"].tolist() == [3, 256 + 7]
    # test_paged_attention.py:256-263: two fresh prefills of 2 tokens.
    m = metadata.tick_metadata([0, 0], [2, 2], [[0], [1]], 256)
    assert m["cu_seq_q"].tolist() == [0, 2, 4]
    assert m["cu_seq_k"].tolist() == [0, 2, 4]
    for key in ("cu_seq_q", "cu_seq_k", "seqused_k"):
        assert m[key].dtype == np.int32
    assert m["write_slots"].dtype == np.int64


@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_brute_force(seed):
    rng = random.Random(seed)
    page_size = rng.choice([1, 4, 16, 256])
    batch = rng.randint(1, 9)
    lengths = [rng.randint(0, 3 * page_size + 2) for _ in range(batch)]
    counts = [rng.randint(1, 2 * page_size + 3) for _ in range(batch)]
    tails = [rng.randint(1, c) for c in counts]
    pool = list(range(200))
    rng.shuffle(pool)
    tables = []
    for length, count in zip(lengths, counts):
        need = -(-(length + count) // page_size)
        tables.append([pool.pop() for _ in range(need)])
    m = metadata.tick_metadata(lengths, counts, tables, page_size, tails)
    cu_q, cu_k, used, positions, slots, logits = brute_force(lengths, counts, tables, page_size, tails)
    assert m["cu_seq_q"].tolist() == cu_q
    assert m["cu_seq_k"].tolist() == cu_k
    assert m["seqused_k"].tolist() == used
    assert m["positions"].tolist() == positions
    assert m["write_slots"].tolist() == slots
    assert m["logit_indices"].tolist() == logits


def _caches(pool, lengths):
    caches = []
    for length in lengths:
        cache = PagedKVCache(pool, 4096)
        if length:
            # Cached tokens: acquire their pages as a prefill would have.
            cache.pages.extend(pool.acquire(-(-length // pool.page_size)))
            cache.length = length
        caches.append(cache)
    return caches


@pytest.mark.parametrize("seed", range(3))
def test_host_path_matches_oracle(seed):
    rng = random.Random(100 + seed)
    config = Qwen3Config(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=8, dtype=torch.float32)
    pool = KVPagePool(config, 64, device="cpu")
    lengths = [rng.randint(0, 700) for _ in range(5)]
    counts = [rng.randint(1, 600) for _ in range(5)]
    tails = [rng.randint(1, c) for c in counts]
    caches = _caches(pool, lengths)
    batch = PackedBatchCache(caches)
    batch.prepare_packed(counts, tails)
    tables = [[p.index for p in c.pages] for c in caches]
    m = metadata.tick_metadata(lengths, counts, tables, 256, tails)
    assert batch.cu_seq_q.tolist() == m["cu_seq_q"].tolist()
    assert batch.cu_seq_k.tolist() == m["cu_seq_k"].tolist()
    assert batch.seqused_k.tolist() == m["seqused_k"].tolist()
    assert batch.positions.tolist() == [m["positions"].tolist()]
    assert batch.write_slots.tolist() == m["write_slots"].tolist()
    assert batch.logit_indices.tolist() == m["logit_indices"].tolist()
    assert batch.write_slots.dtype == torch.int64 and batch.cu_seq_q.dtype == torch.int32

    uniform = PagedBatchCache(_caches(pool, lengths[:3]))
    uniform.prepare(3)
    tables = [[p.index for p in c.pages] for c in uniform.caches]
    m = metadata.tick_metadata(lengths[:3], [3, 3, 3], tables, 256)
    assert uniform.write_slots.tolist() == m["write_slots"].tolist()
    assert uniform.cu_seq_k.tolist() == m["cu_seq_k"].tolist()


def test_device_metadata_needs_a_gpu_pool():
    config = Qwen3Config(n_layers=1, n_heads=2, n_kv_heads=1, head_dim=8, dtype=torch.float32)
    pool = KVPagePool(config, 4, device="cpu")
    with pytest.raises(ValueError):
        PagedBatchCache([PagedKVCache(pool, 512)], device_metadata=True)
