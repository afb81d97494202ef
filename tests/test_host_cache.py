"""Host-side pool, page-table and metadata logic (CPU, no kernels).

Mirrors the reference's tests/test_paged_attention.py:59-151 and :260-263: the same
scenarios and known-answer metadata values, driving ``prepare``/``advance`` directly
because attention itself only runs on the GPU here.
"""

from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import (
    KVPagePool,
    PackedBatchCache,
    PagedBatchCache,
    PagedKVCache,
    _validate_attention_inputs,
)


def tiny_config() -> Qwen3Config:
    # Same shape as the reference's tests (tests/test_paged_attention.py:18-29).
    return Qwen3Config(vocab_size=64, context_length=512, hidden_size=16, n_heads=2, n_layers=2,
                       hidden_dim=32, head_dim=8, n_kv_heads=1, dtype=torch.float32)


@pytest.fixture
def pool():
    return KVPagePool(tiny_config(), 6, device=torch.device("cpu"))


def step(caches, tokens):
    batch = PagedBatchCache(caches)
    batch.prepare(tokens)
    batch.advance(tokens)
    return batch


def test_pool_validation_and_sizes():
    cfg = tiny_config()
    with pytest.raises(ValueError):
        KVPagePool(cfg, 0, device="cpu")
    with pytest.raises(ValueError):
        KVPagePool(cfg, 2, device="cpu", page_size=128)
    p = KVPagePool(cfg, 3, device="cpu")
    assert p.keys[0].shape == (3, 256, 1, 8) and len(p.keys) == len(p.values) == 2
    assert p.bytes_per_token == 2 * 2 * 1 * 8 * 4 and p.bytes_per_page == p.bytes_per_token * 256
    q = KVPagePool(Qwen3Config(n_layers=1), 1, device="meta")
    assert q.bytes_per_token == 4096  # 8 kv heads x 128 x bf16 x (K, V) for one layer


def test_release_inside_acquire_loses_no_page(pool):
    """A page released while ``acquire`` runs (the garbage collector can run a handle's
    finaliser at any allocation, also between acquire's read of the free stack and its
    update) is neither lost nor handed out twice, and comes back first afterwards."""
    held = pool.acquire(3)
    victim = [held.pop()]            # page 2: the only reference left is in this list
    fired = []

    class Trap(np.ndarray):
        def __getitem__(self, key):  # acquire's read of the free stack
            if victim:
                victim.pop()         # drops the last reference: the release runs now
                fired.append(True)
            return np.ndarray.__getitem__(self, key)

    pool._stack = pool._stack.view(Trap)
    got = pool.acquire(2)
    pool._stack = np.asarray(pool._stack)
    assert fired, "the release ran inside acquire"
    ids = [p.index for p in held + got]
    assert ids == [0, 1, 3, 4] and len(set(ids)) == len(ids)
    assert pool.free_pages + len(ids) == 6
    assert [p.index for p in pool.acquire(1)] == [2]   # the id released last comes back first


def test_free_list_is_lifo_from_page_zero(pool):
    pages = pool.acquire(3)
    assert [p.index for p in pages] == [0, 1, 2]
    with pytest.raises(RuntimeError):
        pool.acquire(4)
    with pytest.raises(ValueError):
        pool.acquire(-1)
    del pages
    gc.collect()
    assert pool.free_pages == 6


def test_page_boundary_allocates_the_next_256_token_page(pool):
    # reference tests/test_paged_attention.py:59-74
    cache = PagedKVCache(pool, 512)
    step([cache], 256)
    assert cache.length == 256 and len(cache.pages) == 1
    first = cache.pages[0].index
    step([cache], 1)
    assert cache.length == 257 and len(cache.pages) == 2
    assert cache.pages[0].index == first and cache.pages[1].index != first


def test_released_page_is_reused_in_a_noncontiguous_batch(pool):
    # reference tests/test_paged_attention.py:76-95
    first, survivor = PagedKVCache(pool, 512), PagedKVCache(pool, 512)
    step([first, survivor], 1)
    released, survivor_page = first.pages[0].index, survivor.pages[0].index
    first.close()
    replacement = PagedKVCache(pool, 512)
    step([replacement], 1)
    assert replacement.pages[0].index == released and survivor_page != released


def test_mixed_lengths_metadata_known_answers(pool):
    # reference tests/test_paged_attention.py:97-118
    short, long = PagedKVCache(pool, 512), PagedKVCache(pool, 512)
    step([short], 3)
    step([long], 7)
    batch = PagedBatchCache([short, long])
    batch.prepare(1)
    for t in (batch.block_table, batch.seqused_k, batch.cu_seq_q, batch.cu_seq_k):
        assert t.dtype == torch.int32
    assert batch.write_slots.dtype == torch.int64
    assert batch.seqused_k.tolist() == [4, 8]
    assert batch.cu_seq_q.tolist() == [0, 1, 2]
    assert batch.cu_seq_k.tolist() == [0, 4, 12]
    s0, s1 = short.pages[0].index, long.pages[0].index
    assert batch.write_slots.tolist() == [s0 * 256 + 3, s1 * 256 + 7]
    assert batch.block_table.tolist() == [[s0, 0], [s1, 0]]
    assert (batch.max_q, batch.max_k) == (1, 8)
    batch.advance(1)
    assert (short.length, long.length) == (4, 8)


def test_prefill_metadata_known_answers(pool):
    # reference tests/test_paged_attention.py:256-263 (two caches, prepare(2))
    caches = [PagedKVCache(pool, 512), PagedKVCache(pool, 512)]
    batch = PagedBatchCache(caches)
    batch.prepare(2)
    assert batch.cu_seq_q.tolist() == [0, 2, 4]
    assert batch.cu_seq_k.tolist() == [0, 2, 4]
    assert batch.seqused_k.tolist() == [2, 2]


def test_full_page_snapshot_survives_close_and_restores_shared(pool):
    # reference tests/test_paged_attention.py:120-151 (host side)
    cache = PagedKVCache(pool, 512)
    step([cache], 256)
    snapshot = cache.snapshot_block(0, 256)
    page_index = snapshot.pages[0].index
    cache.close()
    assert pool.free_pages == pool.num_pages - 1
    restored, sibling = PagedKVCache(pool, 512), PagedKVCache(pool, 512)
    restored.restore_blocks([snapshot])
    sibling.restore_blocks([snapshot])
    assert restored.length == 256 and restored.pages[0] is sibling.pages[0]
    assert restored.pages[0].index == page_index
    step([restored, sibling], 1)
    assert restored.pages[1].index != sibling.pages[1].index
    del snapshot
    restored.close()
    assert pool.free_pages == pool.num_pages - 2
    sibling.close()
    gc.collect()
    assert pool.free_pages == pool.num_pages


def test_snapshot_and_restore_validation(pool):
    cache = PagedKVCache(pool, 512)
    step([cache], 300)
    with pytest.raises(ValueError):
        cache.snapshot_block(0, 300)
    with pytest.raises(ValueError):
        cache.snapshot_block(0, 512)
    with pytest.raises(ValueError):
        cache.snapshot_block_slot(1, 0, 256)
    snap = cache.snapshot_block(0, 256)
    with pytest.raises(RuntimeError):
        cache.restore_blocks([snap])  # not empty
    small = PagedKVCache(pool, 100)
    with pytest.raises(ValueError):
        small.restore_blocks([snap])
    cache.truncate(100)
    assert cache.length == 100 and len(cache.pages) == 1
    with pytest.raises(ValueError):
        cache.truncate(200)


def test_prepare_errors_and_pending_protocol(pool):
    cache = PagedKVCache(pool, 10)
    batch = PagedBatchCache([cache])
    with pytest.raises(ValueError):
        batch.prepare(0)
    with pytest.raises(ValueError):
        batch.prepare(11)
    batch.prepare(4)
    with pytest.raises(RuntimeError):
        batch.prepare(1)
    with pytest.raises(RuntimeError):
        batch.advance(3)
    batch.advance(4)
    assert cache.length == 4
    with pytest.raises(ValueError):
        PagedBatchCache([])
    with pytest.raises(ValueError):
        PagedBatchCache([cache, cache])
    other = KVPagePool(tiny_config(), 2, device="cpu")
    with pytest.raises(ValueError):
        PagedBatchCache([cache, PagedKVCache(other, 10)])


def test_pool_exhaustion_is_reported_before_allocation():
    p = KVPagePool(tiny_config(), 2, device="cpu")
    caches = [PagedKVCache(p, 512), PagedKVCache(p, 512)]
    batch = PagedBatchCache(caches)
    with pytest.raises(RuntimeError):
        batch.prepare(300)  # needs 4 pages
    assert p.free_pages == 2 and all(not c.pages for c in caches)


def test_block_table_reupload_only_on_change(pool):
    caches = [PagedKVCache(pool, 512)]
    batch = PagedBatchCache(caches)
    batch.prepare(1)
    table = batch.block_table
    batch.advance(1)
    batch.prepare(1)
    assert batch.block_table is table
    batch.advance(1)


def test_packed_metadata_closed_forms(pool):
    a, b, c = PagedKVCache(pool, 512), PagedKVCache(pool, 512), PagedKVCache(pool, 512)
    step([a], 250)
    step([b], 3)
    packed = PackedBatchCache([a, b, c])
    packed.prepare_packed([10, 1, 5], logit_counts=[2, 1, 5])
    assert packed.cu_seq_q.tolist() == [0, 10, 11, 16]
    assert packed.seqused_k.tolist() == [260, 4, 5]
    assert packed.cu_seq_k.tolist() == [0, 260, 264, 269]
    assert packed.positions.shape == (1, 16)
    assert packed.positions[0].tolist() == list(range(250, 260)) + [3] + list(range(5))
    assert packed.logit_indices.tolist() == [8, 9, 10, 11, 12, 13, 14, 15]
    pa = [p.index for p in a.pages]
    expected = [pa[pos // 256] * 256 + pos % 256 for pos in range(250, 260)]
    expected += [b.pages[0].index * 256 + 3] + [c.pages[0].index * 256 + i for i in range(5)]
    assert packed.write_slots.tolist() == expected
    assert len(a.pages) == 2 and (packed.max_q, packed.max_k) == (10, 260)
    with pytest.raises(ValueError):
        packed.prepare_packed([1, 1, 1])  # pending
    packed.advance_packed()
    assert (a.length, b.length, c.length) == (260, 4, 5)
    with pytest.raises(ValueError):
        PackedBatchCache([a]).prepare_packed([0])
    with pytest.raises(ValueError):
        PackedBatchCache([a]).prepare_packed([3], logit_counts=[4])


def test_attend_has_no_cpu_fallback(pool):
    cache = PagedKVCache(pool, 512)
    batch = PagedBatchCache([cache])
    batch.prepare(1)
    q = torch.randn(1, 2, 1, 8)
    k = torch.randn(1, 1, 1, 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        batch.attend(0, q, k, k.clone())


def test_validate_attention_inputs_errors(pool):
    batch = PagedBatchCache([PagedKVCache(pool, 512)])
    q, k = torch.randn(1, 2, 3, 8), torch.randn(1, 1, 3, 8)
    assert _validate_attention_inputs(batch, 0, q, k, k) == 3
    with pytest.raises(ValueError):
        _validate_attention_inputs(batch, 2, q, k, k)
    with pytest.raises(ValueError):
        _validate_attention_inputs(batch, 0, torch.randn(1, 3, 3, 8), k, k)
    with pytest.raises(ValueError):
        _validate_attention_inputs(batch, 0, q, k, torch.randn(1, 1, 2, 8))


def test_pool_is_one_allocation_of_contiguous_layer_views():
    cfg = tiny_config()
    p = KVPagePool(cfg, 3, device="cpu")
    base = p.storage.data_ptr()
    layer_bytes = 3 * 256 * 1 * 8 * 4
    for layer in range(cfg.n_layers):
        assert p.keys[layer].is_contiguous() and p.values[layer].is_contiguous()
        assert p.keys[layer].data_ptr() == base + layer * layer_bytes
        assert p.values[layer].data_ptr() == base + (cfg.n_layers + layer) * layer_bytes
    p.keys[1][2].fill_(5.0)
    assert bool((p.storage[0, 1, 2] == 5.0).all())


def test_released_ids_come_back_last_in_first_out(pool):
    a, b, c = pool.acquire(3)
    assert [a.index, b.index, c.index] == [0, 1, 2]
    del b
    del a
    # 0 was released last, so it comes back first; then 1; then the untouched 3, 4, 5
    assert [p.index for p in pool.acquire(4)] == [0, 1, 3, 4]


def test_metadata_reuses_the_tensor_and_uploads_on_change(pool):
    batch = PagedBatchCache([PagedKVCache(pool, 512)])
    t = batch.metadata("token_ids", [5, 6, 7], torch.long)
    assert t.dtype == torch.int64 and t.tolist() == [5, 6, 7]
    assert batch.metadata("token_ids", [5, 6, 7], torch.long) is t
    assert batch.metadata("token_ids", [5, 6, 8], torch.long) is t and t.tolist() == [5, 6, 8]
    u = batch.metadata("token_ids", [1, 2], torch.long)
    assert u.tolist() == [1, 2]
    grid = batch.metadata("grid", [[1, 2, 3], [4, 5, 6]], torch.int32)
    assert grid.shape == (2, 3) and grid.dtype == torch.int32 and grid.tolist() == [[1, 2, 3], [4, 5, 6]]


def test_batch_object_reused_with_other_caches(pool):
    # The reference's decoder keeps one batch object and reassigns caches / batch_size
    # every tick (decode.py:235-241, :278-281).
    caches = [PagedKVCache(pool, 512) for _ in range(3)]
    batch = PagedBatchCache(caches[:1])
    for rows in (caches[:1], caches, caches[1:], caches):
        batch.caches, batch.batch_size = tuple(rows), len(rows)
        batch.prepare(1)
        lengths = [c.length for c in rows]
        assert batch.seqused_k.tolist() == [n + 1 for n in lengths]
        assert batch.cu_seq_q.tolist() == list(range(len(rows) + 1))
        assert batch.write_slots.tolist() == [c.pages[0].index * 256 + n for c, n in zip(rows, lengths)]
        assert batch.block_table.shape == (len(rows), 2)
        batch.advance(1)
    assert [c.length for c in caches] == [3, 3, 3]


def test_packed_batch_reused_with_other_caches(pool):
    caches = [PagedKVCache(pool, 512) for _ in range(3)]
    batch = PackedBatchCache(caches)
    batch.prepare_packed([2, 3, 1], logit_counts=[1, 3, 1])
    assert batch.logit_indices.tolist() == [1, 2, 3, 4, 5]
    batch.advance_packed()
    batch.caches, batch.batch_size = (caches[2], caches[0]), 2
    batch.prepare_packed([4, 1])
    assert batch.cu_seq_q.tolist() == [0, 4, 5]
    assert batch.seqused_k.tolist() == [5, 3]
    assert batch.positions[0].tolist() == [1, 2, 3, 4, 2]
    assert batch.logit_indices.tolist() == [3, 4]
    batch.advance_packed()
    assert [c.length for c in caches] == [3, 3, 5]


def test_copying_restore_needs_a_device_pool(pool):
    cache = PagedKVCache(pool, 512)
    step([cache], 256)
    snap = cache.snapshot_block(0, 256)
    other = PagedKVCache(pool, 512)
    with pytest.raises(RuntimeError, match="ROCm device"):
        other.restore_blocks([snap], copy=True)
