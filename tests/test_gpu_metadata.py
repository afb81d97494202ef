"""Tick metadata kernel on the GPU: bit-exact against the oracle, and the paged-cache
classes give identical tensors and attention with device and host metadata."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from helios_amd import ops
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedBatchCache, PagedKVCache
from oracle import metadata
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


def run_kernel(device, lengths, counts, tails, tables, width, page_size):
    batch = len(counts)
    seq = torch.tensor(list(lengths) + list(counts) + list(tails), dtype=torch.int32, device=device)
    bt = np.zeros((batch, width), dtype=np.int32)
    for b, t in enumerate(tables):
        bt[b, : min(len(t), width)] = t[:width]
    bt = torch.from_numpy(bt).to(device)
    total, n_logits = sum(counts), sum(tails)
    out = {
        "cu_seq_q": torch.full((batch + 1,), -7, dtype=torch.int32, device=device),
        "cu_seq_k": torch.full((batch + 1,), -7, dtype=torch.int32, device=device),
        "seqused_k": torch.full((batch,), -7, dtype=torch.int32, device=device),
        "write_slots": torch.full((total,), -7, dtype=torch.int64, device=device),
        "positions": torch.full((total,), -7, dtype=torch.int64, device=device),
        "logit_indices": torch.full((max(n_logits, 1),), -7, dtype=torch.int64, device=device),
    }
    ops.tick_metadata(seq, bt, page_size, total_q=total, n_logits=n_logits, **out)
    torch.cuda.synchronize()
    out["logit_indices"] = out["logit_indices"][:n_logits]
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("case", [
    (1, 1, 1), (3, 40, 256), (64, 1, 256), (129, 9, 256), (300, 70, 256), (4096, 3, 256),
    (7, 3000, 256), (5, 50, 512),
])
def test_kernel_matches_oracle(device, case):
    batch, max_count, page_size = case
    say("tick metadata", case)
    rng = random.Random(batch * 1000 + max_count)
    lengths = [rng.randint(0, 5 * page_size) for _ in range(batch)]
    counts = [rng.randint(1, max_count) for _ in range(batch)]
    tails = [rng.randint(1, c) for c in counts]
    ids = list(range(200_000))
    rng.shuffle(ids)
    tables = []
    for length, count in zip(lengths, counts):
        need = -(-(length + count) // page_size)
        tables.append([ids.pop() for _ in range(need)])
    width = max(len(t) for t in tables) + 1
    got = run_kernel(device, lengths, counts, tails, tables, width, page_size)
    want = metadata.tick_metadata(lengths, counts, tables, page_size, tails)
    for key in ("cu_seq_q", "cu_seq_k", "seqused_k", "positions", "write_slots", "logit_indices"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)


def test_rows_past_the_table_get_slot_minus_one(device):
    say("tick metadata narrow table")
    # Sequence 0 needs 2 pages but the table is 1 wide: its second page's rows get -1.
    got = run_kernel(device, [250], [10], [1], [[5, 6]], 1, 256)
    want = [5 * 256 + p for p in range(250, 256)] + [-1] * 4
    assert got["write_slots"].tolist() == want
    assert got["positions"].tolist() == [250 + i for i in range(10)]
    assert got["cu_seq_k"].tolist() == [0, 260]


def _config():
    return Qwen3Config(context_length=4096, n_layers=2, dtype=torch.bfloat16)


def _fill(pool, seed):
    g = torch.Generator(device=pool.device).manual_seed(seed)
    for t in pool.keys + pool.values:
        t.copy_(torch.randn(t.shape, generator=g, device=pool.device, dtype=torch.float32).to(t.dtype))


def _build(pool, lengths):
    caches = []
    for length in lengths:
        cache = PagedKVCache(pool, 4096)
        if length:
            cache.pages.extend(pool.acquire(-(-length // pool.page_size)))
            cache.length = length
        caches.append(cache)
    return caches


@pytest.mark.parametrize("seed", range(3))
def test_packed_cache_device_equals_host_metadata(device, seed):
    say("packed cache metadata", seed)
    rng = random.Random(seed)
    config = _config()
    lengths = [rng.randint(0, 900) for _ in range(6)] + [0]
    counts = [1] * 4 + [rng.randint(2, 300) for _ in range(2)] + [257]
    tails = [1] * 6 + [3]
    results = []
    for device_meta in (True, False):
        pool = KVPagePool(config, 64, device=device)
        _fill(pool, 11)
        batch = PackedBatchCache(_build(pool, lengths), device_metadata=device_meta)
        batch.prepare_packed(counts, tails)
        total = sum(counts)
        g = torch.Generator(device=device).manual_seed(5)
        q = torch.randn((1, config.n_heads, total, config.head_dim), generator=g, device=device).to(config.dtype)
        k = torch.randn((1, config.n_kv_heads, total, config.head_dim), generator=g, device=device).to(config.dtype)
        v = torch.randn((1, config.n_kv_heads, total, config.head_dim), generator=g, device=device).to(config.dtype)
        out = batch.attend(0, q, k, v)
        torch.cuda.synchronize()
        results.append({
            "cu_seq_q": batch.cu_seq_q.cpu(), "cu_seq_k": batch.cu_seq_k.cpu(),
            "seqused_k": batch.seqused_k.cpu(), "positions": batch.positions.cpu(),
            "write_slots": batch.write_slots.cpu(), "logit_indices": batch.logit_indices.cpu(),
            "block_table": batch.block_table.cpu(), "out": out.cpu(),
            "pool": pool.keys[0].view(torch.int16).cpu(),
        })
        batch.advance_packed()
    dev, host = results
    for key in dev:
        assert dev[key].dtype == host[key].dtype, key
        assert dev[key].shape == host[key].shape, key
        assert torch.equal(dev[key], host[key]), key


def test_uniform_cache_device_metadata_over_ticks(device):
    say("uniform cache metadata ticks")
    config = _config()
    pool = KVPagePool(config, 64, device=device)
    _fill(pool, 3)
    twin = KVPagePool(config, 64, device=device)
    _fill(twin, 3)
    lengths = [255, 3, 511, 0]
    dev_batch = PagedBatchCache(_build(pool, lengths))
    host_batch = PagedBatchCache(_build(twin, lengths), device_metadata=False)
    g = torch.Generator(device=device).manual_seed(9)
    for tick, tokens in enumerate((1, 1, 2, 1, 1)):
        q = torch.randn((4, config.n_heads, tokens, config.head_dim), generator=g, device=device).to(config.dtype)
        k = torch.randn((4, config.n_kv_heads, tokens, config.head_dim), generator=g, device=device).to(config.dtype)
        v = torch.randn((4, config.n_kv_heads, tokens, config.head_dim), generator=g, device=device).to(config.dtype)
        outs = []
        for batch in (dev_batch, host_batch):
            batch.prepare(tokens)
            outs.append(batch.attend(1, q, k, v))
        torch.cuda.synchronize()
        for name in ("cu_seq_q", "cu_seq_k", "seqused_k", "write_slots", "block_table"):
            assert torch.equal(getattr(dev_batch, name).cpu(), getattr(host_batch, name).cpu()), (tick, name)
        assert torch.equal(outs[0], outs[1]), tick
        for batch in (dev_batch, host_batch):
            batch.advance(tokens)
    assert torch.equal(pool.keys[1].view(torch.int16), twin.keys[1].view(torch.int16))
