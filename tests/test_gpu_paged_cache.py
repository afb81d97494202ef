"""The paged_cache mirror end to end on the GPU: the reference's own scenarios
(tests/test_paged_attention.py:120-151, :240-312) at Qwen3-4B head shape."""

from __future__ import annotations

import gc

import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedBatchCache, PagedKVCache
from oracle import dense_torch
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


def config(dtype=torch.bfloat16, n_layers=2):
    return Qwen3Config(context_length=4096, n_layers=n_layers, dtype=dtype)


def dense_reference(pool, caches, query, layer=0):
    """The reference's check (tests/test_paged_attention.py:275-312) in float32 on the CPU."""
    rows = []
    for row, cache in enumerate(caches):
        tokens = query.shape[2]
        start = cache.length - tokens
        pk = torch.cat([pool.keys[layer][p.index] for p in cache.pages])[: cache.length].float().cpu()
        pv = torch.cat([pool.values[layer][p.index] for p in cache.pages])[: cache.length].float().cpu()
        dk = pk.permute(1, 0, 2).unsqueeze(0).repeat_interleave(query.shape[1] // pk.shape[1], dim=1)
        dv = pv.permute(1, 0, 2).unsqueeze(0).repeat_interleave(query.shape[1] // pv.shape[1], dim=1)
        mask = torch.arange(cache.length)[None, None, None, :] <= (start + torch.arange(tokens))[None, None, :, None]
        rows.append(torch.nn.functional.scaled_dot_product_attention(
            query[row:row + 1].float().cpu(), dk, dv, attn_mask=mask))
    return torch.cat(rows)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_varlen_matches_dense_sdpa_for_prefill_and_decode(device, dtype):
    say("batch cache prefill+decode", dtype)
    cfg = config(dtype)
    pool = KVPagePool(cfg, 8, device=device)
    caches = [PagedKVCache(pool, 1024), PagedKVCache(pool, 1024)]
    for tokens in (2, 300, 1, 1):
        q = torch.randn(2, cfg.n_heads, tokens, cfg.head_dim, device=device, dtype=dtype)
        k = torch.randn(2, cfg.n_kv_heads, tokens, cfg.head_dim, device=device, dtype=dtype)
        v = torch.randn_like(k)
        batch = PagedBatchCache(caches)
        batch.prepare(tokens)
        if tokens == 2:
            assert batch.cu_seq_q.tolist() == [0, 2, 4] and batch.cu_seq_k.tolist() == [0, 2, 4]
        out = batch.attend(0, q, k, v)
        out1 = batch.attend(1, q, k, v)  # second layer reuses the plan
        batch.advance(tokens)
        ref = dense_reference(pool, caches, q)
        torch.testing.assert_close(out.float().cpu(), ref, rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(out1.float().cpu(), ref, rtol=2e-2, atol=2e-2)


def test_packed_tick_matches_reference_dense_path(device):
    say("packed tick")
    cfg = config()
    pool = KVPagePool(cfg, 24, device=device)
    a, b, c = (PagedKVCache(pool, 2048) for _ in range(3))
    warm = PackedBatchCache([a, b])
    warm.prepare_packed([700, 40])
    for layer in range(cfg.n_layers):
        k = torch.randn(1, cfg.n_kv_heads, 740, cfg.head_dim, device=device, dtype=cfg.dtype)
        warm.attend(layer, torch.randn(1, cfg.n_heads, 740, cfg.head_dim, device=device,
                                       dtype=cfg.dtype), k, torch.randn_like(k))
    warm.advance_packed()
    tick = PackedBatchCache([a, b, c])
    counts = [1, 333, 1]
    tick.prepare_packed(counts)
    q = torch.randn(1, cfg.n_heads, sum(counts), cfg.head_dim, device=device, dtype=cfg.dtype)
    k = torch.randn(1, cfg.n_kv_heads, sum(counts), cfg.head_dim, device=device, dtype=cfg.dtype)
    v = torch.randn_like(k)
    cached = [a.length, b.length, c.length]
    out = tick.attend(0, q, k, v)
    ref = dense_torch.packed_attention(
        q.float().cpu(), pool.keys[0].float().cpu(), pool.values[0].float().cpu(),
        [[p.index for p in x.pages] for x in (a, b, c)], cached, counts)
    tick.advance_packed()
    torch.testing.assert_close(out.float().cpu(), ref, rtol=2e-2, atol=2e-2)
    assert (a.length, b.length, c.length) == (701, 373, 1)


def test_restore_by_copy_gives_private_identical_pages(device):
    say("restore copy")
    cfg = config(n_layers=3)
    pool = KVPagePool(cfg, 10, device=device)
    src = PagedKVCache(pool, 2048)
    batch = PagedBatchCache([src])
    batch.prepare(512)
    for layer in range(cfg.n_layers):
        q = torch.randn(1, cfg.n_heads, 512, cfg.head_dim, device=device, dtype=cfg.dtype)
        k = torch.randn(1, cfg.n_kv_heads, 512, cfg.head_dim, device=device, dtype=cfg.dtype)
        batch.attend(layer, q, k, torch.randn_like(k))
    batch.advance(512)
    snap = src.snapshot_block(0, 512)
    shared, private = PagedKVCache(pool, 2048), PagedKVCache(pool, 2048)
    shared.restore_blocks([snap])
    private.restore_blocks([snap], copy=True)
    assert [p.index for p in shared.pages] == [p.index for p in snap.pages]
    assert not {p.index for p in private.pages} & {p.index for p in snap.pages}
    torch.cuda.synchronize()
    pairs = [(s.index, d.index) for s, d in zip(snap.pages, private.pages)]
    for layer in range(cfg.n_layers):
        for store in (pool.keys, pool.values):
            for si, di in pairs:
                assert torch.equal(store[layer][si].view(torch.int16), store[layer][di].view(torch.int16))
    # continuing both gives the same attention output
    q = torch.randn(1, cfg.n_heads, 1, cfg.head_dim, device=device, dtype=cfg.dtype)
    k = torch.randn(1, cfg.n_kv_heads, 1, cfg.head_dim, device=device, dtype=cfg.dtype)
    v = torch.randn_like(k)
    outs = []
    for cache in (shared, private):
        b = PagedBatchCache([cache])
        b.prepare(1)
        outs.append(b.attend(0, q, k, v))
        b.advance(1)
    assert torch.equal(outs[0], outs[1])
    del snap, src, shared, private, batch, b, cache
    gc.collect()
    assert pool.free_pages == pool.num_pages


def test_full_hit_restore_recomputes_only_the_last_token(device):
    """Copy-on-write restore of a prompt the prefix cache covers completely: the pages
    stay shared except the last, which is a private bit-copy the request can truncate
    into and rewrite; the shared page is never written."""
    say("restore private tail")
    cfg = config(n_layers=2)
    pool = KVPagePool(cfg, 12, device=device)
    src = PagedKVCache(pool, 2048)
    fill = PagedBatchCache([src])
    fill.prepare(512)
    g = torch.Generator(device=device).manual_seed(5)
    for layer in range(cfg.n_layers):
        q = torch.randn(1, cfg.n_heads, 512, cfg.head_dim, generator=g, device=device).to(cfg.dtype)
        k = torch.randn(1, cfg.n_kv_heads, 512, cfg.head_dim, generator=g, device=device).to(cfg.dtype)
        fill.attend(layer, q, k, torch.randn_like(k))
    fill.advance(512)
    snaps = [src.snapshot_block(0, 256), src.snapshot_block(256, 512)]
    before = [t.clone() for t in pool.keys + pool.values]
    req = PagedKVCache(pool, 2048)
    req.restore_blocks(snaps, private_tail=True)
    assert req.length == 512
    assert req.pages[0] is snaps[0].pages[0]                  # shared
    assert req.pages[1].index != snaps[1].pages[0].index      # private copy
    torch.cuda.synchronize()
    src_i, dst_i = snaps[1].pages[0].index, req.pages[1].index
    for store in (pool.keys, pool.values):
        for layer in range(cfg.n_layers):
            assert torch.equal(store[layer][src_i].view(torch.int16), store[layer][dst_i].view(torch.int16))
    # recompute the last prompt token into the private page
    req.truncate(511)
    tick = PagedBatchCache([req])
    tick.prepare(1)
    assert tick.write_slots.tolist() == [dst_i * 256 + 255]
    for layer in range(cfg.n_layers):
        q = torch.randn(1, cfg.n_heads, 1, cfg.head_dim, generator=g, device=device).to(cfg.dtype)
        k = torch.randn(1, cfg.n_kv_heads, 1, cfg.head_dim, generator=g, device=device).to(cfg.dtype)
        tick.attend(layer, q, k, torch.randn_like(k))
    tick.advance(1)
    torch.cuda.synchronize()
    after = pool.keys + pool.values
    for t0, t1 in zip(before, after):
        assert torch.equal(t0[src_i].view(torch.int16), t1[src_i].view(torch.int16))  # shared page untouched
        assert torch.equal(t0[snaps[0].pages[0].index].view(torch.int16), t1[snaps[0].pages[0].index].view(torch.int16))
