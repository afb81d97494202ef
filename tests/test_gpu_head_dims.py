"""Attention at head dims and group sizes other than Qwen3-4B's (the generic kernel),
against the float64 oracle, and the reference's own GPU test of the paged boundary
(tests/test_paged_attention.py:240-312) at its own tiny shape through the class-level
drop-in: head_dim 8, 2 query heads on 1 KV head, fp16 and bf16, a 2-token prefill of two
requests and then one decode token each."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops, synth
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PagedBatchCache, PagedKVCache
from oracle import attention as oa
from tests.gpu_cases import DeviceTick, compare, say, tolerance

pytestmark = pytest.mark.gpu


def tiny_config(dtype: torch.dtype) -> Qwen3Config:
    # The reference's tiny_config (tests/test_paged_attention.py:18-29) in the given dtype.
    return Qwen3Config(vocab_size=64, context_length=512, hidden_size=16, n_heads=2, n_layers=2,
                       hidden_dim=32, head_dim=8, n_kv_heads=1, dtype=dtype)


def _dense_sdpa(pool, caches, query):
    """The reference test's _assert_dense_match reference (:275-312): gather, repeat_interleave,
    SDPA with the bottom-right mask, in float32 on the CPU."""
    rows = []
    for row, cache in enumerate(caches):
        tokens = query.shape[2]
        start = cache.length - tokens
        keys = torch.cat([pool.keys[0][p.index] for p in cache.pages])[: cache.length].float().cpu()
        vals = torch.cat([pool.values[0][p.index] for p in cache.pages])[: cache.length].float().cpu()
        rep = query.shape[1] // keys.shape[1]
        dk = keys.permute(1, 0, 2).unsqueeze(0).repeat_interleave(rep, dim=1)
        dv = vals.permute(1, 0, 2).unsqueeze(0).repeat_interleave(rep, dim=1)
        mask = torch.arange(cache.length)[None, None, None, :] <= (start + torch.arange(tokens))[None, None, :, None]
        rows.append(torch.nn.functional.scaled_dot_product_attention(
            query[row:row + 1].float().cpu(), dk, dv, attn_mask=mask, dropout_p=0.0))
    return torch.cat(rows)


def _oracle(pool, caches, query):
    """float64 oracle over the same pool for a uniform batch: [B, Hq, T, d]."""
    tokens = query.shape[2]
    q = query.transpose(1, 2).reshape(-1, query.shape[1], query.shape[3]).float().cpu().numpy()
    k = pool.keys[0].float().cpu().numpy()
    v = pool.values[0].float().cpu().numpy()
    tables = [[p.index for p in c.pages] for c in caches]
    ends = [c.length for c in caches]
    cu = [tokens * b for b in range(len(caches) + 1)]
    out, _ = oa.paged_varlen_attention(q, k, v, cu, ends, tables)
    return out.reshape(len(caches), tokens, query.shape[1], query.shape[3]).transpose(0, 2, 1, 3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_native_paged_attention_at_its_tiny_shape(device, dtype):
    say("reference tiny shape", dtype)
    config = tiny_config(dtype)
    pool = KVPagePool(config, 4, device=device)
    caches = [PagedKVCache(pool, 512), PagedKVCache(pool, 512)]
    g = torch.Generator(device=device).manual_seed(18)
    for step, tokens in enumerate((2, 1)):
        q = torch.randn(2, config.n_heads, tokens, config.head_dim, generator=g, device=device, dtype=dtype)
        k = torch.randn(2, config.n_kv_heads, tokens, config.head_dim, generator=g, device=device, dtype=dtype)
        v = torch.randn(k.shape, generator=g, device=device, dtype=dtype)
        batch = PagedBatchCache(caches)
        batch.prepare(tokens)
        out = batch.attend(0, q, k, v)
        batch.advance(tokens)
        torch.cuda.synchronize()
        if step == 0:
            assert batch.cu_seq_q.dtype == torch.int32 and batch.cu_seq_k.dtype == torch.int32
            assert batch.cu_seq_q.tolist() == [0, 2, 4] and batch.cu_seq_k.tolist() == [0, 2, 4]
        assert out.shape == q.shape and out.dtype == dtype
        # the reference's own check and tolerance
        torch.testing.assert_close(out.float().cpu(), _dense_sdpa(pool, caches, q), rtol=2e-2, atol=2e-2)
        # and the float64 oracle at this build's bound for the dtype
        ref = _oracle(pool, caches, q)
        got = out.float().cpu().numpy()
        max_abs, mean_abs = tolerance(dtype)
        err = np.abs(got - ref)
        say("tiny", dtype, tokens, f"max_abs={err.max():.3e} mean_abs={err.mean():.3e}")
        assert err.max() <= max_abs and err.mean() <= mean_abs
    assert [c.length for c in caches] == [3, 3]


SHAPES = [  # (n_q_heads, n_kv_heads, head_dim)
    (2, 1, 8),      # the reference's tiny config
    (8, 2, 16),
    (16, 4, 64),    # G = 4 at head_dim 64
    (12, 4, 96),    # G = 3
    (48, 8, 128),   # G = 6 at Qwen's head_dim: not one of the tuned group sizes
    (16, 1, 256),   # G = 16 at the largest head_dim
    (64, 2, 64),    # G = 32: two head blocks per KV head
]


@pytest.mark.parametrize("hq,hkv,d", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_generic_shapes_match_oracle(device, hq, hkv, d, dtype):
    say("generic", hq, hkv, d, dtype)
    w = synth.small_mixed(200 + d + hq, n_q_heads=hq, n_kv_heads=hkv, head_dim=d, batch=7,
                          max_cached=800, max_chunk=150, num_pages=48)
    tick = DeviceTick(w, dtype, device)
    ref, ref_lse = tick.oracle()
    out, lse = tick.attend(exact_grid=True, return_lse=True)
    compare(out, ref, what=f"generic hq={hq} hkv={hkv} d={d} {dtype}")
    assert np.abs(lse.cpu().numpy() - ref_lse).max() < 5e-3
    again = tick.attend()          # bound-sized grid: same bits
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("window", [(-1, -1), (40, 0), (0, 0), (300, 3)])
def test_generic_windows(device, window):
    say("generic window", window)
    w = synth.small_mixed(260, n_q_heads=8, n_kv_heads=2, head_dim=64, batch=6, max_cached=700,
                          max_chunk=200, num_pages=40)
    tick = DeviceTick(w, torch.bfloat16, device)
    ref, _ = tick.oracle(window=window)
    compare(tick.attend(window=window, exact_grid=True), ref, what=f"generic window {window}")


def test_generic_fused_append_and_packed_keys(device):
    """The append + attention call on the generic path (every row appended first), and
    packed (non-paged) keys."""
    say("generic append / packed keys")
    w = synth.small_mixed(270, n_q_heads=4, n_kv_heads=2, head_dim=32, batch=6, max_cached=600,
                          max_chunk=120, num_pages=40)
    ref_tick = DeviceTick(w, torch.bfloat16, device)
    want = ref_tick.attend(exact_grid=True)
    k_pool, v_pool = ref_tick.fresh_pools()
    out = ref_tick.plan().run(ref_tick.q, k_pool, v_pool, ref_tick.block_table,
                              append=(ref_tick.k_new, ref_tick.v_new, ref_tick.write_slots))
    torch.cuda.synchronize()
    assert torch.equal(k_pool.view(torch.int16), ref_tick.k_pool.view(torch.int16))
    assert torch.equal(v_pool.view(torch.int16), ref_tick.v_pool.view(torch.int16))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    keys = [torch.cat([ref_tick.k_pool[p] for p in t])[:L] for t, L in zip(w.tables, w.k_lens)]
    vals = [torch.cat([ref_tick.v_pool[p] for p in t])[:L] for t, L in zip(w.tables, w.k_lens)]
    packed = ops.varlen_attn(ref_tick.q, torch.cat(keys).contiguous(), torch.cat(vals).contiguous(),
                             ref_tick.cu_seq_q, ref_tick.cu_seq_k, w.max_q, w.max_k, is_causal=True,
                             enable_gqa=True)
    ref, _ = ref_tick.oracle()
    compare(packed, ref, what="generic packed keys")
