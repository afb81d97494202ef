"""The full-model tick's workload (C5) on the GPU: 128 decoders with contexts uniform in
[1024, 8192], each holding up to 16 pages of one 4096-token prefix, plus one request
that prefills a 1024-token chunk after that prefix.

* One attention layer at full size through ``PackedBatchCache.attend_projected`` with
  the default metadata kernel and the shared-prefix cascade under its default cost
  constants (levels of more than 64 rows: several level row blocks, split level tiles
  and multi-row combine records), against the float64 oracle: every decode row and 192
  chunk rows, bf16 bound 2e-2 / 2e-3.
* The 36-layer random-init forward of the same tick with greedy heads: ids in range,
  finite logits, no plan error, and greedy ids equal to the argmax of the logits
  wherever the top two logits are further apart than their rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops, synth
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, _PrefixCascade
from oracle import attention as oa
from oracle import dense_torch
from tests.gpu_cases import compare, say

pytestmark = pytest.mark.gpu


def _pool_and_caches(device, config, seed=5):
    lengths, counts = synth.c5_lengths(seed)
    pool = KVPagePool(config, synth.c5_pool_pages(lengths, counts), device=device)
    pool.storage.normal_(generator=torch.Generator(device=device).manual_seed(seed))
    prefix, caches = synth.shared_prefix_caches(pool, lengths)
    return pool, prefix, caches, lengths, counts


def test_c5_attention_layer_matches_oracle(device):
    say("c5 attention layer (attend_projected, default cascade)")
    config = Qwen3Config(n_layers=1)
    d, hq, hkv = config.head_dim, config.n_heads, config.n_kv_heads
    pool, _prefix, caches, lengths, counts = _pool_and_caches(device, config)
    batch = PackedBatchCache(caches)
    batch.prepare_packed(counts)
    levels = _PrefixCascade.levels(batch, counts)
    assert batch._cascade is not None and levels, "the default cost model should build levels"
    assert max(len(members) for *_, members in levels) > 64
    say("levels", [(first, end, len(members)) for _, first, end, members in levels])
    total = sum(counts)
    g = torch.Generator(device=device).manual_seed(51)
    x_q = torch.randn((1, total, hq * d), generator=g, device=device).to(config.dtype)
    x_k = torch.randn((1, total, hkv * d), generator=g, device=device).to(config.dtype)
    x_v = torch.randn((1, total, hkv * d), generator=g, device=device).to(config.dtype)
    wq = (1 + 0.1 * torch.randn(d, generator=g, device=device)).float()
    wk = (1 + 0.1 * torch.randn(d, generator=g, device=device)).float()
    cos, sin = dense_torch.rope_parameters(d, config.context_length, config.rope_base)
    cos, sin = cos.to(device), sin.to(device)
    # The normalised, rotated queries attention sees: the same kernel attend_projected
    # runs first (it appends the same K/V bits to the same slots again).
    q_rot = ops.qk_norm_rope_append(
        x_q.view(total, hq, d), x_k.view(total, hkv, d), x_v.view(total, hkv, d), wq, wk, cos, sin,
        batch.positions[0], pool.keys[0], pool.values[0], batch.write_slots, config.rms_norm_eps)
    out = batch.attend_projected(0, x_q, x_k, x_v, wq, wk, cos, sin, config.rms_norm_eps)
    torch.cuda.synchronize()
    assert batch._cascade.plan_a.error_word() == 0 and batch._cascade.plan_b.error_word() == 0
    assert out.shape == (1, hq, total, d)
    got = out[0].transpose(0, 1)                       # [total, hq, d]
    # float64 oracle over the pages the tick reads, on the device's rounded inputs
    tables = [[p.index for p in c.pages] for c in caches]
    ends = [n + c for n, c in zip(lengths, counts)]
    used = sorted({p for t, L in zip(tables, ends) for p in t[: -(-L // 256)]})
    remap = {p: i for i, p in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=device)
    kp = pool.keys[0].index_select(0, idx).float().cpu().numpy()
    vp = pool.values[0].index_select(0, idx).float().cpu().numpy()
    local = [[remap.get(p, 0) for p in t] for t in tables]
    chunk = len(counts) - 1
    n = counts[chunk]
    sample = list(range(0, 64)) + list(range(n // 2 - 32, n // 2 + 32)) + list(range(n - 64, n))
    rows = {b: [0] for b in range(chunk)} | {chunk: sample}
    cu = [0, *np.cumsum(counts).tolist()]
    ref, _ = oa.paged_varlen_attention(q_rot.float().cpu().numpy(), kp, vp, cu, ends, local, rows=rows)
    flat = np.array(list(range(chunk)) + [cu[chunk] + r for r in sample])
    compare(got, ref, what="c5 layer (128 decode rows + 192 chunk rows)", rows=flat)
    batch.advance_packed()


def test_c5_full_forward_greedy_properties(device):
    from helios_amd.decoder import PagedQwen3Decoder

    say("c5 36-layer forward, greedy heads")
    config = Qwen3Config()
    pool, _prefix, caches, lengths, counts = _pool_and_caches(device, config)
    model = PagedQwen3Decoder(config, device, seed=5)
    tokens = sum(counts)
    input_ids = torch.randint(0, config.vocab_size, (1, tokens),
                              generator=torch.Generator(device=device).manual_seed(52), device=device)
    batch = PackedBatchCache(caches)
    outs = []
    for greedy in (True, False):
        batch.prepare_packed(counts)
        outs.append(model.forward_packed(input_ids, batch, greedy=greedy))
        torch.cuda.synchronize()
        assert batch._cascade is not None
        assert batch._cascade.plan_a.error_word() == 0 and batch._cascade.plan_b.error_word() == 0
        for cache, n in zip(caches, lengths):   # roll back: the second tick sees the same keys
            cache.truncate(n)
    ids, logits = outs[0].cpu(), outs[1].float().cpu()
    assert ids.shape == (len(counts),) and ids.dtype == torch.int64
    assert bool(((ids >= 0) & (ids < config.vocab_size)).all())
    assert logits.shape == (len(counts), config.vocab_size) and bool(torch.isfinite(logits).all())
    top2 = logits.topk(2, dim=-1).values
    chosen = logits.gather(1, ids.unsqueeze(1))[:, 0]
    ulp = 2.0 ** -7 * top2[:, 0].abs()
    # The fused heads round each logit to bf16 as the Linear does; their pick is the
    # argmax up to that rounding, and exactly the argmax where the top two are apart.
    assert bool(((top2[:, 0] - chosen) <= 2 * ulp + 1e-4).all())
    apart = (top2[:, 0] - top2[:, 1]) > 2 * ulp
    say("clear winners", int(apart.sum()), "of", len(counts))
    assert torch.equal(ids[apart], logits.argmax(dim=-1)[apart])
