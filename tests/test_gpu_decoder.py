"""The packed decoder forward on the paged path: this build's sequence (metadata kernel,
fused norm/RoPE/append) against the reference's sequence on the same weights."""

from __future__ import annotations

import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.decoder import PagedQwen3Decoder
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedKVCache
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


def test_packed_forward_matches_reference_sequence(device):
    say("decoder packed forward")
    config = Qwen3Config(vocab_size=1000, context_length=4096, hidden_size=256, n_layers=2,
                         hidden_dim=512, dtype=torch.bfloat16)
    model = PagedQwen3Decoder(config, device, seed=1, std=0.05)
    lengths, counts = [300, 0, 511], [1, 200, 1]
    logits, pools = [], []
    for device_meta, fused in ((True, True), (False, False)):
        pool = KVPagePool(config, 16, device=device)
        g = torch.Generator(device=device).manual_seed(4)
        for t in pool.keys + pool.values:
            t.normal_(generator=g)
        caches = []
        for n in lengths:
            cache = PagedKVCache(pool, config.context_length)
            if n:
                cache.pages.extend(pool.acquire(-(-n // 256)))
                cache.length = n
            caches.append(cache)
        batch = PackedBatchCache(caches, device_metadata=device_meta)
        ids = torch.randint(0, config.vocab_size, (1, sum(counts)),
                            generator=torch.Generator(device=device).manual_seed(9), device=device)
        for tick in range(2):  # the second tick attends to keys the first one appended
            batch.prepare_packed(counts if tick == 0 else [1, 1, 1])
            out = model.forward_packed(ids if tick == 0 else ids[:, :3], batch, fused_rope=fused)
        torch.cuda.synchronize()
        logits.append(out.float().cpu())
        pools.append(pool.values[0].float().cpu())  # layer 0: same inputs on both paths
    assert logits[0].shape == (3, config.vocab_size)
    assert torch.isfinite(logits[0]).all()
    scale = logits[1].abs().max().item()
    assert (logits[0] - logits[1]).abs().max().item() <= 2e-2 * max(scale, 1.0)
    assert torch.equal(pools[0], pools[1])  # values are appended bit-exactly by both paths


def test_greedy_heads_match_logits_argmax(device):
    say("decoder greedy heads")
    config = Qwen3Config(vocab_size=1000, context_length=4096, hidden_size=256, n_layers=2,
                         hidden_dim=512, dtype=torch.bfloat16)
    model = PagedQwen3Decoder(config, device, seed=2, std=0.05)
    outs = []
    for greedy in (False, True):
        pool = KVPagePool(config, 8, device=device)
        caches = [PagedKVCache(pool, config.context_length) for _ in range(3)]
        batch = PackedBatchCache(caches)
        counts = [5, 130, 1]
        ids = torch.randint(0, config.vocab_size, (1, sum(counts)),
                            generator=torch.Generator(device=device).manual_seed(3), device=device)
        batch.prepare_packed(counts)
        outs.append(model.forward_packed(ids, batch, greedy=greedy))
    torch.cuda.synchronize()
    logits, picks = outs[0].float().cpu(), outs[1].cpu()
    assert picks.shape == (3,) and picks.dtype == torch.int64
    top = logits.max(dim=-1).values
    chosen = logits.gather(1, picks.unsqueeze(1))[:, 0]
    # the kernel's pick is the argmax up to one bf16 rounding of the logits
    assert ((top - chosen) <= 2 * 2.0 ** -7 * top.abs() + 1e-4).all()
