"""A restored paged prefix, continued by mixed prefill/decode ticks on the paged path,
against the dense-KV model in fp32 on the CPU.

The reference states this for its own paged path in
tests/test_paged_attention.py:153-178 (restored prefix continuation == dense-KV model).
Here the paged side is this build's whole tick: device metadata, fused q/k norm + RoPE +
append, the HIP attention kernels (decode rows, chunk rows, the shared-prefix cascade
when pages are shared) and the decoder's torch GEMMs in bf16. The dense side is an
independent fp32 forward with causal softmax over dense K/V (layers.py:165-191), so the
two share the weights and nothing else. A request that failed to see its restored prefix,
a RoPE position off by one or a key appended to the wrong slot moves logits by O(1); the
bound below is set by bf16 rounding over two layers.
"""

from __future__ import annotations

import math

import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.decoder import PagedQwen3Decoder
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedKVCache
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu

# Largest logit difference allowed, relative to the largest dense logit of the row, and
# the mean difference, relative to the mean dense logit magnitude. Measured on MI355X:
# at most 0.7 % of the largest logit and 0.75 % of the mean magnitude (bf16 activations).
MAX_REL = 3e-2
MEAN_REL = 1.5e-2


def dense_logits(model: PagedQwen3Decoder, ids: list[int]) -> torch.Tensor:
    """Logits at every position of ``ids`` from one causal pass over dense K/V, fp32."""
    cfg = model.config

    def f(t: torch.Tensor) -> torch.Tensor:
        return t.detach().float().cpu()

    T = len(ids)
    hq, hkv, d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    eps = cfg.rms_norm_eps
    x = f(model.embedding)[torch.tensor(ids)]
    cos, sin = f(model.cos)[:T], f(model.sin)[:T]

    def rms(v: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps) * w

    def rope(v: torch.Tensor) -> torch.Tensor:  # [heads, T, d], position of row t is t
        half = d // 2
        return v * cos + torch.cat((-v[..., half:], v[..., :half]), -1) * sin

    visible = torch.ones(T, T, dtype=torch.bool).tril()
    for layer in model.layers:
        h = rms(x, f(layer["input_norm"]))
        qkv = h @ f(layer["qkv"]).t()
        q = qkv[:, :hq * d].reshape(T, hq, d).transpose(0, 1)
        k = qkv[:, hq * d:(hq + hkv) * d].reshape(T, hkv, d).transpose(0, 1)
        v = qkv[:, (hq + hkv) * d:].reshape(T, hkv, d).transpose(0, 1)
        q = rope(rms(q, f(layer["q_norm"])))
        k = rope(rms(k, f(layer["k_norm"])))
        k = k.repeat_interleave(hq // hkv, 0)
        v = v.repeat_interleave(hq // hkv, 0)
        scores = (q @ k.transpose(1, 2)) / math.sqrt(d)
        context = torch.softmax(scores.masked_fill(~visible, float("-inf")), -1) @ v
        x = x + context.transpose(0, 1).reshape(T, hq * d) @ f(layer["o"]).t()
        h = rms(x, f(layer["post_norm"]))
        gate, up = (h @ f(layer["gate_up"]).t()).chunk(2, -1)
        x = x + (torch.nn.functional.silu(gate) * up) @ f(layer["down"]).t()
    return rms(x, f(model.final_norm)) @ f(model.embedding).t()


@pytest.mark.parametrize("restore", ["shared", "copy"])
def test_restored_prefix_continuation_matches_dense_model(device, restore):
    say(f"restored prefix continuation vs dense fp32 model ({restore} restore)")
    config = Qwen3Config(vocab_size=1000, context_length=4096, hidden_size=256, n_layers=2,
                         hidden_dim=512, dtype=torch.bfloat16)
    model = PagedQwen3Decoder(config, device, seed=3, std=0.05)
    gen = torch.Generator().manual_seed(11)

    def draw(n: int) -> list[int]:
        return torch.randint(0, config.vocab_size, (n,), generator=gen).tolist()

    prompt, a_next, b_own, b_next = draw(300), draw(3), draw(40), draw(2)
    pool = KVPagePool(config, 16, device=device)

    def tick(caches, counts, tokens):
        batch = PackedBatchCache(caches)
        batch.prepare_packed(counts)
        out = model.forward_packed(torch.tensor([tokens], device=device), batch)
        torch.cuda.synchronize()
        return out.float().cpu()

    got_a, got_b = [], []
    a = PagedKVCache(pool, config.context_length)
    out = tick([a], [300], prompt)  # A prefills its whole prompt (two pages)
    got_a.append((299, out[0]))

    b = PagedKVCache(pool, config.context_length)
    b.restore_blocks([a.snapshot_block(0, 256)], copy=restore == "copy")
    assert (b.pages[0] is a.pages[0]) == (restore == "shared")
    # A decodes while B prefills its own 40 tokens after the restored page, in one tick.
    out = tick([a, b], [1, 40], [a_next[0]] + b_own)
    got_a.append((300, out[0]))
    got_b.append((295, out[1]))
    for step in range(2):
        out = tick([a, b], [1, 1], [a_next[1 + step], b_next[step]])
        got_a.append((301 + step, out[0]))
        got_b.append((296 + step, out[1]))

    for name, seq, got in (("A", prompt + a_next, got_a), ("B", prompt[:256] + b_own + b_next, got_b)):
        dense = dense_logits(model, seq)
        for pos, row in got:
            ref = dense[pos]
            diff = (row - ref).abs()
            scale = ref.abs().max().item()
            print(f"{name} pos {pos}: max {diff.max().item():.3e} mean {diff.mean().item():.3e} "
                  f"(logit scale {scale:.3f})", flush=True)
            assert torch.isfinite(row).all()
            assert diff.max().item() <= MAX_REL * scale, (name, pos)
            assert diff.mean().item() <= MEAN_REL * ref.abs().mean().item(), (name, pos)
