"""The reference's dense-KV CPU attention path, op for op in torch (test infrastructure).

This is the CPU restatement the reference itself runs when the pool is not on CUDA,
src/helios/runtime/qwen3/paged_cache.py:521-546 (packed ticks; the uniform form at
:378-402 is the same per sequence): gather each sequence's pages with index_select
(:405-414), repeat_interleave the KV heads to the query heads, and call
scaled_dot_product_attention with the bool mask ``arange(end) <= cached + arange(n)``.
It is the timed CPU baseline of bench.py and a library-based cross-check of the
float64 oracle.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch


def gather(storage: torch.Tensor, pages: Sequence[int], length: int) -> torch.Tensor:
    """``[1, Hkv, length, d]`` (paged_cache.py:405-414)."""
    indices = torch.tensor(list(pages), device=storage.device)
    return (
        storage.index_select(0, indices)
        .reshape(-1, *storage.shape[2:])[:length]
        .permute(1, 0, 2)
        .unsqueeze(0)
    )


def packed_attention(queries: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                     tables: Sequence[Sequence[int]], cached: Sequence[int],
                     counts: Sequence[int]) -> torch.Tensor:
    """queries ``[1, Hq, sum(counts), d]`` -> ``[1, Hq, sum(counts), d]``."""
    page_size = k_pool.shape[1]
    outputs = []
    offset = 0
    for pages, length, count in zip(tables, cached, counts, strict=True):
        end = length + count
        used = list(pages)[: (end + page_size - 1) // page_size]
        k = gather(k_pool, used, end)
        v = gather(v_pool, used, end)
        repeat = queries.shape[1] // k.shape[1]
        k, v = k.repeat_interleave(repeat, dim=1), v.repeat_interleave(repeat, dim=1)
        mask = torch.arange(end)[None, :] <= (length + torch.arange(count))[:, None]
        outputs.append(
            torch.nn.functional.scaled_dot_product_attention(
                queries[:, :, offset:offset + count], k, v, attn_mask=mask, dropout_p=0.0
            )
        )
        offset += count
    return torch.cat(outputs, dim=2)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward, op for op (layers.py:36-40)."""
    input_dtype = x.dtype
    x = x.float()
    normalized = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (normalized * weight).to(input_dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               position_ids: torch.Tensor) -> torch.Tensor:
    """apply_rope with position_ids, op for op (layers.py:54-72); x is [B, H, T, d] and
    position_ids [B, T]."""
    head_dim = x.shape[-1]
    cos = cos[position_ids].unsqueeze(1)
    sin = sin[position_ids].unsqueeze(1)
    first, second = x[..., : head_dim // 2], x[..., head_dim // 2:]
    return (x * cos + torch.cat((-second, first), dim=-1) * sin).to(x.dtype)


def rope_parameters(head_dim: int, rows: int, base: float) -> tuple[torch.Tensor, torch.Tensor]:
    """rope_parameters (layers.py:43-51) for `rows` positions."""
    inverse_frequencies = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    positions = torch.arange(rows, dtype=torch.float32)
    angles = positions.unsqueeze(1) * inverse_frequencies.unsqueeze(0)
    angles = torch.cat((angles, angles), dim=1)
    return torch.cos(angles), torch.sin(angles)
