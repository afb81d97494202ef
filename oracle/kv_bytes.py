"""Bit-exact restatements of the KV byte movers (test infrastructure only).

Arrays are handled as raw integer views (uint16 for bf16/fp16) so every comparison
is bit for bit.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np


def kv_append(k_pool: np.ndarray, v_pool: np.ndarray, write_slots: np.ndarray,
              k_new: np.ndarray, v_new: np.ndarray) -> None:
    """In place: ``pool.reshape(-1, Hkv, d)[write_slots[t]] = new[t]`` for K and V.

    Follows PagedBatchCache._write (paged_cache.py:335-345): index_copy_ along dim 0
    of ``pool.view(-1, n_kv_heads, head_dim)``.
    """
    n_kv, d = k_pool.shape[-2], k_pool.shape[-1]
    kf = k_pool.reshape(-1, n_kv, d)
    vf = v_pool.reshape(-1, n_kv, d)
    for t, slot in enumerate(np.asarray(write_slots, dtype=np.int64)):
        kf[slot] = k_new[t]
        vf[slot] = v_new[t]


def kv_gather(pool: np.ndarray, pages: Sequence[int], length: int) -> np.ndarray:
    """Paged -> dense ``[1, Hkv, length, d]`` (paged_cache.py:405-414:
    index_select(0, pages).reshape(-1, Hkv, d)[:length].permute(1, 0, 2).unsqueeze(0))."""
    n_kv, d = pool.shape[-2], pool.shape[-1]
    rows = pool[np.asarray(pages, dtype=np.int64)].reshape(-1, n_kv, d)[:length]
    return np.ascontiguousarray(rows.transpose(1, 0, 2))[None]


def kv_copy_pages(pools: Sequence[np.ndarray], src_pages: Sequence[int],
                  dst_pages: Sequence[int]) -> None:
    """In place, per layer tensor: ``pool[dst[i]] = pool[src[i]]`` (the page form of
    KVCache.snapshot_block clone + restore_blocks copy_, cache.py:109-147)."""
    src = np.asarray(src_pages, dtype=np.int64)
    dst = np.asarray(dst_pages, dtype=np.int64)
    for pool in pools:
        pool[dst] = pool[src].copy()
