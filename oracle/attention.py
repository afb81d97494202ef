"""float64 numpy restatement of paged varlen GQA attention (test infrastructure only).

Follows the reference's CPU path, src/helios/runtime/qwen3/paged_cache.py:378-414
(uniform batches) and :521-546 (packed ticks): gather each sequence's pages in table
order and keep its first L keys, repeat each KV head for its G = Hq / Hkv query heads
(repeat_interleave: query head h reads KV head h // G, :386-391), and take a masked
softmax with the mask ``key_pos <= cached_len + i`` (:392-396, :532-535), i.e. the
bottom-right causal mask of varlen_attn(window_size=(-1, 0)) at :316-329 / :506-519.
The general (left, right) window of that call is restated too:
row i sits at qpos = L - n + i and sees keys j with j <= qpos + right (right >= 0),
j >= qpos - left (left >= 0) and j < L. A row that sees no key returns zeros and
lse = -inf (the reference never builds one; the kernels define it this way).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np


def gather_sequence(pool: np.ndarray, table: Sequence[int], length: int) -> np.ndarray:
    """Keys/values of one sequence as ``[length, Hkv, d]`` (paged_cache.py:405-414)."""
    page_size = pool.shape[1]
    n_pages = (length + page_size - 1) // page_size
    pages = np.asarray(list(table)[:n_pages], dtype=np.int64)
    return pool[pages].reshape(-1, pool.shape[2], pool.shape[3])[:length]


def visible_range(L: int, n: int, i: int, window: tuple[int, int]) -> tuple[int, int]:
    """Inclusive key range [lo, hi] of row i (hi < lo means no visible key)."""
    left, right = window
    qpos = L - n + i
    hi = L - 1 if right < 0 else min(L - 1, qpos + right)
    lo = 0 if left < 0 else max(0, qpos - left)
    return lo, hi


def attend_dense(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, scale: float,
                 window: tuple[int, int] = (-1, 0), rows: Sequence[int] | None = None,
                 block_rows: int = 256) -> tuple[np.ndarray, np.ndarray]:
    """One sequence: q ``[n, Hq, d]``, k / v ``[L, Hkv, d]`` -> out ``[n, Hq, d]``,
    lse ``[Hq, n]`` (float64). ``rows`` restricts the computed rows (others are NaN)."""
    n, hq, d = q.shape
    L, hkv = k.shape[0], k.shape[1]
    G = hq // hkv
    out = np.full((n, hq, d), np.nan, dtype=np.float64)
    lse = np.full((hq, n), np.nan, dtype=np.float64)
    want = np.arange(n) if rows is None else np.asarray(sorted(rows), dtype=np.int64)
    if L == 0:
        out[want] = 0.0
        lse[:, want] = -np.inf
        return out, lse
    k64 = k.astype(np.float64)
    v64 = v.astype(np.float64)
    j = np.arange(L)
    for start in range(0, len(want), block_rows):
        idx = want[start:start + block_rows]
        qb = q[idx].astype(np.float64).reshape(len(idx), hkv, G, d)
        # scores[h_kv, g, row, key]
        s = np.einsum("rhgd,lhd->hgrl", qb, k64, optimize=True) * scale
        lo_hi = np.array([visible_range(L, n, int(i), window) for i in idx])
        mask = (j[None, :] >= lo_hi[:, :1]) & (j[None, :] <= lo_hi[:, 1:])
        s = np.where(mask[None, None], s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        empty = ~np.isfinite(m)
        m = np.where(empty, 0.0, m)
        p = np.exp(s - m)
        denom = p.sum(axis=-1, keepdims=True)
        o = np.einsum("hgrl,lhd->rhgd", p / np.where(denom > 0, denom, 1.0), v64, optimize=True)
        o = np.where(empty.transpose(2, 0, 1, 3).reshape(len(idx), hkv, G, 1), 0.0, o)
        out[idx] = o.reshape(len(idx), hq, d)
        l_ = np.where(empty[..., 0], -np.inf, np.log(np.where(denom[..., 0] > 0, denom[..., 0], 1.0)) + m[..., 0])
        lse[:, idx] = l_.reshape(hq, len(idx))
    return out, lse


def paged_varlen_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                           cu_seq_q: Sequence[int], k_lens: Sequence[int],
                           tables: Sequence[Sequence[int]], *, scale: float | None = None,
                           window: tuple[int, int] = (-1, 0),
                           rows: dict[int, Sequence[int]] | None = None
                           ) -> tuple[np.ndarray, np.ndarray]:
    """Packed varlen paged attention: q ``[T, Hq, d]``, pools ``[P, S, Hkv, d]``.

    Sequence b owns query rows cu_seq_q[b]..cu_seq_q[b+1] and k_lens[b] keys read
    through tables[b]. Returns out ``[T, Hq, d]`` and lse ``[Hq, T]`` in float64.
    ``rows`` optionally maps b to the sequence-local rows to compute.
    """
    T, hq, d = q.shape
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    out = np.full((T, hq, d), np.nan, dtype=np.float64)
    lse = np.full((hq, T), np.nan, dtype=np.float64)
    for b in range(len(k_lens)):
        q0, q1 = int(cu_seq_q[b]), int(cu_seq_q[b + 1])
        if q1 == q0:
            continue
        L = int(k_lens[b])
        k = gather_sequence(k_pool, tables[b], L)
        v = gather_sequence(v_pool, tables[b], L)
        sel = None if rows is None else rows.get(b)
        o, l_ = attend_dense(q[q0:q1], k, v, scale=scale, window=window, rows=sel)
        out[q0:q1] = o
        lse[:, q0:q1] = l_
    return out, lse


def brute_force_attention(q, k, v, *, scale, window=(-1, 0)):
    """Pure-Python loops over one sequence (tiny inputs only): q [n][Hq][d],
    k / v [L][Hkv][d] nested lists -> out [n][Hq][d]. Independent of numpy's
    reductions; used to pin attend_dense."""
    import math

    n, hq, d = len(q), len(q[0]), len(q[0][0])
    L = len(k)
    hkv = len(k[0]) if L else 1
    G = hq // hkv
    out = []
    for i in range(n):
        lo, hi = visible_range(L, n, i, window)
        row = []
        for h in range(hq):
            kh = h // G
            keys = list(range(lo, hi + 1))
            if not keys:
                row.append([0.0] * d)
                continue
            scores = [scale * sum(q[i][h][t] * k[j][kh][t] for t in range(d)) for j in keys]
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            z = sum(w)
            row.append([sum(w[a] * v[j][kh][t] for a, j in enumerate(keys)) / z for t in range(d)])
        out.append(row)
    return out
