"""Per-tick attention metadata, restated in numpy (test infrastructure only).

Follows PagedBatchCache.prepare (paged_cache.py:221-270) and
PackedBatchCache.prepare_packed (paged_cache.py:418-494): from each sequence's cached
length before the tick, the tokens it appends, its logit rows and its page table.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np


def tick_metadata(lengths: Sequence[int], counts: Sequence[int],
                  tables: Sequence[Sequence[int]], page_size: int,
                  logit_counts: Sequence[int] | None = None) -> dict[str, np.ndarray]:
    """The arrays the reference builds for one tick.

    cu_seq_q = [0, cumsum(counts)]; ends = lengths + counts; cu_seq_k = [0, cumsum(ends)];
    seqused_k = ends; positions = concat(range(length_b, end_b)); write_slots[pos] =
    table_b[pos // page_size] * page_size + pos % page_size (paged_cache.py:262-269,
    :484-493); logit_indices = concat(range(cu_seq_q[b+1] - tail_b, cu_seq_q[b+1]))
    (:474-482).
    """
    lengths = np.asarray(lengths, dtype=np.int64)
    counts = np.asarray(counts, dtype=np.int64)
    ends = lengths + counts
    cu_q = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(ends)]).astype(np.int32)
    positions, slots = [], []
    for b in range(len(counts)):
        pos = np.arange(lengths[b], ends[b], dtype=np.int64)
        pages = np.asarray(tables[b], dtype=np.int64)[pos // page_size]
        positions.append(pos)
        slots.append(pages * page_size + pos % page_size)
    out = {
        "cu_seq_q": cu_q,
        "cu_seq_k": cu_k,
        "seqused_k": ends.astype(np.int32),
        "positions": np.concatenate(positions) if positions else np.zeros(0, np.int64),
        "write_slots": np.concatenate(slots) if slots else np.zeros(0, np.int64),
    }
    if logit_counts is not None:
        tails = np.asarray(logit_counts, dtype=np.int64)
        out["logit_indices"] = np.concatenate(
            [np.arange(cu_q[b + 1] - tails[b], cu_q[b + 1], dtype=np.int64) for b in range(len(counts))]
        )
    return out
