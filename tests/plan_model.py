"""Python model of the attention work planner, for checking the device plan entry by entry.

The planner (plan_kernel in helios_amd/csrc/paged_attn.hip) writes four lists into the
workspace. This module builds the same lists from the host lengths:

- decode items {b, split, q0, L}: one per 256-key split of each one-token row;
- chunk items {b, row0, head quad, sp | (S - 1) << 16}: one per row block, head quad and
  key-tile split;
- each chunk item's first partial row;
- combine records {b, first slot, splits | (rows - 1) << 24, first output row}: one per
  multi-split decode row, and one per 8 rows of a split chunk block.

Sequences go in order and a chunk's row blocks from the last to the first. When the tick
has at most 256 row blocks, the chunk items are then reordered block by block, longest
first: by key tiles per item, descending, ties in that order. The split size
follows the documented rule (at least max(4, ceil(tiles * Hkv / 512)) tiles when the
unsplit chunk items launch fewer than 512 workgroups, raised to the smallest size that
fits whole rounds of 256 workgroups, or one round when the size that fits one round is
at most 1.25 x the chunk tiles per CU); then only blocks longer than max(split size,
1.25 x the chunk tiles per CU) split. The workspace offsets mirror make_layout.
"""

from __future__ import annotations

import numpy as np

SPLIT = 256
TILE = 64
FILL_WGS = 512
CUS = 256
MIN_SPLIT_TILES = 4
MAX_SPLITS = 64
COMB_ROWS = 8
SORT_BLOCKS = 256  # ticks of at most this many row blocks list chunk items longest first
HEADER_WORDS = 64
HEAD_DIM = 128


def _ceil(a: int, b: int) -> int:
    return -(-a // b)


def geometry(hq: int, hkv: int) -> tuple[int, int]:
    """(rows per chunk item, head quads)."""
    g = hq // hkv
    gw = min(g, 4)
    return 64 * (4 // gw), g // gw


def chunk_tiles(n: int, L: int, row0: int, rows_per_item: int, window: tuple[int, int]) -> int:
    off = L - n
    row_end = min(n, row0 + rows_per_item)
    klo = 0 if window[0] < 0 else max(0, off + row0 - window[0])
    khi = L - 1 if window[1] < 0 else min(L - 1, off + row_end - 1 + window[1])
    return (khi // TILE + 1 - klo // TILE) if khi >= klo else 0


def split_count(tiles: int, st: int, keep: int | None = None) -> int:
    keep = st if keep is None else keep
    return 1 if st <= 0 or tiles <= keep else min(MAX_SPLITS, _ceil(tiles, st))


def keep_tiles(q_lens, k_lens, hq: int, hkv: int, window, st: int) -> int:
    """Blocks of at most this many tiles stay whole: 1.25 x the chunk tiles per CU."""
    rpi, quads = geometry(hq, hkv)
    tiles = quads * sum(chunk_tiles(n, L, r0, rpi, window)
                        for n, L in zip(q_lens, k_lens) if n >= 2 for r0 in range(0, n, rpi))
    return max(st, _ceil(5 * tiles * hkv, 4 * CUS))


def split_tiles(q_lens, k_lens, hq: int, hkv: int, window) -> int:
    rpi, quads = geometry(hq, hkv)
    blocks = [chunk_tiles(n, L, r0, rpi, window)
              for n, L in zip(q_lens, k_lens) if n >= 2 for r0 in range(0, n, rpi)]
    items0 = len(blocks) * quads
    if not items0 or items0 * hkv >= FILL_WGS:
        return 0
    st = max(MIN_SPLIT_TILES, _ceil(sum(blocks) * quads * hkv, FILL_WGS))

    def wgs(s):
        return hkv * quads * sum(split_count(t, s) for t in blocks)

    max_t = max(blocks)
    if max_t <= st:
        return st
    st0 = st
    w0 = wgs(st)
    rounds = w0 // CUS
    if rounds >= 1 and w0 % CUS and wgs(max_t) <= rounds * CUS:
        st = min(s for s in range(st0, max_t + 1) if wgs(s) <= rounds * CUS)
    # one round instead, when its pieces are no longer than 1.25 x the tiles per CU
    if w0 > CUS and wgs(max_t) <= CUS:
        s1 = min(s for s in range(st0, max_t + 1) if wgs(s) <= CUS)
        if s1 <= _ceil(5 * sum(blocks) * quads * hkv, 4 * CUS):
            st = s1
    return st


def decode_splits(L: int, win_left: int) -> tuple[int, int]:
    if L <= 0:
        return 0, 1
    lo = 0 if win_left < 0 else max(0, L - 1 - win_left)
    return lo // SPLIT, (L - 1) // SPLIT - lo // SPLIT + 1


def layout(batch: int, max_q: int, max_k: int, hq: int, hkv: int) -> dict[str, int]:
    """Byte offsets and capacities of the workspace lists (make_layout)."""
    rpi, quads = geometry(hq, hkv)
    a256 = lambda x: (x + 255) & ~255  # noqa: E731
    max_dec = batch * (_ceil(max_k, SPLIT) if max_k > 0 else 1)
    max_pf = cslot = 0
    if max_q >= 2:
        max_pf = batch * _ceil(max_q, rpi) * quads + 2 * FILL_WGS
        cslot = _ceil(2 * FILL_WGS, hkv * quads) * min(max_q, rpi)
    max_comb = batch + cslot
    off = a256(HEADER_WORDS * 4)
    lay = {"seq_info": off}
    off = a256(off + batch * 16)
    lay["dec_items"] = off
    off = a256(off + max_dec * 16)
    lay["comb_seqs"] = off
    off = a256(off + max_comb * 16)
    lay["pf_items"] = off
    off = a256(off + max_pf * 16)
    lay["pf_base"] = off
    off = a256(off + max_pf * 4)
    lay["pf_seq"] = off
    lay.update(max_dec=max_dec, max_pf=max_pf, max_comb=max_comb, cslot_cap=cslot)
    return lay


def plan_lists(q_lens, k_lens, hq: int, hkv: int, window, max_dec: int, cslot_cap: int, page_size: int,
               cu_k=None):
    """(seq_info, decode items, chunk items, chunk partial bases, combine records) as int32
    arrays, in the planner's order."""
    rpi, quads = geometry(hq, hkv)
    st = split_tiles(q_lens, k_lens, hq, hkv, window)
    keep = keep_tiles(q_lens, k_lens, hq, hkv, window, st)
    seq, dec, comb = [], [], []
    blocks = []  # flat order: (tiles per item, chunk items, their partial bases)
    q0 = 0
    slot = 0
    for b, (n, L) in enumerate(zip(q_lens, k_lens)):
        kvb = 0 if page_size > 0 else int(cu_k[b])
        seq.append((q0, n, L, kvb))
        if n == 1:
            first, splits = decode_splits(L, window[0])
            d0 = len(dec)
            dec += [(b, first + k, q0, L) for k in range(splits)]
            if splits > 1:
                comb.append((b, d0, splits, q0))
        elif n >= 2:
            for blk in reversed(range(_ceil(n, rpi))):
                row0 = blk * rpi
                S = split_count(chunk_tiles(n, L, row0, rpi, window), st, keep)
                rows = min(rpi, n - row0)
                assert S == 1 or slot + rows * S <= cslot_cap, "model cases must fit the slots"
                tiles = chunk_tiles(n, L, row0, rpi, window)
                items = [(b, row0, hq_i, sp | ((S - 1) << 16)) for hq_i in range(quads) for sp in range(S)]
                blocks.append((_ceil(tiles, S), items, [slot] * len(items)))
                if S > 1:
                    for r in range(0, rows, COMB_ROWS):
                        nr = min(COMB_ROWS, rows - r)
                        comb.append((b, max_dec + slot + r * S, S | ((nr - 1) << 24), q0 + row0 + r))
                    slot += rows * S
        q0 += n
    if len(blocks) <= SORT_BLOCKS:
        blocks.sort(key=lambda blk: -blk[0])  # stable: ties keep the flat order
    pf = [it for blk in blocks for it in blk[1]]
    pfb = [base for blk in blocks for base in blk[2]]
    as_arr = lambda x, w: np.array(x, dtype=np.int64).reshape(-1, w).astype(np.int32)  # noqa: E731
    return as_arr(seq, 4), as_arr(dec, 4), as_arr(pf, 4), np.array(pfb, dtype=np.int32), as_arr(comb, 4)
