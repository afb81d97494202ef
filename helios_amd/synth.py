"""Seeded synthetic workloads for the paged-KV hot path at Qwen3-4B shape.

Inputs come from a counter-based SplitMix64 stream turned into N(0, 1) by
Box-Muller, written here with numpy so the same seed gives the same inputs on any
machine and numpy version (small cases). Large pools for benchmarks are filled on
the device with ``torch.randn`` from a seeded generator instead.

Workloads (the five benchmark configurations):
  c1  4 sequences with cached lengths 37, 256, 300, 611, one new token each,
      16-page pool, page tables from a seeded permutation of the pool.
  c2  64 decode sequences, cached length uniform in [512, 4096], 2048-page pool.
  c3  32 decode sequences (cached 1k-4k) + chunks of 1024 tokens at 0 and 992 at 512.
  c4  8 decode sequences at 32768 keys whose first 16 pages are shared, + a
      4096-token chunk at positions 4096-8191 whose first 16 pages are a copy.
  c5  (request caches on a real pool) 128 decoders, contexts uniform in [1024, 8192],
      each holding min(16, cached // 256) pages of one 4096-token prefix, + one
      request that has cached that prefix and prefills a 1024-token chunk.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Outputs ``offset .. offset+count-1`` of the SplitMix64 stream started at ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Doubles in (0, 1] from the top 53 bits of the stream."""
    z = splitmix64(seed, count, offset) >> np.uint64(11)
    return (z.astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape: tuple[int, ...], dtype=np.float32) -> np.ndarray:
    """N(0, 1) samples by Box-Muller over consecutive pairs of the stream."""
    n = int(np.prod(shape)) if shape else 1
    pairs = (n + 1) // 2
    u = uniform01(seed, 2 * pairs)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    theta = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(theta)
    z[1::2] = r * np.sin(theta)
    return z[:n].reshape(shape).astype(dtype)


def randint(seed: int, count: int, low: int, high: int) -> np.ndarray:
    """Integers uniform in [low, high] (inclusive)."""
    span = np.uint64(high - low + 1)
    return (splitmix64(seed, count) % span).astype(np.int64) + low


def permutation(seed: int, n: int) -> np.ndarray:
    """A seeded permutation of range(n) (argsort of distinct 64-bit keys)."""
    keys = splitmix64(seed, n)
    return np.argsort(keys, kind="stable").astype(np.int64)


@dataclass
class Workload:
    """One tick of one attention layer: per-sequence query rows and key lengths."""

    name: str
    q_lens: list[int]            # query rows of each sequence this tick (n_b)
    cached: list[int]            # keys already in the cache before the tick
    tables: list[list[int]]      # physical page ids, logical page order
    num_pages: int
    page_size: int = 256
    n_q_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    seed: int = 0
    shared_prefix_pages: int = 0  # pages at the head of every table that are shared
    notes: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return len(self.q_lens)

    @property
    def k_lens(self) -> list[int]:
        return [c + n for c, n in zip(self.cached, self.q_lens)]

    @property
    def total_q(self) -> int:
        return sum(self.q_lens)

    @property
    def max_q(self) -> int:
        return max(self.q_lens)

    @property
    def max_k(self) -> int:
        return max(self.k_lens)

    @property
    def cu_seq_q(self) -> list[int]:
        out = [0]
        for n in self.q_lens:
            out.append(out[-1] + n)
        return out

    @property
    def cu_seq_k(self) -> list[int]:
        out = [0]
        for n in self.k_lens:
            out.append(out[-1] + n)
        return out

    def block_table(self, width: int | None = None) -> np.ndarray:
        width = width or max(len(t) for t in self.tables)
        bt = np.zeros((self.batch, width), dtype=np.int32)
        for b, t in enumerate(self.tables):
            bt[b, : len(t)] = t
        return bt

    def write_slots(self) -> np.ndarray:
        """Flat pool slot of every new token, in packed query order (int64)."""
        slots = []
        for b in range(self.batch):
            for pos in range(self.cached[b], self.cached[b] + self.q_lens[b]):
                slots.append(self.tables[b][pos // self.page_size] * self.page_size + pos % self.page_size)
        return np.asarray(slots, dtype=np.int64)

    def positions(self) -> np.ndarray:
        return np.concatenate(
            [np.arange(c, c + n, dtype=np.int64) for c, n in zip(self.cached, self.q_lens)]
        ) if self.batch else np.zeros(0, dtype=np.int64)

    def unique_pages(self) -> int:
        return len({p for t in self.tables for p in t})

    def decode_bytes(self, elem_bytes: int = 2) -> int:
        """Algorithmic HBM bytes of the decode rows (n == 1): every visible key's K and V
        for all KV heads (shared pages counted once), q read and o written."""
        row = self.n_kv_heads * self.head_dim * elem_bytes
        seen: set[int] = set()
        keys = 0
        for b in range(self.batch):
            if self.q_lens[b] != 1:
                continue
            L = self.k_lens[b]
            for lp in range((L + self.page_size - 1) // self.page_size):
                page = self.tables[b][lp]
                if page in seen:
                    continue
                seen.add(page)
                keys += min(self.page_size, L - lp * self.page_size)
        n_dec = sum(1 for n in self.q_lens if n == 1)
        qo = 2 * n_dec * self.n_q_heads * self.head_dim * elem_bytes
        return 2 * keys * row + qo

    def append_bytes(self, elem_bytes: int = 2) -> int:
        """KV append: read the new K and V rows and write them into the pool."""
        return 2 * 2 * self.total_q * self.n_kv_heads * self.head_dim * elem_bytes

    def chunk_flops(self) -> int:
        """QK^T + PV flops of the chunk rows (n > 1) over their visible keys."""
        visible = 0
        for n, L in zip(self.q_lens, self.k_lens):
            if n <= 1:
                continue
            off = L - n
            visible += sum(off + i + 1 for i in range(n))
        return 4 * self.n_q_heads * self.head_dim * visible


def _assign_pages(lengths: list[int], free: list[int], page_size: int) -> list[list[int]]:
    tables = []
    cursor = 0
    for L in lengths:
        need = (L + page_size - 1) // page_size
        tables.append([int(p) for p in free[cursor:cursor + need]])
        cursor += need
    if cursor > len(free):
        raise ValueError("pool too small for the workload")
    return tables


def c1(seed: int = 1) -> Workload:
    cached = [37, 256, 300, 611]
    q_lens = [1, 1, 1, 1]
    num_pages = 16
    free = list(permutation(seed, num_pages))
    tables = _assign_pages([c + n for c, n in zip(cached, q_lens)], free, 256)
    return Workload("c1", q_lens, cached, tables, num_pages, seed=seed)


def c2(seed: int = 2, batch: int = 64, num_pages: int = 2048) -> Workload:
    cached = [int(x) for x in randint(seed, batch, 512, 4096)]
    q_lens = [1] * batch
    free = list(permutation(seed + 1000, num_pages))
    tables = _assign_pages([c + 1 for c in cached], free, 256)
    return Workload("c2", q_lens, cached, tables, num_pages, seed=seed)


def c3(seed: int = 3, num_pages: int = 2048) -> Workload:
    dec_cached = [int(x) for x in randint(seed, 32, 1024, 4096)]
    cached = dec_cached + [0, 512]
    q_lens = [1] * 32 + [1024, 992]
    free = list(permutation(seed + 1000, num_pages))
    tables = _assign_pages([c + n for c, n in zip(cached, q_lens)], free, 256)
    return Workload("c3", q_lens, cached, tables, num_pages, seed=seed)


def c4(seed: int = 4, num_pages: int = 1024) -> Workload:
    """8 decoders at 32768 keys sharing their first 16 pages, plus a 4096-token chunk
    at positions 4096..8191 whose first 16 pages are private copies of the prefix."""
    free = list(permutation(seed + 1000, num_pages))
    shared = free[:16]
    cursor = 16
    tables = []
    for _ in range(8):
        tables.append(shared + free[cursor:cursor + 112])
        cursor += 112
    copied = free[cursor:cursor + 16]
    cursor += 16
    chunk_new = free[cursor:cursor + 16]
    cursor += 16
    tables.append(copied + chunk_new)
    cached = [32767] * 8 + [4096]
    q_lens = [1] * 8 + [4096]
    w = Workload("c4", q_lens, cached, tables, num_pages, seed=seed, shared_prefix_pages=16)
    w.notes["prefix_src"] = shared
    w.notes["prefix_dst"] = copied
    return w


def small_mixed(seed: int, *, n_q_heads: int = 32, n_kv_heads: int = 8, batch: int = 6,
                max_cached: int = 900, max_chunk: int = 200, num_pages: int = 64,
                page_size: int = 256, head_dim: int = 128) -> Workload:
    """A random mixed tick small enough for the float64 oracle in a second."""
    kinds = splitmix64(seed, 3 * batch)
    q_lens, cached = [], []
    for b in range(batch):
        if int(kinds[3 * b]) % 2 == 0:
            q_lens.append(1)
        else:
            q_lens.append(2 + int(kinds[3 * b + 1]) % (max_chunk - 1))
        cached.append(int(kinds[3 * b + 2]) % (max_cached + 1))
    free = list(permutation(seed + 7, num_pages))
    tables = _assign_pages([c + n for c, n in zip(cached, q_lens)], free, page_size)
    return Workload(f"mixed{seed}", q_lens, cached, tables, num_pages, page_size=page_size,
                    n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, head_dim=head_dim, seed=seed)


def host_inputs(w: Workload, dtype=np.float32) -> dict[str, np.ndarray]:
    """q [T, Hq, d], new k / v [T, Hkv, d], pools [P, S, Hkv, d] from the seed."""
    s = w.seed * 7919
    T = w.total_q
    return {
        "q": normal(s + 1, (T, w.n_q_heads, w.head_dim), dtype),
        "k_new": normal(s + 2, (T, w.n_kv_heads, w.head_dim), dtype),
        "v_new": normal(s + 3, (T, w.n_kv_heads, w.head_dim), dtype),
        "k_pool": normal(s + 4, (w.num_pages, w.page_size, w.n_kv_heads, w.head_dim), dtype),
        "v_pool": normal(s + 5, (w.num_pages, w.page_size, w.n_kv_heads, w.head_dim), dtype),
    }


# ----------------------------------------------------------------- c5: request caches
C5_PREFIX_PAGES = 16


def c5_lengths(seed: int = 5, decoders: int = 128, chunk: int = 1024,
               prefix_pages: int = C5_PREFIX_PAGES) -> tuple[list[int], list[int]]:
    """Cached lengths and tokens this tick of the full-model tick: ``decoders`` requests
    whose contexts are uniform in [1024, 8192] (cached = context - 1, one decode token)
    and one request that has cached the whole prefix and prefills ``chunk`` tokens."""
    rng = np.random.default_rng(seed)
    contexts = [int(x) for x in rng.integers(1024, 8193, decoders)]
    return [c - 1 for c in contexts] + [prefix_pages * 256], [1] * decoders + [chunk]


def c5_pool_pages(lengths: list[int], counts: list[int], prefix_pages: int = C5_PREFIX_PAGES,
                  page_size: int = 256) -> int:
    """Pool pages the tick needs: the prefix, each request's own pages after the tick,
    and one spare page per request (a tick that crosses a page boundary)."""
    own = sum(-(-(n + c) // page_size) - min(prefix_pages, n // page_size) + 1
              for n, c in zip(lengths, counts))
    return prefix_pages + own + 8


def shared_prefix_caches(pool, lengths: list[int], prefix_pages: int = C5_PREFIX_PAGES):
    """A prefix request of ``prefix_pages`` full pages and one request cache per entry of
    ``lengths`` that holds min(prefix_pages, length // page_size) of its pages (the same
    page handles, as a prefix-cache restore leaves them) and owns the rest. Page
    contents are whatever the pool holds. Returns (prefix, caches)."""
    from helios_amd.paged_cache import PagedKVCache

    size = pool.page_size
    limit = pool.config.context_length
    prefix = PagedKVCache(pool, limit)
    prefix.pages.extend(pool.acquire(prefix_pages))
    prefix.length = prefix_pages * size
    caches = []
    for n in lengths:
        cache = PagedKVCache(pool, limit)
        shared = min(prefix_pages, n // size)
        cache.pages.extend(prefix.pages[:shared])
        cache.pages.extend(pool.acquire(-(-n // size) - shared))
        cache.length = n
        caches.append(cache)
    return prefix, caches
