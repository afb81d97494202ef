// Paged varlen GQA attention for gfx950 (MI355X).
//
// Replaces torch varlen_attn(..., block_table=..., seqused_k=..., window_size=(-1, 0))
// as called by the reference at src/helios/runtime/qwen3/paged_cache.py:316-329 and
// :506-519; its CPU restatement (the semantics matched here) is paged_cache.py:378-414
// and :521-546.
//
// Kernels, all launched on the caller's stream:
//   plan_kernel     one workgroup: validates the metadata, classifies every sequence as
//                   a decode row (one query token) or a chunk (several), and writes the
//                   work lists into the workspace. Run once per tick, reused per layer.
//   decode_kernel   one workgroup per (256-key split, KV head). The G query heads of the
//                   KV group share one read of the split's K and V (64 KiB each at
//                   Qwen3-4B shape), streamed by buffer loads as whole 256-byte rows per
//                   16-lane group, the four waves interleaved over 16-token blocks.
//                   QK^T runs on VALU dot2 with a DPP reduce-scatter across the 16 lanes;
//                   each wave keeps its own softmax max and sum; PV runs on VALU dot2
//                   over token pairs with P rounded to the element type; the waves'
//                   (max, sum, o) merge once through LDS.
//                   A sequence that fits one split writes its output directly; longer ones
//                   write partials: fp32 (m, l) and o / l rounded to the element type (the
//                   partial stores cost more than their 1.6% of the bytes suggests, so they
//                   are 16-bit; the extra error is one more rounding of the output in its
//                   own precision).
//   chunk_kernel    prefill chunks: 8 waves per workgroup (2 per SIMD), each wave owning
//                   32 query rows of one head; 64-key K / V tiles are copied from HBM
//                   straight into LDS (the next tile's copies in flight while the current
//                   one is consumed; V read back transposed); S^T = K Q^T and O^T = V^T P^T
//                   both run on 16x16x32 MFMA with online softmax in between. When the chunk
//                   rows alone would not fill the GPU, row blocks are split over their key
//                   tiles and write partials like decode splits.
//   combine_kernel  merges the partials of each long decode row and each split chunk row
//                   in split order, so results do not depend on scheduling. Runs last.
//                   Given a shared-prefix cascade merge, it also folds the cascade's level
//                   results into the member rows: in the member's combine record, or, for
//                   a member whose row has one split, in workgroups after the records.

#include "hx_common.h"

#include <math.h>

#include <mutex>
#include <type_traits>

namespace {

constexpr int kD = 128;          // head_dim built
constexpr int kSplit = 256;      // keys per decode workgroup
constexpr int kThreads = 256;    // 4 wavefronts
constexpr int kXcds = 8;         // XCDs of an MI355X (gfx950); workgroups are dealt round-robin
constexpr int kTile = 64;        // keys per chunk-kernel tile
constexpr int kPlanThreads = 1024;
// Chunk split-K: when the chunk work items would launch fewer than kChunkFillWGs
// workgroups, each row block's key tiles are cut into splits of at least
// kMinSplitTiles tiles so that about kChunkFillWGs workgroups run; split partials are
// merged by the combine kernel like decode splits. A CU holds one chunk workgroup
// (228 VGPRs x 8 waves), so workgroups run in rounds of kChunkCUs: when rounding the
// split count per block spills past whole rounds, the split size grows to the smallest
// one that fits them (refine_split_tiles). On the full-model tick this took the 1024-row
// chunk from about 550 workgroups (a third, partial round) to 512: 143 -> 110 us.
// Pieces of 4 tiles: the full-model tick's shared-prefix levels (4 sequences of 69-128
// rows over 3-5 pages) then run in 256 workgroups instead of 144 (chunk 24.5 -> 17.1 us,
// with its combine 32.7 -> 29.2 us); chunks of 2016 rows and more plan as with 8.
constexpr int kChunkFillWGs = 512;
constexpr int kChunkCUs = 256;  // CUs of an MI355X
constexpr int kMinSplitTiles = 4;
constexpr int kMaxChunkSplits = 64;
constexpr int kCombRows = 8;  // output rows per combine record of a split chunk block
constexpr int kAppendWGs = 256;  // append workgroups in a decode launch, at most
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Workspace header words.
enum {
  H_NDEC = 0, H_NPF = 1, H_NCOMB = 2, H_ERR = 3,
  // shape the plan was built for; every run kernel checks it before using the lists
  H_BATCH = 4, H_MAXQ = 5, H_MAXK = 6, H_HQ = 7, H_HKV = 8, H_STAMP = 9,
  H_WORDS = 64
};
constexpr int kPlanStamp = 0x48585031;  // marks a header written by plan_kernel

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Geometry {
  int G, Gw, R, head_quads, rows_per_item;
};

inline Geometry geometry(int hq, int hkv) {
  Geometry g;
  g.G = hq / hkv;
  g.Gw = g.G < 4 ? g.G : 4;
  g.R = 4 / g.Gw;
  g.head_quads = g.G / g.Gw;
  g.rows_per_item = 64 * g.R;
  return g;
}

struct Layout {
  size_t seq_info, dec_items, comb_seqs, pf_items, pf_base, pf_seq, part_ml, part_o, total;
  int64_t max_dec, max_pf, max_comb, cslot_cap;
};

// Partial slots: decode splits use [0, max_dec), chunk split rows [max_dec, + cslot_cap).
// Splitting happens only while the unsplit items launch < kChunkFillWGs workgroups, and
// the split size keeps the split items near that many, so sum over row blocks of the
// split count is below 2 * kChunkFillWGs / (hkv * head_quads); a block has at most
// min(rows_per_item, max_q) rows, so that bounds the chunk partial rows. Each split adds
// at most one item per block and head quad.
inline Layout make_layout(int batch, int max_q, int max_k, int hq, int hkv) {
  const Geometry geo = geometry(hq, hkv);
  Layout l;
  const int64_t splits = max_k > 0 ? ceil_div(max_k, kSplit) : 1;
  l.max_dec = (int64_t)batch * splits;
  l.max_pf = 0;
  l.cslot_cap = 0;
  if (max_q >= 2) {
    l.max_pf = (int64_t)batch * ceil_div(max_q, geo.rows_per_item) * geo.head_quads + 2 * kChunkFillWGs;
    const int64_t block_rows = max_q < geo.rows_per_item ? max_q : geo.rows_per_item;
    l.cslot_cap = ceil_div(2 * kChunkFillWGs, (int64_t)hkv * geo.head_quads) * block_rows;
  }
  l.max_comb = (int64_t)batch + l.cslot_cap;
  size_t off = align256(H_WORDS * sizeof(int32_t));
  l.seq_info = off;  off = align256(off + (size_t)batch * sizeof(int4));
  l.dec_items = off; off = align256(off + (size_t)l.max_dec * sizeof(int4));
  l.comb_seqs = off; off = align256(off + (size_t)l.max_comb * sizeof(int4));
  l.pf_items = off;  off = align256(off + (size_t)l.max_pf * sizeof(int4));
  l.pf_base = off;   off = align256(off + (size_t)l.max_pf * sizeof(int32_t));
  l.pf_seq = off;    off = align256(off + (size_t)l.max_pf * sizeof(int4));
  const int64_t slots = l.max_dec + l.cslot_cap;
  l.part_ml = off;   off = align256(off + (size_t)slots * hq * sizeof(float2));
  l.part_o = off;    off = align256(off + (size_t)slots * hq * kD * sizeof(uint16_t));
  l.total = off;
  return l;
}

// Key tiles [*tb, *te) of the chunk row block starting at row0 (rows_per_item rows) of a
// sequence with n query rows and L keys, under the (left, right) window.
__host__ __device__ inline void chunk_tiles(int n, int L, int row0, int rows_per_item, int win_left,
                                            int win_right, int* tb, int* te) {
  const int off = L - n;
  const int row_end = n < row0 + rows_per_item ? n : row0 + rows_per_item;
  int klo = 0;
  if (win_left >= 0) {
    klo = off + row0 - win_left;
    if (klo < 0) klo = 0;
  }
  int khi = L - 1;
  if (win_right >= 0 && off + row_end - 1 + win_right < khi) khi = off + row_end - 1 + win_right;
  *tb = klo / kTile;
  *te = khi >= klo ? khi / kTile + 1 : *tb;
}

// Tiles per chunk split for a tick whose chunk items total `items` (row blocks x head
// quads) and `tiles` key tiles: 0 when the items already launch kChunkFillWGs
// workgroups (no split).
__host__ __device__ inline int chunk_split_tiles(int64_t tiles, int64_t items, int hkv) {
  if (items == 0 || items * hkv >= kChunkFillWGs) return 0;
  int64_t t = (tiles * hkv + kChunkFillWGs - 1) / kChunkFillWGs;
  return (int)(t > kMinSplitTiles ? t : kMinSplitTiles);
}

__host__ __device__ inline int chunk_split_count(int tiles, int split_tiles, int keep_tiles) {
  if (split_tiles <= 0 || tiles <= keep_tiles) return 1;
  const int s = (tiles + split_tiles - 1) / split_tiles;
  return s < kMaxChunkSplits ? s : kMaxChunkSplits;
}
// Splits of a block at split size st while the split size is searched: every block longer
// than st splits.
__host__ __device__ inline int chunk_split_count(int tiles, int split_tiles) {
  return chunk_split_count(tiles, split_tiles, split_tiles);
}

// Once the split size is set, blocks of at most this many key tiles stay whole: 1.25 times
// the tick's chunk tiles per CU (`tiles` counts each block once per head quad; the launch
// holds hkv workgroups per item), and at least the split size. The planner lists items
// longest first, so these blocks start in the first round and the split pieces of longer
// blocks fill in around them; splitting them too would add partial rows and combine work
// without shortening the longest item. On a tick of chunks of 1024 and 992 rows: combine
// 10.1 -> 4.7 us, the chunk kernel unchanged (42.6 -> 42.4 us).
__host__ __device__ inline int chunk_keep_tiles(int64_t tiles, int hkv, int split_tiles) {
  const int64_t k = (5 * tiles * hkv + 4 * kChunkCUs - 1) / (4 * kChunkCUs);
  return k > split_tiles ? (k < INT32_MAX ? (int)k : INT32_MAX) : split_tiles;
}

// Split size that keeps the chunk workgroups within whole rounds of kChunkCUs. wgs(st)
// is the workgroup count at split size st (non-increasing in st); max_tiles is the
// largest block's tile count (no block splits at that size). From st0, when wgs(st0)
// spills past R >= 1 whole rounds, returns the smallest st whose count fits R rounds,
// if one does; otherwise st0. The plan kernel and the host count call it with the same
// counts, so both reach the same split size.
// Smallest split size in (lo, hi] whose workgroups fit `target`, given wgs(lo) > target;
// 0 when even hi does not fit.
template <typename WgsFn>
__host__ __device__ inline int smallest_fitting_split(int lo, int hi, int64_t target, WgsFn wgs) {
  if (wgs(hi) > target) return 0;
  while (hi - lo > 1) {
    const int mid = lo + (hi - lo) / 2;
    if (wgs(mid) <= target) hi = mid;
    else lo = mid;
  }
  return hi;
}

// One round instead of several: when the smallest split size whose workgroups fit one
// round of kChunkCUs is at most one_round_tiles (1.25 x the chunk tiles per CU,
// chunk_keep_tiles), the pieces are no longer than the blocks the planner keeps whole,
// so one round of them ends about when the longest item would anyway, without a second
// round's fixed costs and with fewer partial rows. Blocks of a chunk far into its
// sequence have nearly equal tile counts: a 1024-row chunk at position 4096 (blocks of
// 65-80 tiles) takes 40-tile splits in 256 workgroups instead of 21-tile splits in 512
// (chunk 88.8 -> 88.1 us, combine 12.8 -> 10.6 us).
template <typename WgsFn>
__host__ __device__ inline int refine_split_tiles(int st0, int max_tiles, int one_round_tiles, WgsFn wgs) {
  if (st0 <= 0 || max_tiles <= st0) return st0;
  int st = st0;
  const int64_t w0 = wgs(st0);
  const int64_t rounds = w0 / kChunkCUs;
  if (rounds >= 1 && w0 % kChunkCUs != 0) {
    const int s = smallest_fitting_split(st0, max_tiles, rounds * kChunkCUs, wgs);
    if (s > 0) st = s;
  }
  if (w0 > kChunkCUs) {
    const int s1 = smallest_fitting_split(st0, max_tiles, kChunkCUs, wgs);
    if (s1 > 0 && s1 <= one_round_tiles) st = s1;
  }
  return st;
}

// Decode key window of a one-token row at position L-1: keys [lo, L).
__host__ __device__ inline int decode_lo(int L, int win_left) {
  if (win_left < 0) return 0;
  const int lo = L - 1 - win_left;
  return lo > 0 ? lo : 0;
}

// Number of 256-key splits a decode row covers, and the first split. A row with no
// keys still gets one (empty) split so its output row is written (zeros).
__host__ __device__ inline void decode_splits(int L, int win_left, int* first, int* count) {
  if (L <= 0) {
    *first = 0;
    *count = 1;
    return;
  }
  const int lo = decode_lo(L, win_left);
  *first = lo / kSplit;
  *count = (L - 1) / kSplit - lo / kSplit + 1;
}

// ------------------------------------------------------------------ plan
struct PlanArgs {
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* used_k;
  int32_t* hdr;
  int4* seq_info;
  int4* dec_items;
  int4* comb_seqs;
  int4* pf_items;
  int32_t* pf_base;
  int4* pf_seq;  // per chunk item: its sequence's seq_info entry, read with the item
  int64_t total_k_rows;
  int64_t max_dec, max_pf, max_comb, cslot_cap;
  int32_t batch, total_q, max_q, max_k;
  int32_t page_size, bt_stride;
  int32_t rows_per_item, head_quads;
  int32_t win_left, win_right;
  int32_t hq, hkv;
};

__device__ int block_exclusive_scan(int v, int* wave_tot, int* total) {
  const int lane = hx::tid_x() & 63, w = hx::tid_x() >> 6, nw = hx::wg_size_x() >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_tot[w] = x;
  __syncthreads();
  int pre = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    const int t = wave_tot[i];
    pre += i < w ? t : 0;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return pre + x - v;
}

// Per-sequence metadata with the bounds checks of every run kernel: rows [q0, q0 + n),
// L keys, packed-key base kvb; error bits for anything clamped.
struct SeqMeta {
  int q0, n, L, kvb;
};
__device__ SeqMeta plan_seq(const PlanArgs& a, int b, int& err) {
  SeqMeta m{0, 0, 0, 0};
  m.q0 = a.cu_q[b];
  const int q1 = a.cu_q[b + 1];
  if (m.q0 < 0 || q1 < m.q0 || q1 > a.total_q) {
    err |= HX_WERR_BAD_CU_SEQ;
    m.q0 = 0;
    m.n = 0;
  } else {
    m.n = q1 - m.q0;
  }
  if (m.n > a.max_q) {
    err |= HX_WERR_CLAMPED_LEN;
    m.n = a.max_q;
  }
  m.L = a.used_k ? a.used_k[b] : a.cu_k[b + 1] - a.cu_k[b];
  if (m.L < 0) {
    err |= HX_WERR_CLAMPED_LEN;
    m.L = 0;
  }
  if (m.L > a.max_k) {
    err |= HX_WERR_CLAMPED_LEN;
    m.L = a.max_k;
  }
  if (a.page_size > 0) {
    const int64_t cap = (int64_t)a.bt_stride * a.page_size;
    if (m.L > cap) {
      err |= HX_WERR_CLAMPED_LEN;
      m.L = (int)cap;
    }
  } else {
    m.kvb = a.cu_k[b];
    if (m.kvb < 0 || m.kvb > a.total_k_rows) {
      err |= HX_WERR_CLAMPED_LEN;
      m.kvb = 0;
      m.L = 0;
    } else if ((int64_t)m.kvb + m.L > a.total_k_rows) {
      err |= HX_WERR_CLAMPED_LEN;
      m.L = (int)(a.total_k_rows - m.kvb);
    }
  }
  return m;
}

// The plan header: item counts (clamped to the lists' capacities), the error word and the
// stamp of the shape the plan was built for.
__device__ void write_plan_header(const PlanArgs& a, int err, int4 totals) {
  const int base_dec = totals.x, base_pf = totals.y, base_comb = totals.z;
  if (base_dec > a.max_dec || base_pf > a.max_pf || base_comb > a.max_comb) err |= HX_WERR_GRID;
  a.hdr[H_NDEC] = base_dec < a.max_dec ? base_dec : (int)a.max_dec;
  a.hdr[H_NPF] = base_pf < a.max_pf ? base_pf : (int)a.max_pf;
  a.hdr[H_NCOMB] = base_comb < a.max_comb ? base_comb : (int)a.max_comb;
  a.hdr[H_ERR] = err;
  a.hdr[H_BATCH] = a.batch;
  a.hdr[H_MAXQ] = a.max_q;
  a.hdr[H_MAXK] = a.max_k;
  a.hdr[H_HQ] = a.hq;
  a.hdr[H_HKV] = a.hkv;
  a.hdr[H_STAMP] = kPlanStamp;
}

// The planner's serial form: one thread walks each sequence's row blocks in every pass.
// Used when the chunk sequences or their row blocks exceed the LDS lists of plan_kernel.
__device__ void plan_serial(const PlanArgs& a, int* wave_tot, int* err_bits, int4* totals) {
  int err = 0;

  // Pass 1: chunk work before splitting (items and key tiles, head quads counted; the
  // largest block's tiles).
  __shared__ int max_blk_tiles;
  if (hx::tid_x() == 0) max_blk_tiles = 0;
  __syncthreads();
  int64_t pf_items0 = 0, pf_tiles = 0;
  for (int b0 = 0; b0 < a.batch; b0 += kPlanThreads) {
    const int b = b0 + hx::tid_x();
    int items = 0, tiles = 0, tmax = 0;
    if (b < a.batch) {
      int e = 0;
      const SeqMeta m = plan_seq(a, b, e);
      if (m.n >= 2) {
        for (int row0 = 0; row0 < m.n; row0 += a.rows_per_item) {
          int tb, te;
          chunk_tiles(m.n, m.L, row0, a.rows_per_item, a.win_left, a.win_right, &tb, &te);
          tiles += (te - tb) * a.head_quads;
          items += a.head_quads;
          tmax = max(tmax, te - tb);
        }
      }
    }
    if (tmax > 0) atomicMax(&max_blk_tiles, tmax);  // LDS atomic
    int tot_i, tot_t;
    block_exclusive_scan(items, wave_tot, &tot_i);
    block_exclusive_scan(tiles, wave_tot, &tot_t);
    pf_items0 += tot_i;
    pf_tiles += tot_t;
  }
  __syncthreads();
  // Workgroups of the chunk launch at split size st (a block-wide pass; every thread
  // runs it the same number of times, since the search depends only on block totals).
  auto chunk_wgs = [&](int st) -> int64_t {
    int64_t total = 0;
    for (int b0 = 0; b0 < a.batch; b0 += kPlanThreads) {
      const int b = b0 + hx::tid_x();
      int wg = 0;
      if (b < a.batch) {
        int e = 0;
        const SeqMeta m = plan_seq(a, b, e);
        if (m.n >= 2) {
          for (int row0 = 0; row0 < m.n; row0 += a.rows_per_item) {
            int tb, te;
            chunk_tiles(m.n, m.L, row0, a.rows_per_item, a.win_left, a.win_right, &tb, &te);
            wg += chunk_split_count(te - tb, st) * a.head_quads;
          }
        }
      }
      int tot;
      block_exclusive_scan(wg, wave_tot, &tot);
      total += tot;
    }
    return total * a.hkv;
  };
  const int split_tiles = refine_split_tiles(chunk_split_tiles(pf_tiles, pf_items0, a.hkv), max_blk_tiles,
                                             chunk_keep_tiles(pf_tiles, a.hkv, 0), chunk_wgs);
  const int keep_tiles = chunk_keep_tiles(pf_tiles, a.hkv, split_tiles);

  // Pass 2: work lists.
  int base_dec = 0, base_pf = 0, base_comb = 0, base_slot = 0;
  for (int b0 = 0; b0 < a.batch; b0 += kPlanThreads) {
    const int b = b0 + hx::tid_x();
    const bool active = b < a.batch;
    SeqMeta m{0, 0, 0, 0};
    if (active) m = plan_seq(a, b, err);
    int nd = 0, np = 0, nc = 0, ns = 0, s_first = 0, splits = 0, nblk = 0;
    if (active && m.n == 1) {
      decode_splits(m.L, a.win_left, &s_first, &splits);
      nd = splits;
      nc = splits > 1 ? 1 : 0;
    } else if (active && m.n >= 2) {
      nblk = (m.n + a.rows_per_item - 1) / a.rows_per_item;
      for (int blk = 0; blk < nblk; ++blk) {
        const int row0 = blk * a.rows_per_item;
        int tb, te;
        chunk_tiles(m.n, m.L, row0, a.rows_per_item, a.win_left, a.win_right, &tb, &te);
        const int S = chunk_split_count(te - tb, split_tiles, keep_tiles);
        const int rows = min(a.rows_per_item, m.n - row0);
        np += S * a.head_quads;
        if (S > 1) {
          ns += rows * S;
          nc += (rows + kCombRows - 1) / kCombRows;
        }
      }
    }
    int tot_d, tot_p, tot_c, tot_s;
    const int off_d = base_dec + block_exclusive_scan(nd, wave_tot, &tot_d);
    const int off_p = base_pf + block_exclusive_scan(np, wave_tot, &tot_p);
    const int off_c = base_comb + block_exclusive_scan(nc, wave_tot, &tot_c);
    const int off_s = base_slot + block_exclusive_scan(ns, wave_tot, &tot_s);
    if (active) {
      a.seq_info[b] = make_int4(m.q0, m.n, m.L, m.kvb);
      for (int k = 0; k < nd; ++k) {
        if (off_d + k < a.max_dec) a.dec_items[off_d + k] = make_int4(b, s_first + k, m.q0, m.L);
      }
      if (nc && m.n == 1 && off_c < a.max_comb) a.comb_seqs[off_c] = make_int4(b, off_d, splits, m.q0);
      if (m.n >= 2) {
        // Later row blocks see more keys under a causal mask: list them first. A split
        // block's rows own S consecutive partial slots each, merged by one combine
        // record per row.
        int k = 0, slot = off_s, comb = off_c;
        for (int blk = nblk - 1; blk >= 0; --blk) {
          const int row0 = blk * a.rows_per_item;
          int tb, te;
          chunk_tiles(m.n, m.L, row0, a.rows_per_item, a.win_left, a.win_right, &tb, &te);
          const int S = chunk_split_count(te - tb, split_tiles, keep_tiles);
          const int rows = min(a.rows_per_item, m.n - row0);
          const bool fits = S == 1 || slot + rows * S <= a.cslot_cap;
          if (!fits) err |= HX_WERR_GRID;
          for (int hq = 0; hq < a.head_quads; ++hq) {
            for (int sp = 0; sp < S; ++sp, ++k) {
              if (off_p + k < a.max_pf) {
                a.pf_items[off_p + k] = make_int4(b, row0, hq, fits ? (sp | ((S - 1) << 16)) : 0);
                a.pf_base[off_p + k] = slot;
                a.pf_seq[off_p + k] = make_int4(m.q0, m.n, m.L, m.kvb);
              }
            }
          }
          if (S > 1) {
            for (int r = 0; r < rows; r += kCombRows, ++comb) {
              const int nr = min(kCombRows, rows - r);
              if (fits && comb < a.max_comb)
                a.comb_seqs[comb] = make_int4(b, (int)a.max_dec + slot + r * S, S | ((nr - 1) << 24),
                                              m.q0 + row0 + r);
            }
            slot += rows * S;
          }
        }
      }
    }
    base_dec += tot_d;
    base_pf += tot_p;
    base_comb += tot_c;
    base_slot += tot_s;
  }
  if (err) atomicOr(err_bits, err);
  *totals = make_int4(base_dec, base_pf, base_comb, base_slot);
}


// Inclusive scan (sum, or max when MAX) over the 64 lanes of a wave by DPP: row shifts by
// 1, 2, 4 and 8 within each 16-lane row, then the row broadcasts of lane 15 (to rows 1
// and 3) and lane 31 (to rows 2 and 3). Lanes whose DPP source lies outside the row, or
// whose row is masked off, take the identity.
template <bool MAX>
__device__ __forceinline__ int wave_incl_scan(int x) {
  constexpr int kId = MAX ? INT32_MIN : 0;
  auto op = [](int p, int q) { return MAX ? max(p, q) : p + q; };
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x111, 0xf, 0xf, false));  // row_shr:1
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x112, 0xf, 0xf, false));  // row_shr:2
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x114, 0xf, 0xf, false));  // row_shr:4
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x118, 0xf, 0xf, false));  // row_shr:8
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x142, 0xa, 0xf, false));  // row_bcast:15
  x = op(x, __builtin_amdgcn_update_dpp(kId, x, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return x;
}

// Per-wave totals for block-wide scans, in two buffers used in turn: a buffer is written
// again only two scans later, after a barrier every thread passed once done reading it,
// so each scan needs one barrier.
struct WaveTotals {
  int4 buf[2][kPlanThreads / 64];
};

// Block-wide exclusive scan of four counters at once; *total gets the block sums.
__device__ int4 block_exclusive_scan4(int4 v, WaveTotals& wt, int& turn, int4* total) {
  const int lane = hx::tid_x() & 63, w = hx::tid_x() >> 6, nw = hx::wg_size_x() >> 6;
  int4* t4 = wt.buf[turn];
  turn ^= 1;
  const int4 x = make_int4(wave_incl_scan<false>(v.x), wave_incl_scan<false>(v.y), wave_incl_scan<false>(v.z),
                           wave_incl_scan<false>(v.w));
  if (lane == 63) t4[w] = x;
  __syncthreads();
  int4 pre = make_int4(0, 0, 0, 0), tot = make_int4(0, 0, 0, 0);
  for (int i = 0; i < nw; ++i) {
    const int4 t = t4[i];
    if (i < w) pre = make_int4(pre.x + t.x, pre.y + t.y, pre.z + t.z, pre.w + t.w);
    tot = make_int4(tot.x + t.x, tot.y + t.y, tot.z + t.z, tot.w + t.w);
  }
  *total = tot;
  return make_int4(pre.x + x.x - v.x, pre.y + x.y - v.y, pre.z + x.z - v.z, pre.w + x.w - v.w);
}

// Block-wide sum of v and max of m.
__device__ int2 block_sum_max(int v, int m, WaveTotals& wt, int& turn) {
  const int lane = hx::tid_x() & 63, w = hx::tid_x() >> 6, nw = hx::wg_size_x() >> 6;
  int4* t4 = wt.buf[turn];
  turn ^= 1;
  const int sv = __builtin_amdgcn_readlane(wave_incl_scan<false>(v), 63);
  const int mv = __builtin_amdgcn_readlane(wave_incl_scan<true>(m), 63);
  if (lane == 0) t4[w] = make_int4(sv, mv, 0, 0);
  __syncthreads();
  int s = 0, mx = INT32_MIN;
  for (int i = 0; i < nw; ++i) {
    s += t4[i].x;
    mx = max(mx, t4[i].y);
  }
  return make_int2(s, mx);
}

// Work planner: one workgroup. Each sequence is a decode row (n == 1: one work item per
// 256-key split) or a chunk (n >= 2: row blocks of rows_per_item rows, each one work item
// per head quad, or several when the tick's chunk items alone would not fill the GPU
// and blocks are split over their key tiles; see chunk_split_tiles / refine_split_tiles).
//
// The row blocks of all chunks are listed in LDS once (kPlanBlocks at most, over at most
// kPlanChunkSeqs chunk sequences) in flat order: sequences in order, each sequence's
// blocks from the last to the first (later blocks see more keys under a causal mask).
// Every pass over them runs on all threads: the split-size search sums split counts over
// the list, and a scan over the list gives each block its partial-slot and
// combine-record offsets. Chunk items follow the flat order, except that a tick of at
// most kPlanSortBlocks blocks lists them longest first (see phase 5). Larger ticks take
// the serial walk (plan_serial), which produces the same lists.
constexpr int kPlanChunkSeqs = 1024;
constexpr int kPlanBlocks = 4096;
constexpr int kPlanSearchWork = 1 << 16;  // candidates x blocks evaluated in one pass
constexpr int kPlanSortBlocks = 256;
static_assert(2 * kPlanSortBlocks <= kPlanThreads, "sort keys and item counts share the search buffer");

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanArgs a) {
  __shared__ int wave_tot[kPlanThreads / 64];
  __shared__ WaveTotals wt;
  __shared__ int err_bits;
  __shared__ int cand_wgs[kPlanThreads];  // split-size search: workgroups per candidate
  __shared__ int best_st, best_one;
  // Chunk sequence k: its sequence index, first row, clamped (n, L), first flat block, and its item /
  // combine-record / partial-slot offsets once known.
  __shared__ int cs_b[kPlanChunkSeqs], cs_q0[kPlanChunkSeqs], cs_n[kPlanChunkSeqs], cs_L[kPlanChunkSeqs];
  __shared__ int cs_kvb[kPlanChunkSeqs];
  __shared__ int cs_first[kPlanChunkSeqs + 1];
  __shared__ int cs_off_p[kPlanChunkSeqs], cs_off_c[kPlanChunkSeqs], cs_off_s[kPlanChunkSeqs];
  // Flat block i: key tiles, then (after the split) its offsets within the flat order.
  __shared__ int fb_tiles[kPlanBlocks], fb_p[kPlanBlocks + 1], fb_c[kPlanBlocks + 1], fb_s[kPlanBlocks + 1];
  const int tid = hx::tid_x();
  if (tid == 0) {  // published by the barrier of phase 0's scan
    err_bits = 0;
    best_st = INT32_MAX;
    best_one = INT32_MAX;
  }
  int err = 0;
  int turn = 0;  // WaveTotals buffer of the next block-wide scan

  // Phase 0: list the chunk sequences and count their row blocks. A batch of one round
  // keeps each thread's sequence metadata and chunk sequence index for phase 4.
  int n_cs = 0, n_blk = 0;
  SeqMeta m_kept{0, 0, 0, 0};
  int k_kept = 0;
  for (int b0 = 0; b0 < a.batch; b0 += kPlanThreads) {
    const int b = b0 + tid;
    SeqMeta m{0, 0, 0, 0};
    if (b < a.batch) m = plan_seq(a, b, err);
    m_kept = m;
    const int is_chunk = b < a.batch && m.n >= 2;
    const int nblk = is_chunk ? (m.n + a.rows_per_item - 1) / a.rows_per_item : 0;
    int4 tot;
    const int4 pre = block_exclusive_scan4(make_int4(is_chunk, nblk, 0, 0), wt, turn, &tot);
    const int k = n_cs + pre.x;
    k_kept = k;
    if (is_chunk && k < kPlanChunkSeqs) {
      cs_b[k] = b;
      cs_q0[k] = m.q0;
      cs_n[k] = m.n;
      cs_L[k] = m.L;
      cs_kvb[k] = m.kvb;
      cs_first[k] = n_blk + pre.y;
    }
    n_cs += tot.x;
    n_blk += tot.y;
  }
  if (n_cs > kPlanChunkSeqs || n_blk > kPlanBlocks) {
    int4 totals;
    plan_serial(a, wave_tot, &err_bits, &totals);
    if (err) atomicOr(&err_bits, err);
    __syncthreads();
    if (tid == 0) write_plan_header(a, err_bits, totals);
    return;
  }
  if (tid == 0) cs_first[n_cs] = n_blk;
  __syncthreads();

  // Flat block i -> chunk sequence k (the last k with cs_first[k] <= i) and row block.
  auto block_of = [&](int i, int& k, int& blk) {
    int lo = 0, hi = n_cs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cs_first[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    k = lo;
    const int nblk = cs_first[k + 1] - cs_first[k];
    blk = nblk - 1 - (i - cs_first[k]);
  };

  // Phase 1: key tiles of every block; totals before splitting. (The chunk-free branches
  // below are workgroup-uniform.)
  int2 tm = make_int2(0, 0);
  if (n_blk > 0) {
    int my_tiles = 0, my_max = 0;
    for (int i = tid; i < n_blk; i += kPlanThreads) {
      int k, blk;
      block_of(i, k, blk);
      int tb, te;
      chunk_tiles(cs_n[k], cs_L[k], blk * a.rows_per_item, a.rows_per_item, a.win_left, a.win_right, &tb, &te);
      fb_tiles[i] = te - tb;
      my_tiles += te - tb;
      my_max = max(my_max, te - tb);
    }
    tm = block_sum_max(my_tiles, my_max, wt, turn);  // its barrier publishes fb_tiles
  }
  const int64_t pf_items0 = (int64_t)n_blk * a.head_quads;
  const int64_t pf_tiles = (int64_t)tm.x * a.head_quads;

  // Phase 2: split size, as refine_split_tiles (the host count uses that). wgs(st) is
  // non-increasing, so its binary search finds the smallest st in (st0, max] whose
  // workgroups fit the target; when candidates x blocks is small, every candidate is
  // evaluated at once (one per thread) and the smallest fitting one taken.
  auto chunk_wgs = [&](int st) -> int64_t {
    int wg = 0;
    for (int i = tid; i < n_blk; i += kPlanThreads) wg += chunk_split_count(fb_tiles[i], st);
    return (int64_t)block_sum_max(wg, 0, wt, turn).x * a.head_quads * a.hkv;
  };
  const int st0 = chunk_split_tiles(pf_tiles, pf_items0, a.hkv);
  int split_tiles = st0;
  if (st0 > 0 && tm.y > st0) {
    const int ncand = tm.y - st0;  // candidates st0 + 1 .. max tiles
    if (ncand < kPlanThreads && (int64_t)(ncand + 1) * n_blk <= kPlanSearchWork) {
      // Thread j <= ncand counts the workgroups at split size st0 + j; the smallest
      // fitting candidate wins an LDS atomicMin.
      if (tid <= ncand) {
        int wg = 0;
        for (int i = 0; i < n_blk; ++i) wg += chunk_split_count(fb_tiles[i], st0 + tid);
        cand_wgs[tid] = wg;
      }
      __syncthreads();
      const int64_t w0 = (int64_t)cand_wgs[0] * a.head_quads * a.hkv;
      const int64_t rounds = w0 / kChunkCUs;
      if (rounds >= 1 && w0 % kChunkCUs != 0) {
        if (tid >= 1 && tid <= ncand && (int64_t)cand_wgs[tid] * a.head_quads * a.hkv <= rounds * kChunkCUs)
          atomicMin(&best_st, st0 + tid);
        __syncthreads();
        if (best_st != INT32_MAX) split_tiles = best_st;
      }
      // One round instead, as refine_split_tiles.
      if (w0 > kChunkCUs) {
        if (tid >= 1 && tid <= ncand && (int64_t)cand_wgs[tid] * a.head_quads * a.hkv <= kChunkCUs)
          atomicMin(&best_one, st0 + tid);
        __syncthreads();
        if (best_one <= chunk_keep_tiles(pf_tiles, a.hkv, 0)) split_tiles = best_one;
      }
    } else {
      split_tiles = refine_split_tiles(st0, tm.y, chunk_keep_tiles(pf_tiles, a.hkv, 0), chunk_wgs);
    }
  }

  const int keep_tiles = chunk_keep_tiles(pf_tiles, a.hkv, split_tiles);

  // Phase 3: per block, items (S per head quad), partial rows (rows * S when split) and
  // combine records (one per kCombRows split rows); exclusive scans in flat order.
  if (n_blk > 0) {
    int base_p = 0, base_c = 0, base_s = 0;
    for (int i0 = 0; i0 < n_blk; i0 += kPlanThreads) {
      const int i = i0 + tid;
      int4 v = make_int4(0, 0, 0, 0);
      if (i < n_blk) {
        int k, blk;
        block_of(i, k, blk);
        const int S = chunk_split_count(fb_tiles[i], split_tiles, keep_tiles);
        const int rows = min(a.rows_per_item, cs_n[k] - blk * a.rows_per_item);
        v.x = S * a.head_quads;
        if (S > 1) {
          v.y = (rows + kCombRows - 1) / kCombRows;
          v.z = rows * S;
        }
      }
      int4 tot;
      const int4 pre = block_exclusive_scan4(v, wt, turn, &tot);
      if (i < n_blk) {
        fb_p[i] = base_p + pre.x;
        fb_c[i] = base_c + pre.y;
        fb_s[i] = base_s + pre.z;
      }
      base_p += tot.x;
      base_c += tot.y;
      base_s += tot.z;
    }
    if (tid == 0) {
      fb_p[n_blk] = base_p;
      fb_c[n_blk] = base_c;
      fb_s[n_blk] = base_s;
    }
    __syncthreads();
  }

  // Phase 4: per sequence, item counts and offsets; decode items and sequence info.
  int base_dec = 0, base_pf = 0, base_comb = 0, base_slot = 0;
  int kc = 0;  // chunk sequences before this b0 round
  for (int b0 = 0; b0 < a.batch; b0 += kPlanThreads) {
    const int b = b0 + tid;
    const bool active = b < a.batch;
    SeqMeta m = m_kept;
    if (active && a.batch > kPlanThreads) m = plan_seq(a, b, err);
    const int is_chunk = active && m.n >= 2;
    int4 cnt = make_int4(0, 0, 0, 0);  // decode items, chunk items, combine records, slots
    int s_first = 0, splits = 0;
    if (active && m.n == 1) {
      decode_splits(m.L, a.win_left, &s_first, &splits);
      cnt.x = splits;
      cnt.z = splits > 1 ? 1 : 0;
    }
    // The chunk sequence index of b: the same compaction as phase 0.
    int k = k_kept;
    if (n_cs > 0 && a.batch > kPlanThreads) {
      int4 ctot;
      k = kc + block_exclusive_scan4(make_int4(is_chunk, 0, 0, 0), wt, turn, &ctot).x;
      kc += ctot.x;
    }
    if (is_chunk) {
      const int f0 = cs_first[k], f1 = cs_first[k + 1];
      cnt.y = fb_p[f1] - fb_p[f0];
      cnt.z = fb_c[f1] - fb_c[f0];
      cnt.w = fb_s[f1] - fb_s[f0];
    }
    int4 tot;
    const int4 pre = block_exclusive_scan4(cnt, wt, turn, &tot);
    const int off_d = base_dec + pre.x, off_p = base_pf + pre.y;
    const int off_c = base_comb + pre.z, off_s = base_slot + pre.w;
    if (active) {
      a.seq_info[b] = make_int4(m.q0, m.n, m.L, m.kvb);
      for (int j = 0; j < cnt.x; ++j) {
        if (off_d + j < a.max_dec) a.dec_items[off_d + j] = make_int4(b, s_first + j, m.q0, m.L);
      }
      if (cnt.z && m.n == 1 && off_c < a.max_comb) a.comb_seqs[off_c] = make_int4(b, off_d, splits, m.q0);
      if (is_chunk) {
        cs_off_p[k] = off_p;
        cs_off_c[k] = off_c;
        cs_off_s[k] = off_s;
      }
    }
    base_dec += tot.x;
    base_pf += tot.y;
    base_comb += tot.z;
    base_slot += tot.w;
  }
  __syncthreads();

  // Phase 5: chunk items, their first partial rows, and combine records, one block per
  // thread. A split block's rows own S consecutive partial slots each; its combine
  // records cover kCombRows rows each. A block's items stay together (head quads, then
  // splits). With at most kPlanSortBlocks blocks the blocks go longest first: by key
  // tiles per item, descending, ties in flat order. Workgroups start in index order as
  // CUs free up, so the short items fill the last round instead of the long ones
  // (greedy longest-first scheduling); on a tick of two chunks of 1024 and 992 rows the
  // chunk kernel's 512 split workgroups otherwise end with a sequence's long blocks.
  const bool by_length = n_blk > 0 && n_blk <= kPlanSortBlocks;
  int* const blk_key = cand_wgs;                      // free after the split search
  int* const blk_items = cand_wgs + kPlanSortBlocks;
  if (by_length) {
    if (tid < n_blk) {
      const int S = chunk_split_count(fb_tiles[tid], split_tiles, keep_tiles);
      blk_key[tid] = (fb_tiles[tid] + S - 1) / S;
      blk_items[tid] = S * a.head_quads;
    }
    __syncthreads();
  }
  for (int i = tid; i < n_blk; i += kPlanThreads) {
    int k, blk;
    block_of(i, k, blk);
    const int f0 = cs_first[k];
    const int b = cs_b[k], n = cs_n[k];
    const int row0 = blk * a.rows_per_item;
    const int S = chunk_split_count(fb_tiles[i], split_tiles, keep_tiles);
    const int rows = min(a.rows_per_item, n - row0);
    int item0 = cs_off_p[k] + fb_p[i] - fb_p[f0];
    if (by_length) {
      const int key = blk_key[i];
      item0 = 0;
      for (int j = 0; j < n_blk; ++j) {
        const int kj = blk_key[j];
        item0 += kj > key || (kj == key && j < i) ? blk_items[j] : 0;
      }
    }
    const int slot = cs_off_s[k] + fb_s[i] - fb_s[f0];
    const int comb0 = cs_off_c[k] + fb_c[i] - fb_c[f0];
    const bool fits = S == 1 || slot + rows * S <= a.cslot_cap;
    if (!fits) err |= HX_WERR_GRID;
    for (int hq = 0, j = 0; hq < a.head_quads; ++hq) {
      for (int sp = 0; sp < S; ++sp, ++j) {
        if (item0 + j < a.max_pf) {
          a.pf_items[item0 + j] = make_int4(b, row0, hq, fits ? (sp | ((S - 1) << 16)) : 0);
          a.pf_base[item0 + j] = slot;
          a.pf_seq[item0 + j] = make_int4(cs_q0[k], n, cs_L[k], cs_kvb[k]);
        }
      }
    }
    if (S > 1) {
      const int q0 = cs_q0[k];
      for (int r = 0, comb = comb0; r < rows; r += kCombRows, ++comb) {
        const int nr = min(kCombRows, rows - r);
        if (fits && comb < a.max_comb)
          a.comb_seqs[comb] = make_int4(b, (int)a.max_dec + slot + r * S, S | ((nr - 1) << 24), q0 + row0 + r);
      }
    }
  }
  if (err) atomicOr(&err_bits, err);
  __syncthreads();
  if (tid == 0) write_plan_header(a, err_bits, make_int4(base_dec, base_pf, base_comb, base_slot));
}

// ------------------------------------------------------------------ run arguments
struct RunArgs {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  uint8_t* out;
  float* lse;
  const int32_t* bt;
  int32_t* hdr;
  const int4* seq_info;
  const int4* dec_items;
  const int4* comb_seqs;
  const int4* pf_items;
  const int32_t* pf_base;  // per chunk item: first partial row of its block (split blocks)
  const int4* pf_seq;      // per chunk item: its sequence's seq_info entry
  float2* part_ml;   // per (slot, head): running max m (log2 units) and sum l
  uint16_t* part_o;  // per (slot, head, dim): o / l in the element type T
  int64_t dec_cap;   // decode slots [0, dec_cap); chunk split rows follow
  int64_t slot_cap;  // all partial slots
  int64_t q_row, q_head;     // element strides
  int64_t kv_row, kv_head;
  int64_t o_row, o_head;
  int32_t num_pages, page_size, bt_stride;
  int32_t batch, max_q, max_k;
  int32_t total_q, hq, hkv;
  float scale_log2;
  int32_t win_left, win_right;
  int32_t grid_dec, grid_pf, grid_comb;  // work items the launch grids cover
  // Fused KV append of decode rows (k_new == nullptr: none). Row t of k_new / v_new is
  // the new key / value of packed query row t; it goes to pool row write_slots[t].
  const uint8_t* k_new;
  const uint8_t* v_new;
  const int64_t* write_slots;
  int64_t kn_row, kn_head, vn_row, vn_head;  // element strides
  int64_t pool_rows;
  // Workgroups after the decode workgroups of the decode launch that append every row of
  // the tick (0: none; the chunk rows then went in by a separate append beforehand).
  int32_t app_wgs;
  // Query row of each packed row (nullptr: the packed row itself); q holds q_rows_total
  // rows when the map is given.
  const int64_t* q_rows;
  int64_t q_rows_total;
  // Shared-prefix cascade merge done by the combine launch (mg_start == nullptr: none).
  // Member k is the decode row of sequence mg_seq[k] (mg_of_seq[b]: sequence b's member
  // index, or -1); it folds the level results mg_idx[mg_start[k]] .. mg_idx[mg_start[k+1]
  // - 1] (rows of mg_o, log-sum-exps mg_lse[h * mg_lse_stride + row], mg_rows rows) into
  // its own result by log-sum-exp.
  const uint16_t* mg_o;
  int64_t mg_o_row, mg_o_head;
  const float* mg_lse;
  int64_t mg_lse_stride, mg_rows;
  const int32_t* mg_seq;
  const int32_t* mg_of_seq;
  const int32_t* mg_start;
  const int32_t* mg_idx;
  int32_t mg_members, mg_n_idx;
  // Combine records of a second plan (a cascade's level batch, whose decode and chunk
  // phases ran before this launch) done by sc_wgs workgroups after the decode launch's
  // own (sc_wgs == 0: none): that plan's header, lists, partials, outputs and shape,
  // i.e. the fields a combine launch of that plan reads (side_combine_args).
  int32_t* sc_hdr;
  const int4* sc_comb_seqs;
  float2* sc_part_ml;
  uint16_t* sc_part_o;
  uint8_t* sc_out;
  float* sc_lse;
  int64_t sc_o_row, sc_o_head;
  int64_t sc_dec_cap, sc_slot_cap;
  int32_t sc_batch, sc_max_q, sc_max_k, sc_total_q, sc_grid_comb;
  int32_t sc_wgs;
};

// The arguments of the second plan's combine launch (RunArgs::sc_*): the same pools,
// heads and scale, that plan's workspace and outputs, no cascade merge of its own.
__host__ __device__ inline RunArgs side_combine_args(const RunArgs& a) {
  RunArgs b = a;
  b.hdr = a.sc_hdr;
  b.comb_seqs = a.sc_comb_seqs;
  b.part_ml = a.sc_part_ml;
  b.part_o = a.sc_part_o;
  b.out = a.sc_out;
  b.lse = a.sc_lse;
  b.o_row = a.sc_o_row;
  b.o_head = a.sc_o_head;
  b.dec_cap = a.sc_dec_cap;
  b.slot_cap = a.sc_slot_cap;
  b.batch = a.sc_batch;
  b.max_q = a.sc_max_q;
  b.max_k = a.sc_max_k;
  b.total_q = a.sc_total_q;
  b.grid_comb = a.sc_grid_comb;
  b.mg_start = nullptr;
  b.mg_members = 0;
  b.sc_wgs = 0;
  return b;
}

// Row of q that packed row r reads. A map entry outside the query tensor reads row 0 and
// is reported in the error word.
__device__ __forceinline__ int64_t query_row(const RunArgs& a, int64_t r) {
  if (a.q_rows == nullptr) return r;
  const int64_t m = a.q_rows[r];
  if ((uint64_t)m < (uint64_t)a.q_rows_total) return m;
  atomicOr(&a.hdr[H_ERR], HX_WERR_BAD_QUERY_ROW);
  return 0;
}

// True when the workspace holds a plan for this run's shape; otherwise the block
// raises HX_WERR_PLAN_MISMATCH (once) and the caller must return without touching
// the work lists.
// The header is read with three wide loads issued together and compared with
// non-short-circuit ands, so the check costs one memory round trip.
struct Header {
  int4 counts;  // H_NDEC, H_NPF, H_NCOMB, H_ERR
  bool ok;
};
__device__ __forceinline__ Header read_header(const RunArgs& a, int wg) {
  const int4 h0 = *reinterpret_cast<const int4*>(a.hdr);
  const int4 h1 = *reinterpret_cast<const int4*>(a.hdr + 4);
  const int2 h2 = *reinterpret_cast<const int2*>(a.hdr + 8);
  Header r;
  r.counts = h0;
  r.ok = (h2.y == kPlanStamp) & (h1.x == a.batch) & (h1.y == a.max_q) & (h1.z == a.max_k) &
         (h1.w == a.hq) & (h2.x == a.hkv);
  if (!r.ok && wg == 0 && hx::tid_x() == 0) atomicOr(&a.hdr[H_ERR], HX_WERR_PLAN_MISMATCH);
  return r;
}
__device__ __forceinline__ Header read_header(const RunArgs& a) { return read_header(a, hx::wg_x()); }

template <typename T>
__device__ __forceinline__ uint4 ld16(const T* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// ------------------------------------------------------------------ decode (split-K)
// Reduce-scatter across the 16 lanes of a row group: lane c holds partial dot products
// part[i][h] of rows i = 0..15 over its own 8 dims; afterwards out[h] is the full dot
// product of row c. Four DPP butterfly steps (mirror, half-mirror, xor 2, xor 1), each
// pairing lanes that differ in one more bit of c and agree on the bits already used; the
// half a lane keeps is chosen by a bit select on that bit of c.
template <int G>
__device__ __forceinline__ void row_reduce_scatter(float (&part)[16][G], float (&out)[G], int c) {
  constexpr uint64_t b3 = hx::row_bit_lanes(3), b2 = hx::row_bit_lanes(2), b1 = hx::row_bit_lanes(1),
                     b0 = hx::row_bit_lanes(0);
  float s8[8][G], s4[4][G], s2[2][G];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float lo = part[j][h] + hx::dpp<hx::kDppMirror>(part[j][h]);
      const float hi = part[j + 8][h] + hx::dpp<hx::kDppMirror>(part[j + 8][h]);
      s8[j][h] = hx::lane_sel(b3, hi, lo);
    }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float lo = s8[j][h] + hx::dpp<hx::kDppHalfMirror>(s8[j][h]);
      const float hi = s8[j + 4][h] + hx::dpp<hx::kDppHalfMirror>(s8[j + 4][h]);
      s4[j][h] = hx::lane_sel(b2, hi, lo);
    }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float lo = s4[j][h] + hx::dpp<hx::kDppXor2>(s4[j][h]);
      const float hi = s4[j + 2][h] + hx::dpp<hx::kDppXor2>(s4[j + 2][h]);
      s2[j][h] = hx::lane_sel(b1, hi, lo);
    }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float lo = s2[0][h] + hx::dpp<hx::kDppXor1>(s2[0][h]);
    const float hi = s2[1][h] + hx::dpp<hx::kDppXor1>(s2[1][h]);
    out[h] = hx::lane_sel(b0, hi, lo);
  }
}

// Max / sum over all 64 lanes: DPP inside each 16-lane row, then across rows.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, hx::dpp<hx::kDppXor1>(v));
  v = fmaxf(v, hx::dpp<hx::kDppXor2>(v));
  v = fmaxf(v, hx::dpp<hx::kDppHalfMirror>(v));
  v = fmaxf(v, hx::dpp<hx::kDppMirror>(v));
  return hx::max_xor32(hx::max_xor16(v));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += hx::dpp<hx::kDppXor1>(v);
  v += hx::dpp<hx::kDppXor2>(v);
  v += hx::dpp<hx::kDppHalfMirror>(v);
  v += hx::dpp<hx::kDppMirror>(v);
  return hx::add_xor32(hx::add_xor16(v));
}

// The append workgroups of a decode launch: every row t of the tick goes to pool row
// write_slots[t] (index_copy_ semantics; slots outside the pool are skipped), 16 bytes
// per thread step. The chunk kernel, launched after this launch, reads the chunk rows;
// a decode row's split workgroup also writes its own row (the same bits) and takes the
// new token from k_new / v_new, never from the pool.
template <typename T>
__device__ void append_rows(const RunArgs& a, int wg, int n_wg) {
  constexpr int kWords = kD / 8;  // 16-byte words per head row
  const int64_t per_token = (int64_t)a.hkv * kWords;
  const int64_t total = (int64_t)a.total_q * per_token;
  for (int64_t idx = (int64_t)wg * kThreads + hx::tid_x(); idx < total; idx += (int64_t)n_wg * kThreads) {
    const int64_t t = idx / per_token;
    const int rem = (int)(idx - t * per_token);
    const int h = rem / kWords, w = rem - h * kWords;
    const int64_t slot = a.write_slots[t];
    if (slot < 0 || slot >= a.pool_rows) continue;
    const uint4 kw = ld16(reinterpret_cast<const T*>(a.k_new) + t * a.kn_row + (int64_t)h * a.kn_head + 8 * w);
    const uint4 vw = ld16(reinterpret_cast<const T*>(a.v_new) + t * a.vn_row + (int64_t)h * a.vn_head + 8 * w);
    const int64_t off = (slot * a.kv_row + (int64_t)h * a.kv_head + 8 * w) * (int64_t)sizeof(T);
    *reinterpret_cast<uint4*>(const_cast<uint8_t*>(a.k) + off) = kw;
    *reinterpret_cast<uint4*>(const_cast<uint8_t*>(a.v) + off) = vw;
  }
}

// Broadcast lane `SRC` of each 16-lane row to the whole row (DPP row_newbcast).
template <int SRC>
__device__ __forceinline__ uint32_t row_bcast(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x150 + SRC, 0xF, 0xF, false);
}

// Sum over the four 16-lane rows of a wave, scattered: x[v] (NV values per lane) becomes
// NV / 4 values per lane, lane row q holding the sums of x[q * NV / 4 + k]. Two
// permlane-swap steps; each swap exchanges half a register pair, so one swap and one add
// produce one reduced value.
template <int NV>
__device__ __forceinline__ void rows_reduce_scatter(const float (&x)[NV], float (&z)[NV / 4]) {
  float y[NV / 2];
#pragma unroll
  for (int k = 0; k < NV / 2; ++k) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[k]), __float_as_uint(x[k + NV / 2]), false, false);
    y[k] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
#pragma unroll
  for (int k = 0; k < NV / 4; ++k) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(y[k]), __float_as_uint(y[k + NV / 4]), false, false);
    z[k] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
}

template <typename T, int G, int THREADS>
__device__ __forceinline__ void combine_records(const RunArgs& a, int wg, float (&sh)[10][THREADS]);

// EXTRA: workgroups of the launch after the decode workgroups. kExtraAppend: a.app_wgs
// append workgroups. kExtraCombine: those, then a.sc_wgs workgroups running the combine
// records of a second plan (a cascade's level batch). Each kind is its own
// instantiation, so launches without them carry no trace of them (with the combine code
// inlined, hipcc allocates the decode path for four waves per SIMD instead of three).
// Occupancy: three workgroups per CU (at most 168 VGPRs) up to G = 4.
constexpr int kExtraNone = 0, kExtraAppend = 1, kExtraCombine = 2;
template <typename T, int G>
constexpr int decode_min_wgs() {
  return G <= 4 ? 3 : 2;
}
template <typename T, int G, int EXTRA>
__global__ __launch_bounds__(kThreads, (decode_min_wgs<T, G>())) void decode_kernel(RunArgs a) {
  typedef hx::Elem<T> E;
  constexpr int NV = G * 8;  // o values per lane: G heads x 8 dims
  // Per wave: max and sum of its 64 keys (log2 units), and its o summed over its rows.
  __shared__ float w_max[4][G];
  __shared__ float w_sum[4][G];
  __shared__ __attribute__((aligned(16))) float w_o[4][G * kD];

  const int tid = hx::tid_x(), lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, held in a scalar register
  // XCD-aware order: workgroups go to the kXcds XCDs round-robin, so the hkv consecutive
  // workgroups an XCD receives are the KV heads of one split; each XCD then streams whole
  // token rows of the pages it reads (about 4 % faster than one head per XCD). The grid
  // covers the work items rounded up to a multiple of kXcds.
  if constexpr (EXTRA != kExtraNone) {
    const int dec_wgs = (a.grid_dec + kXcds - 1) / kXcds * kXcds * a.hkv;
    if (hx::wg_x() >= dec_wgs) {  // append, then combine workgroups follow the decode ones
      const int j = hx::wg_x() - dec_wgs;
      if (j < a.app_wgs) {
        append_rows<T>(a, j, a.app_wgs);
      } else if constexpr (EXTRA == kExtraCombine) {
        __shared__ float comb_sh[10][kThreads];
        combine_records<T, G, kThreads>(side_combine_args(a), j - a.app_wgs, comb_sh);
      }
      return;
    }
  }
  const int xcd = hx::wg_x() % kXcds, jx = hx::wg_x() / kXcds;
  const int g = jx % a.hkv;
  const int item = (jx / a.hkv) * kXcds + xcd;
  if (item >= a.grid_dec) return;
  // The work item is read together with the header (item < grid_dec <= the list's
  // capacity, so the read stays inside the workspace) and used only once both check out.
  const Header hd = read_header(a);
  const int4 it = a.dec_items[item];  // {b, split, q0, L}
  if (!hd.ok) return;
  const int n_dec = hd.counts.x;
  if (hx::wg_x() == 0 && tid == 0 && n_dec > a.grid_dec) atomicOr(&a.hdr[H_ERR], HX_WERR_GRID);
  if (item >= n_dec) return;
  // Workgroup-uniform: kept in scalar registers.
  const int b = __builtin_amdgcn_readfirstlane(it.x), s = __builtin_amdgcn_readfirstlane(it.y);
  const int q0 = __builtin_amdgcn_readfirstlane(it.z), L = __builtin_amdgcn_readfirstlane(it.w);
  if ((unsigned)b >= (unsigned)a.batch) return;
  int s_first, splits;
  decode_splits(L, a.win_left, &s_first, &splits);
  const int key0 = s * kSplit;
  const int kb = max(decode_lo(L, a.win_left), key0);
  const int ke = min(L, key0 + kSplit);

  int64_t row0;
  bool page_ok = true;
  if (a.page_size > 0) {
    const int page = a.bt[(int64_t)b * a.bt_stride + key0 / a.page_size];
    page_ok = page >= 0 && page < a.num_pages;
    if (!page_ok && tid == 0 && kb < ke) atomicOr(&a.hdr[H_ERR], HX_WERR_BAD_PAGE);
    row0 = (int64_t)(page_ok ? page : 0) * a.page_size + key0 % a.page_size;
  } else {
    row0 = (int64_t)a.seq_info[b].w + key0;
  }
  const int kvr = (int)a.kv_row;
  const T* kbase = reinterpret_cast<const T*>(a.k) + row0 * a.kv_row + (int64_t)g * a.kv_head;
  const T* vbase = reinterpret_cast<const T*>(a.v) + row0 * a.kv_row + (int64_t)g * a.kv_head;

  // Lane (r, c) = (lane / 16, lane % 16) owns the 16-byte chunk c (dims 8c..8c+7) of
  // tokens 16i + 4w + r, i = 0..15: every wave instruction reads four whole 256-byte head
  // rows, and the four waves' i-th loads together read 16 consecutive tokens. Reading
  // the split front to back this way streams about 5 % faster than giving each wave a
  // contiguous quarter of the split.
  const int r = lane >> 4, c = lane & 15;
  uint4 qf[G];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + query_row(a, q0) * a.q_row + (int64_t)(g * G) * a.q_head + 8 * c;
#pragma unroll
    for (int h = 0; h < G; ++h) qf[h] = ld16(qp + (int64_t)h * a.q_head);
  }
  const bool any = page_ok && kb < ke;
  const int nend = ke - key0;

  // Fused append (decode rows only): the split holding key L-1, this row's new token,
  // writes that token's K/V from k_new / v_new to pool row write_slots[q0] (the 16 lanes
  // that load the token's row each store their 16-byte chunk of head g), waits for the
  // stores, and then reads the row from the pool like every other key, as the reference
  // reads its pool after _write. No other workgroup reads that slice of the row during
  // this launch.
  if (a.k_new != nullptr && L >= 1 && L - 1 >= key0 && L - 1 < key0 + kSplit) {
    const int nn = L - 1 - key0;
    if (((nn >> 2) & 3) == w) {  // wave-uniform: this wave loads the token's row
      if ((nn & 3) == r) {
        const int64_t slot = a.write_slots[q0];
        if (slot >= 0 && slot < a.pool_rows) {
          const T* kp = reinterpret_cast<const T*>(a.k_new) + (int64_t)q0 * a.kn_row + (int64_t)g * a.kn_head + 8 * c;
          const T* vp = reinterpret_cast<const T*>(a.v_new) + (int64_t)q0 * a.vn_row + (int64_t)g * a.vn_head + 8 * c;
          const int64_t off = slot * a.kv_row + (int64_t)g * a.kv_head + 8 * c;
          *reinterpret_cast<uint4*>(const_cast<uint8_t*>(a.k) + off * (int64_t)sizeof(T)) = ld16(kp);
          *reinterpret_cast<uint4*>(const_cast<uint8_t*>(a.v) + off * (int64_t)sizeof(T)) = ld16(vp);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }

  // Per wave: max and sum of p over its keys (log2 units), and o = P V. An empty split
  // (no visible key, or a bad page id) loads nothing and keeps (-inf, 0, 0).
  float mx[G], ps[G], o[G][8];
  if (any) {
    // Buffer loads at a 32-bit lane offset plus a scalar step of 16 rows per load: no
    // per-load vector address work. The resource ends after the split's last visible row,
    // so rows past it read zeros (the range check covers the scalar offset too); rows
    // before the first visible one (a window's start) are earlier keys of the sequence.
    // Either way the data is finite, and its score is masked below. Offsets stay below
    // 2^32: the host caps the row stride at 2^23 elements (the range is clamped to fit).
    uint4 kr[16], vr[16];
    const uint32_t row_bytes = (uint32_t)kvr * (uint32_t)sizeof(T);
    const uint32_t loff = (uint32_t)(4 * w + r) * row_bytes + 16u * (uint32_t)c;
    const uint32_t step = 16u * row_bytes;
    const uint64_t span = (uint64_t)nend * row_bytes;
    const uint32_t range = span > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)span;
    const __amdgpu_buffer_rsrc_t kres = hx::buffer_rsrc(kbase, range);
    const __amdgpu_buffer_rsrc_t vres = hx::buffer_rsrc(vbase, range);
#pragma unroll
    for (int i = 0; i < 16; ++i) kr[i] = hx::ld16_stream(kres, loff, (uint32_t)i * step);
#pragma unroll
    for (int i = 0; i < 16; ++i) vr[i] = hx::ld16_stream(vres, loff, (uint32_t)i * step);

    // q . k on VALU (packed dot2, fp32 accumulate), then the 16 lanes of each row group
    // exchange partial sums so that lane (r, c) ends with token 16c + 4w + r.
    float part[16][G];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int h = 0; h < G; ++h) part[i][h] = hx::dot8_zero<T>(qf[h], kr[i]);
    float sc[G];
    row_reduce_scatter<G>(part, sc, c);

    // Softmax inside the wave: its own max (no barrier), p = 2^(s - max) rounded to the
    // element type, and the sum of the rounded p, so that o / l is exactly the average of
    // V under the weights that multiply it. The waves' (max, sum, o) merge at the end.
    const int t = 16 * c + 4 * w + r;
    const bool tok_ok = key0 + t >= kb && key0 + t < ke;
    uint32_t pp[G];  // {p of token 16c' + 4w + r, p of token 16(c'+1) + 4w + r}, c' = c & ~1
    constexpr uint64_t odd = hx::row_bit_lanes(0);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = tok_ok ? sc[h] * a.scale_log2 : -INFINITY;
      mx[h] = wave_max(x);
      const float p = x == -INFINITY ? 0.f : hx::fast_exp2(x - mx[h]);
      const float q = hx::dpp<hx::kDppXor1>(p);
      pp[h] = hx::pack2_round<T>(hx::lane_sel(odd, q, p), hx::lane_sel(odd, p, q));
      ps[h] = wave_sum(E::lo(hx::lane_sel(odd, pp[h] >> 16, pp[h])));
    }

#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
    // O = P V with dot2 over token pairs: pair j is tokens 32j + 4w + r and
    // 32j + 16 + 4w + r (loads 2j and 2j + 1 of this lane); its p pair sits in lane 2j
    // of the row.
#define HX_PV_PAIR(J)                                                                          \
  {                                                                                            \
    uint32_t pb[G];                                                                            \
    _Pragma("unroll") for (int h = 0; h < G; ++h) pb[h] = row_bcast<2 * (J)>(pp[h]);           \
    const uint4 v0 = vr[2 * (J)], v1 = vr[2 * (J) + 1];                                        \
    const uint32_t vp[8] = {hx::interleave_lo(v0.x, v1.x), hx::interleave_hi(v0.x, v1.x),      \
                            hx::interleave_lo(v0.y, v1.y), hx::interleave_hi(v0.y, v1.y),      \
                            hx::interleave_lo(v0.z, v1.z), hx::interleave_hi(v0.z, v1.z),      \
                            hx::interleave_lo(v0.w, v1.w), hx::interleave_hi(v0.w, v1.w)};     \
    _Pragma("unroll") for (int h = 0; h < G; ++h)                                              \
      _Pragma("unroll") for (int e = 0; e < 8; ++e) o[h][e] = E::dot2(pb[h], vp[e], o[h][e]); \
  }
    HX_PV_PAIR(0) HX_PV_PAIR(1) HX_PV_PAIR(2) HX_PV_PAIR(3)
    HX_PV_PAIR(4) HX_PV_PAIR(5) HX_PV_PAIR(6) HX_PV_PAIR(7)
#undef HX_PV_PAIR
  } else {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      mx[h] = -INFINITY;
      ps[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
    }
  }

  // The wave's o summed over its four rows: lane row r keeps values v = r*2G .. r*2G+2G-1
  // of v = 8h + e, i.e. head v / 8, dims 8c + v % 8.
  {
    float x[NV];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[h * 8 + e] = o[h][e];
    float z[NV / 4];
    rows_reduce_scatter<NV>(x, z);
    constexpr int NQ = NV / 4;
    if constexpr (NQ % 4 == 0) {
#pragma unroll
      for (int k = 0; k < NQ; k += 4) {
        const int v = r * NQ + k;
        *reinterpret_cast<float4*>(&w_o[w][(v >> 3) * kD + 8 * c + (v & 7)]) = make_float4(z[k], z[k + 1], z[k + 2], z[k + 3]);
      }
    } else {
      const int v = r * NQ;
      *reinterpret_cast<float2*>(&w_o[w][(v >> 3) * kD + 8 * c + (v & 7)]) = make_float2(z[0], z[1]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      w_max[w][h] = mx[h];
      w_sum[w][h] = ps[h];
    }
  }
  __syncthreads();

  // G x 16 lanes finish: lane f = 16h + cc merges head h, dims 8cc..8cc+7 over the four
  // waves and stores them as one 16-byte row piece.
  if (tid < G * 16) {
    const int h = tid >> 4, cc = tid & 15;
    float m = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) m = fmaxf(m, w_max[ww][h]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float mw = w_max[ww][h];
      const float alpha = mw == -INFINITY ? 0.f : hx::fast_exp2(mw - m);
      l = fmaf(alpha, w_sum[ww][h], l);
      const float4 a0 = *reinterpret_cast<const float4*>(&w_o[ww][h * kD + 8 * cc]);
      const float4 a1 = *reinterpret_cast<const float4*>(&w_o[ww][h * kD + 8 * cc + 4]);
      acc[0] = fmaf(alpha, a0.x, acc[0]);
      acc[1] = fmaf(alpha, a0.y, acc[1]);
      acc[2] = fmaf(alpha, a0.z, acc[2]);
      acc[3] = fmaf(alpha, a0.w, acc[3]);
      acc[4] = fmaf(alpha, a1.x, acc[4]);
      acc[5] = fmaf(alpha, a1.y, acc[5]);
      acc[6] = fmaf(alpha, a1.z, acc[6]);
      acc[7] = fmaf(alpha, a1.w, acc[7]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const uint4 val = make_uint4(hx::pack2_round<T>(acc[0] * inv, acc[1] * inv), hx::pack2_round<T>(acc[2] * inv, acc[3] * inv),
                                 hx::pack2_round<T>(acc[4] * inv, acc[5] * inv), hx::pack2_round<T>(acc[6] * inv, acc[7] * inv));
    const int qh = g * G + h;
    if (splits == 1) {
      T* orow = reinterpret_cast<T*>(a.out) + (int64_t)q0 * a.o_row + (int64_t)qh * a.o_head + 8 * cc;
      if (a.o_row % 8 == 0 && a.o_head % 8 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0) {
        *reinterpret_cast<uint4*>(orow) = val;
      } else {  // rows 8-byte aligned (checked on the host)
        uint2* o2 = reinterpret_cast<uint2*>(orow);
        o2[0] = make_uint2(val.x, val.y);
        o2[1] = make_uint2(val.z, val.w);
      }
      if (a.lse && cc == 0)
        a.lse[(int64_t)qh * a.total_q + q0] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
    } else {
      *reinterpret_cast<uint4*>(a.part_o + ((int64_t)item * a.hq + qh) * kD + 8 * cc) = val;
      if (cc == 0) a.part_ml[(int64_t)item * a.hq + qh] = make_float2(m, l);
    }
  }
}

// ------------------------------------------------------------------ split combine
// A combine record {b, first slot, splits | (rows - 1) << 24, first output row} covers
// `rows` consecutive output rows (1 for a decode row, up to kCombRows rows of a split
// chunk block) whose partials sit at slots first + r * splits + s. A task is one (row,
// head, 8-dim chunk): 16-byte partial loads, merged with an online max in groups of
// kCombChunk splits whose (m, l) pairs and partial rows are loaded together. When the
// record has fewer tasks than threads, the workgroup splits the partials into
// THREADS / tasks contiguous ranges (a decode row at G = 4 and 256 threads: four, one
// per wave), and the ranges are merged in LDS in range order, so the result does not
// depend on scheduling. Workgroups have 256 threads, or 512 when a row may have more
// than kCombSmallSplits splits (more ranges keep each thread's loads to one or two
// groups): smaller workgroups finish the short records of decode ticks and split chunk
// blocks sooner (C3's combine 14.7 -> 12.4 us), while long rows want the ranges.
constexpr int kCombChunk = 8;
constexpr int kCombSmallSplits = 32;

struct CombAcc {
  float m, l;
  float acc[8];
};

// Merges the partials of splits [s0, s_end), s_end - s0 <= NC, into r: the NC (m, l)
// pairs and partial rows are loaded together (indices past s_end re-read s_end - 1 and
// get weight 0).
template <typename T, int NC>
__device__ __forceinline__ void combine_step(const float2* ml, const uint16_t* po, int64_t step_ml,
                                             int64_t step_o, int s0, int s_end, CombAcc& r) {
  float2 mlv[NC];
  uint4 ov[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int sj = s0 + j < s_end ? s0 + j : s_end - 1;
    mlv[j] = ml[(int64_t)sj * step_ml];
    ov[j] = *reinterpret_cast<const uint4*>(po + (int64_t)sj * step_o);
  }
  float cm = r.m;
#pragma unroll
  for (int j = 0; j < NC; ++j)
    if (s0 + j < s_end) cm = fmaxf(cm, mlv[j].x);
  if (cm == -INFINITY) return;
  const float rescale = r.m == -INFINITY ? 0.f : hx::fast_exp2(r.m - cm);
  r.l *= rescale;
#pragma unroll
  for (int e = 0; e < 8; ++e) r.acc[e] *= rescale;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const bool live = s0 + j < s_end && mlv[j].x != -INFINITY;
    const float wgt = live ? hx::fast_exp2(mlv[j].x - cm) * mlv[j].y : 0.f;  // partial stores o / l
    r.l += wgt;
    const uint32_t w4[4] = {ov[j].x, ov[j].y, ov[j].z, ov[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r.acc[2 * e] += wgt * hx::Elem<T>::lo(w4[e]);
      r.acc[2 * e + 1] += wgt * hx::Elem<T>::hi(w4[e]);
    }
  }
  r.m = cm;
}

// Online merge of the partials of splits [s_lo, s_hi) for one task, in split order:
// (m, l, acc) with acc = sum over splits of 2^(m_s - m) * l_s * (o_s / l_s), so the
// output is acc / l. Groups of kCombChunk while more than four splits remain (the last
// of them may re-read clamped entries), then one group of four or two: records of up to
// four splits load no more than the next power of two.
template <typename T>
__device__ __forceinline__ CombAcc combine_range(const RunArgs& a, int64_t base, int qh, int ch,
                                                 int s_lo, int s_hi) {
  const float2* ml = a.part_ml + base * a.hq + qh;
  const uint16_t* po = a.part_o + (base * a.hq + qh) * kD + 8 * ch;
  const int64_t step_o = (int64_t)a.hq * kD;
  CombAcc r;
  r.m = -INFINITY;
  r.l = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) r.acc[e] = 0.f;
  int s0 = s_lo;
  for (; s_hi - s0 > 4; s0 += kCombChunk) combine_step<T, kCombChunk>(ml, po, a.hq, step_o, s0, min(s_hi, s0 + kCombChunk), r);
  if (s_hi - s0 > 2)
    combine_step<T, 4>(ml, po, a.hq, step_o, s0, s_hi, r);
  else if (s_hi > s0)
    combine_step<T, 2>(ml, po, a.hq, step_o, s0, s_hi, r);
  return r;
}

template <typename T>
__device__ __forceinline__ void combine_store(const RunArgs& a, const CombAcc& r, int row, int qh, int ch) {
  const float inv = r.l > 0.f ? 1.f / r.l : 0.f;
  const uint4 u = make_uint4(hx::pack2_round<T>(r.acc[0] * inv, r.acc[1] * inv), hx::pack2_round<T>(r.acc[2] * inv, r.acc[3] * inv),
                             hx::pack2_round<T>(r.acc[4] * inv, r.acc[5] * inv), hx::pack2_round<T>(r.acc[6] * inv, r.acc[7] * inv));
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)row * a.o_row + (int64_t)qh * a.o_head + 8 * ch;
  if (a.o_row % 8 == 0 && a.o_head % 8 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0) {
    hx::st16_nt(orow, u);  // written once, read by a later launch
  } else {
    uint2* o2 = reinterpret_cast<uint2*>(orow);  // rows are 8-byte aligned (checked on the host)
    o2[0] = make_uint2(u.x, u.y);
    o2[1] = make_uint2(u.z, u.w);
  }
  if (a.lse && ch == 0)
    a.lse[(int64_t)qh * a.total_q + row] = r.l > 0.f ? (r.m + log2f(r.l)) * kLn2 : -INFINITY;
}

// Part range of cascade member k, clipped to the part list.
__device__ __forceinline__ void member_parts(const RunArgs& a, int k, int64_t* p0, int64_t* p1) {
  *p0 = max((int64_t)a.mg_start[k], (int64_t)0);
  *p1 = min((int64_t)a.mg_start[k + 1], (int64_t)a.mg_n_idx);
}

// combine_store for the decode row of cascade member k: its result over the batch's
// keys, rounded to T and given its log-sum-exp exactly as combine_store writes them,
// then its levels folded in (hx::fold_parts), i.e. the bits combine_store followed by
// hx_attn_merge's pass give. Output rows are 16-byte aligned (checked on the host).
template <typename T>
__device__ __forceinline__ void combine_store_member(const RunArgs& a, const CombAcc& r, int row, int qh, int ch,
                                                     int k) {
  const float inv = r.l > 0.f ? 1.f / r.l : 0.f;
  uint32_t w4[4] = {hx::pack2_round<T>(r.acc[0] * inv, r.acc[1] * inv), hx::pack2_round<T>(r.acc[2] * inv, r.acc[3] * inv),
                    hx::pack2_round<T>(r.acc[4] * inv, r.acc[5] * inv), hx::pack2_round<T>(r.acc[6] * inv, r.acc[7] * inv)};
  float m = r.l > 0.f ? (r.m + log2f(r.l)) * kLn2 : -INFINITY;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc[2 * e] = hx::Elem<T>::lo(w4[e]);
    acc[2 * e + 1] = hx::Elem<T>::hi(w4[e]);
  }
  int64_t p0, p1;
  member_parts(a, k, &p0, &p1);
  if (hx::fold_parts<T>(acc, m, a.mg_o, a.mg_o_row, a.mg_o_head, a.mg_lse, a.mg_lse_stride, a.mg_rows, qh, ch,
                        a.mg_idx, p0, p1)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) w4[e] = hx::pack2_round<T>(acc[2 * e], acc[2 * e + 1]);
  }
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)row * a.o_row + (int64_t)qh * a.o_head + 8 * ch;
  hx::st16_nt(orow, make_uint4(w4[0], w4[1], w4[2], w4[3]));
  if (a.lse && ch == 0) a.lse[(int64_t)qh * a.total_q + row] = m;
}

// Workgroups after the combine records' in the combine launch: cascade members whose
// decode row has one split (the decode kernel wrote its result and log-sum-exp) fold
// their levels in place; 16 lanes per (member, head). A member whose row has more splits
// is merged by its combine record instead.
template <typename T, int THREADS>
__device__ __forceinline__ void merge_unsplit_members(const RunArgs& a, int j) {
  const Header hd = read_header(a);
  if (!hd.ok) return;
  const int64_t item = (int64_t)j * (THREADS / 16) + (hx::tid_x() >> 4);
  const int li = hx::tid_x() & 15;
  if (item >= (int64_t)a.mg_members * a.hq) return;
  const int k = (int)(item / a.hq);
  const int h = (int)(item - (int64_t)k * a.hq);
  const int b = a.mg_seq[k];
  if ((unsigned)b >= (unsigned)a.batch) return;
  const int4 si = a.seq_info[b];
  if (si.y != 1) return;
  int s_first, splits;
  decode_splits(si.z, a.win_left, &s_first, &splits);
  if (splits > 1) return;
  const int row = si.x;
  if (row < 0 || row >= a.total_q) return;
  uint16_t* po = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.o_row + (int64_t)h * a.o_head + 8 * li;
  float* lb = a.lse + (int64_t)h * a.total_q + row;
  float m = *lb;  // the row's result is normalised, with log-sum-exp m
  const uint4 ov = *reinterpret_cast<const uint4*>(po);
  float acc[8];
  {
    const uint32_t w4[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[2 * e] = hx::Elem<T>::lo(w4[e]);
      acc[2 * e + 1] = hx::Elem<T>::hi(w4[e]);
    }
  }
  int64_t p0, p1;
  member_parts(a, k, &p0, &p1);
  if (!hx::fold_parts<T>(acc, m, a.mg_o, a.mg_o_row, a.mg_o_head, a.mg_lse, a.mg_lse_stride, a.mg_rows, h, li,
                         a.mg_idx, p0, p1))
    return;
  uint4 u;
  u.x = hx::pack2_round<T>(acc[0], acc[1]);
  u.y = hx::pack2_round<T>(acc[2], acc[3]);
  u.z = hx::pack2_round<T>(acc[4], acc[5]);
  u.w = hx::pack2_round<T>(acc[6], acc[7]);
  // The 16 lanes of an entry sit in one wave: each read the old lse above, in program
  // order before lane 0 stores the merged one.
  *reinterpret_cast<uint4*>(po) = u;
  if (li == 0) *lb = m;
}

// Combine record cs = wg / hkv of KV head wg % hkv: workgroup wg of a combine launch, or
// of the extra combine workgroups of a decode launch (then with the other plan's
// arguments, side_combine_args). sh: (m, l, acc[8]) of every range, one column per thread.
template <typename T, int G, int THREADS>
__device__ __forceinline__ void combine_records(const RunArgs& a, int wg, float (&sh)[10][THREADS]) {
  constexpr int kPerRow = G * (kD / 8);  // tasks per output row
  const int cs = wg / a.hkv;
  const int g = wg - cs * a.hkv;
  const Header hd = read_header(a);
  const int4 c = a.comb_seqs[cs];  // cs < grid_comb <= max_comb
  if (!hd.ok) {
    // read_header reports for the launch's first workgroup; extra workgroups report here.
    if (wg == 0 && hx::wg_x() != 0 && hx::tid_x() == 0) atomicOr(&a.hdr[H_ERR], HX_WERR_PLAN_MISMATCH);
    return;
  }
  const int n_comb = hd.counts.z;
  if (wg == 0 && hx::tid_x() == 0 && n_comb > a.grid_comb) atomicOr(&a.hdr[H_ERR], HX_WERR_GRID);
  if (cs >= n_comb) return;
  const int first = c.y, splits = c.z & 0xffffff, rows = (c.z >> 24) + 1, q0 = c.w;
  if ((unsigned)c.x >= (unsigned)a.batch || first < 0 || splits < 1 || rows > kCombRows) return;
  if ((int64_t)first + (int64_t)rows * splits > a.slot_cap) return;
  if (q0 < 0 || q0 + rows > a.total_q) return;
  const int tasks = rows * kPerRow;
  const int ranges = min(THREADS / tasks, splits);  // workgroup-uniform
  // A decode row (its partials in the decode slots) that is a cascade member stores its
  // merged result.
  int member = -1;
  if (a.mg_start != nullptr && first < a.dec_cap) {
    const int k = a.mg_of_seq[c.x];
    member = k < a.mg_members ? k : -1;
  }
  auto store = [&](const CombAcc& res, int row, int qh, int ch) {
    if (member >= 0)
      combine_store_member<T>(a, res, row, qh, ch, member);
    else
      combine_store<T>(a, res, row, qh, ch);
  };
  if (ranges <= 1) {
    for (int t = hx::tid_x(); t < tasks; t += THREADS) {
      const int r = t / kPerRow;
      const int h = (t - r * kPerRow) >> 4, ch = t & 15;
      const CombAcc res = combine_range<T>(a, (int64_t)first + (int64_t)r * splits, g * G + h, ch, 0, splits);
      store(res, q0 + r, g * G + h, ch);
    }
    return;
  }
  // ranges >= 2: thread t < ranges * tasks takes task t % tasks over range t / tasks.
  const int t = hx::tid_x();
  const int task = t % tasks, rg = t / tasks;
  const int r = task / kPerRow;
  const int h = (task - r * kPerRow) >> 4, ch = task & 15;
  const int span = (splits + ranges - 1) / ranges;
  if (rg < ranges) {
    const int s_lo = min(splits, rg * span), s_hi = min(splits, s_lo + span);
    const CombAcc res = combine_range<T>(a, (int64_t)first + (int64_t)r * splits, g * G + h, ch, s_lo, s_hi);
    sh[0][t] = res.m;
    sh[1][t] = res.l;
#pragma unroll
    for (int e = 0; e < 8; ++e) sh[2 + e][t] = res.acc[e];
  }
  __syncthreads();
  if (rg == 0) {
    float m = -INFINITY;
    for (int q = 0; q < ranges; ++q) m = fmaxf(m, sh[0][q * tasks + task]);
    CombAcc res;
    res.m = m;
    res.l = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) res.acc[e] = 0.f;
    if (m != -INFINITY) {
      for (int q = 0; q < ranges; ++q) {
        const int col = q * tasks + task;
        const float mq = sh[0][col];
        const float wq = mq == -INFINITY ? 0.f : hx::fast_exp2(mq - m);
        res.l += wq * sh[1][col];
#pragma unroll
        for (int e = 0; e < 8; ++e) res.acc[e] += wq * sh[2 + e][col];
      }
    }
    store(res, q0 + r, g * G + h, ch);
  }
}

template <typename T, int G, int THREADS>
__global__ __launch_bounds__(THREADS, 4) void combine_kernel(RunArgs a) {
  __shared__ float sh[10][THREADS];
  if (hx::wg_x() >= a.grid_comb * a.hkv) {  // the cascade merge's workgroups (mg_start set)
    if (a.mg_start != nullptr) merge_unsplit_members<T, THREADS>(a, hx::wg_x() - a.grid_comb * a.hkv);
    return;
  }
  combine_records<T, G, THREADS>(a, hx::wg_x(), sh);
}

// ------------------------------------------------------------------ chunk (prefill) MFMA
constexpr int kChunkThreads = 512;     // 8 waves: 2 per SIMD
constexpr float kLazyLog2 = 8.f;       // softmax terms stay <= 2^8 between max updates
constexpr int kTileRowBytes = kD * 2;  // one key row of one KV head in a tile: 256 B
constexpr int kTileBytes = kTile * kTileRowBytes;  // 16 KiB
// Instruction classes of __builtin_amdgcn_sched_group_barrier's mask.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
// Tile layout in LDS. Two K and two V tiles of 64 key rows x 256 B, each its own LDS
// variable (64 KiB in all). The tiles arrive by direct-to-LDS buffer loads: one wave
// instruction writes 1 KiB, four whole key rows, so rows cannot be padded; the 16-byte
// chunks of a row are permuted instead. Chunk c of key row r sits at position
// c ^ (r & 15) in a K tile, so the 16 rows one QK^T fragment read touches (one chunk
// each) hit 16 distinct positions, and at c ^ (2 (r & 7)) in a V tile, so the 8 rows x
// 32 B each half-wave of a transposing P V operand read touches hit 8 distinct 32-byte
// slots. Both reads are free of bank conflicts. After the tile loop the same 64 KiB
// stage the output: 8 KiB per wave, its 32 rows of one head at 256 B, chunks placed as in
// a K tile.
__device__ __forceinline__ int k_chunk_pos(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_chunk_pos(int r, int c) { return c ^ (2 * (r & 7)); }

// One workgroup per (sequence, block of 256/Gw query rows, group of Gw <= 4 query
// heads of KV head g). Wave w owns 32 rows (two 16-row MFMA blocks) of head w % Gw.
// Each 64-key tile of K and V goes from HBM straight into LDS (no register staging) and
// feeds all 8 waves: K rows as the QK^T operand, V rows read transposed
// (ds_read_b64_tr_b16) as the P V operand. The next tile's copies are issued while the
// current one is consumed; tiles alternate between two LDS buffers, so one wait and one
// barrier per tile suffice: a buffer is written again two tiles later, after every wave
// has passed the barrier that follows its last read. The loop body covers two tiles, so
// every LDS access names its buffer variable statically: the compiler then knows that
// the copies in flight (into the other buffer) do not alias the reads, and adds no wait
// for them. Two waves per SIMD hide each other's LDS and memory latency.
// The body of one workgroup: work item and KV head from workgroup index wg of a's items.
// side: a is the second plan of a paired launch (chunk_pair_kernel). Both copies of the
// body in that launch share one set of LDS tiles.
template <typename T, int G>
__device__ __forceinline__ void chunk_body(const RunArgs& a, const int wg, const bool side) {
  typedef hx::Elem<T> E;
  typedef typename E::v8 v8;
  constexpr int Gw = G < 4 ? G : 4;
  __shared__ __attribute__((aligned(16))) uint8_t k_lds0[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t k_lds1[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds0[kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds1[kTileBytes];

  const int tid = hx::tid_x(), lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, held in a scalar register
  const int item = wg / a.hkv;
  const int g = wg - item * a.hkv;
  const Header hd = read_header(a, wg);
  const int4 it = a.pf_items[item];  // item < grid_pf <= the list's capacity
  // The item's sequence fields (its seq_info entry, copied by the planner), loaded with
  // the item instead of after it: one dependent round trip less before the first tile.
  const int4 si = a.pf_seq[item];
  if (!hd.ok) return;
  const int n_pf = hd.counts.y;
  if (wg == 0 && tid == 0 && n_pf > a.grid_pf) atomicOr(&a.hdr[H_ERR], HX_WERR_GRID);
  // The level batch of a paired launch has no decode launch in this call: decode items in
  // its plan would be left unwritten.
  if (side && wg == 0 && tid == 0 && hd.counts.x > 0) atomicOr(&a.hdr[H_ERR], HX_WERR_GRID);
  if (item >= n_pf) return;
  // Work-item and sequence fields are workgroup-uniform: keep them (and the tile loop
  // they bound) in scalar registers.
  const int b = __builtin_amdgcn_readfirstlane(it.x);
  const int row0 = __builtin_amdgcn_readfirstlane(it.y);
  const int hquad = __builtin_amdgcn_readfirstlane(it.z);
  if ((unsigned)b >= (unsigned)a.batch) return;
  const int q0 = __builtin_amdgcn_readfirstlane(si.x), n = __builtin_amdgcn_readfirstlane(si.y);
  const int L = __builtin_amdgcn_readfirstlane(si.z), kvb = __builtin_amdgcn_readfirstlane(si.w);
  const int off = L - n;  // key position of query row 0
  // Split sp of S covers an equal share of the block's key tiles (S = 1: all of them).
  const int sp = __builtin_amdgcn_readfirstlane(it.w & 0xffff);
  const int S = __builtin_amdgcn_readfirstlane((it.w >> 16) + 1);
  int t_begin, t_end;
  chunk_tiles(n, L, row0, 256 / Gw, a.win_left, a.win_right, &t_begin, &t_end);
  const int khi = t_end > t_begin ? min(L - 1, t_end * kTile - 1) : -1;  // last key the pages cover
  if (S > 1) {
    const int span = (t_end - t_begin + S - 1) / S;
    t_begin = min(t_end, t_begin + sp * span);
    t_end = min(t_end, t_begin + span);
  }

  const int wr0 = row0 + 32 * (w / Gw);
  const int qh = g * G + hquad * Gw + (w % Gw);
  const float sl2 = a.scale_log2;
  // Raw-score margin before the reference max moves (finite, so -inf + margin = -inf).
  const float lazy_thr = fminf(kLazyLog2 / sl2, 1e30f);

  // Q^T as the MFMA B operand: lane holds row wr0+16rb+(lane&15), dims 32st+8(lane>>4)..+7.
  uint4 qf[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int rr = wr0 + 16 * rb + (lane & 15);
    const bool ok = rr < n;
    const T* qp = reinterpret_cast<const T*>(a.q) + query_row(a, q0 + (ok ? rr : 0)) * a.q_row +
                  (int64_t)qh * a.q_head + 8 * (lane >> 4);
#pragma unroll
    for (int st = 0; st < 4; ++st) qf[rb][st] = ok ? ld16(qp + 32 * st) : hx::zero4();
  }

  hx::f32x4_t oacc[8][2];
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) oacc[db][rb] = hx::f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};  // running row max of the raw scores
  float l_run[2] = {0.f, 0.f};              // this lane's share of the row sum

  // Page ids of the key range, 64 at a time: lane j holds the id of page pg_base + j,
  // so a tile finds its page with one v_readlane instead of a dependent global load.
  const bool paged = a.page_size > 0;
  const int last_pg = paged && khi >= 0 ? khi / a.page_size : -1;
  int pg_base = paged ? (t_begin * kTile) / a.page_size : 0;
  int pg_ids = -1;
  auto fetch_pages = [&]() {
    const int p = pg_base + lane;
    pg_ids = p <= last_pg ? a.bt[(int64_t)b * a.bt_stride + p] : -1;
  };
  if (paged) fetch_pages();
  // Tiles are loaded in key order; (ld_pi, ld_off) = page index and in-page key offset of
  // the next tile to load (pages hold a whole number of tiles).
  int ld_pi = pg_base, ld_off = paged ? t_begin * kTile - pg_base * a.page_size : 0;

  // Wave w copies key rows 8w..8w+7 of each tile, four rows per instruction: lane l of
  // copy j moves the 16-byte chunk of row 8w + 4j + l / 16 that belongs at position l % 16
  // (the permutation above). Its byte offsets from the tile's first row of KV head g are
  // the same for every tile.
  const uint32_t row_bytes = (uint32_t)a.kv_row * (uint32_t)sizeof(T);
  uint32_t koffs[2], voffs[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 8 * w + 4 * j + (lane >> 4), p = lane & 15;
    koffs[j] = (uint32_t)r * row_bytes + 16u * (uint32_t)k_chunk_pos(r, p);
    voffs[j] = (uint32_t)r * row_bytes + 16u * (uint32_t)v_chunk_pos(r, p);
  }

  // Each tile's K and V rows are read through buffer resources that end after the tile's
  // last key (row L - 1 in the last tile): rows past it arrive as zeros, whose scores are
  // masked to -inf (the last tile is never "full"), so no branch or clamp guards the
  // copies and a tile's addressing is scalar work. A bad page id reads page 0 and is
  // reported in the error word.
  bool bad_page = false;  // some tile's page id was outside the pool
  auto load_tile = [&](int t, uint8_t* k_dst, uint8_t* v_dst) {
    const int key_base = t * kTile;
    int64_t rowb;
    if (paged) {
      if (ld_pi - pg_base >= 64) {
        pg_base = ld_pi;
        fetch_pages();
      }
      // Wave-uniform: the page id, the row base and the bad-page flag stay in scalar
      // registers (a branch around the error report here moved them to the VALU).
      int page = __builtin_amdgcn_readlane(pg_ids, ld_pi - pg_base);
      const bool bad = (unsigned)page >= (unsigned)a.num_pages;
      bad_page |= bad;
      page = bad ? 0 : page;
      rowb = (int64_t)page * a.page_size + ld_off;
      ld_off += kTile;
      if (ld_off == a.page_size) {
        ld_off = 0;
        ++ld_pi;
      }
    } else {
      rowb = (int64_t)kvb + key_base;
    }
    const int64_t head0 = rowb * a.kv_row + (int64_t)g * a.kv_head;
    const T* kt = reinterpret_cast<const T*>(a.k) + head0;
    const T* vt = reinterpret_cast<const T*>(a.v) + head0;
    const int rows = min(L - key_base, kTile);  // >= 1: key_base <= khi <= L - 1
    const __amdgpu_buffer_rsrc_t kres = hx::buffer_rsrc(kt, (uint32_t)rows * row_bytes);
    const __amdgpu_buffer_rsrc_t vres = hx::buffer_rsrc(vt, (uint32_t)rows * row_bytes);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      hx::ld16_to_lds(kres, k_dst + (8 * w + 4 * j) * kTileRowBytes, koffs[j]);
      hx::ld16_to_lds(vres, v_dst + (8 * w + 4 * j) * kTileRowBytes, voffs[j]);
    }
  };

  // V^T operands of key step ks (keys 32 ks .. 32 ks + 31) of a V tile, dim block db in
  // vf[db]: lane (g, j) = (lane / 16, lane % 16) needs dim 16 db + j of keys 32 ks + 4g
  // + 0..3 and 32 ks + 16 + 4g + 0..3 (the key order of the P operand). Each transposing
  // read gives a 16-lane group the 4 x 16 block of 4 key rows x 16 dims its lanes address
  // (lane i: row i / 4, dims 4 (i % 4)..+3), lane j taking column j.
  auto read_v = [&](const uint8_t* vl, int ks, uint4 (&vf)[8]) __attribute__((always_inline)) {
    const int gg = lane >> 4, i = lane & 15;
    const int r0 = 32 * ks + 4 * gg + (i >> 2), r1 = r0 + 16;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int c = 2 * db + ((i >> 1) & 1);
      const uint2 lo = hx::ld8_lds_tr16(vl + r0 * kTileRowBytes + 16 * v_chunk_pos(r0, c) + 8 * (i & 1));
      const uint2 hi = hx::ld8_lds_tr16(vl + r1 * kTileRowBytes + 16 * v_chunk_pos(r1, c) + 8 * (i & 1));
      vf[db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  };

  // Tile t (in buffers kl, vl): wait for it, start tile t + 1 into (kn, vn), consume t.
  auto tile_step = [&](int t, const uint8_t* kl, const uint8_t* vl, uint8_t* kn, uint8_t* vn)
                       __attribute__((always_inline)) {
    // This wave's copies of tile t have landed; after the barrier, every wave's have, and
    // every wave is done with tile t - 1, whose buffers tile t + 1 now fills.
    __builtin_amdgcn_s_waitcnt(hx::kWaitVm0);
    __syncthreads();
    if (t + 1 < t_end) load_tile(t + 1, kn, vn);

    const int t0 = t * kTile;
    // S^T = K Q^T: lane holds keys 16kb+4(lane>>4)+i of row 16rb+(lane&15).
    hx::f32x4_t sacc[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) sacc[kb][rb] = hx::f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int kr = 16 * kb + (lane & 15);
        const uint4 af = *reinterpret_cast<const uint4*>(
            kl + kr * kTileRowBytes + 16 * k_chunk_pos(kr, 4 * st + (lane >> 4)));
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          sacc[kb][rb] = E::mfma16x16x32(hx::as_v8<T>(af), hx::as_v8<T>(qf[rb][st]), sacc[kb][rb]);
      }
    }

    // V operands of the first P V key step, in flight during the softmax.
    uint4 vf0[8];
    read_v(vl, 0, vf0);
    // Issue order for this block: 8 K fragment reads, then one more read after each pair
    // of QK MFMAs (a K read 8 fragments ahead of its use), then the V reads two per MFMA
    // pair under the last 16 MFMAs. Left to itself, hipcc issues each K read one or two
    // MFMA pairs ahead and waits for it at lgkmcnt(0).
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
    }

    // Mask only where the tile is not fully visible to every row of this wave (a
    // wave-uniform test, evaluated on the scalar unit).
    int full_i = (n - wr0 >= 32) & (t0 + kTile - 1 <= L - 1);
    full_i &= (a.win_left < 0) | (off + wr0 + 31 - a.win_left <= t0);
    full_i &= (a.win_right < 0) | (off + wr0 + a.win_right >= t0 + kTile - 1);
    const bool full = __builtin_amdgcn_readfirstlane(full_i) != 0;

    v8 pb[2][2];
    float mx[2];
    bool move[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (!full) {
        // Visible keys of this lane's row, relative to the lane's first key in the tile,
        // so each element compares its compile-time offset 16*kb + i.
        const int rr = wr0 + 16 * rb + (lane & 15);
        const int qpos = off + rr;
        const int kbase = t0 + 4 * (lane >> 4);
        const int rlo = a.win_left >= 0 ? qpos - a.win_left - kbase : -kTile;
        int rhi = L - 1;
        if (a.win_right >= 0) rhi = min(rhi, qpos + a.win_right);
        rhi = rr < n ? rhi - kbase : -1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // The lanes to mask as a lane mask in scalar registers, so the select is the
            // fast three-operand form (hx::lane_sel).
            const uint64_t hidden = __builtin_amdgcn_ballot_w64(16 * kb + i < rlo) |
                                    __builtin_amdgcn_ballot_w64(16 * kb + i > rhi);
            sacc[kb][rb][i] = hx::lane_sel(hidden, -INFINITY, sacc[kb][rb][i]);
          }
      }
      // Row max on raw scores (the scale is positive), folded into exp2 by one FMA.
      float m = fmaxf(fmaxf(sacc[0][rb][0], sacc[0][rb][1]), fmaxf(sacc[0][rb][2], sacc[0][rb][3]));
#pragma unroll
      for (int kb = 1; kb < 4; ++kb)
        m = fmaxf(m, fmaxf(fmaxf(sacc[kb][rb][0], sacc[kb][rb][1]), fmaxf(sacc[kb][rb][2], sacc[kb][rb][3])));
      mx[rb] = hx::max_xor32(hx::max_xor16(m));
      // Lazy max: the row's reference max moves only when the tile max exceeds it by more
      // than kLazyLog2 (log2 units). Until then p = 2^((s - m_run) * sl2) <= 2^kLazyLog2,
      // which the fp32 sums and bf16 P carry as accurately as p <= 1. With m_run = -inf
      // the test is mx > -inf (the first finite max sets it; alpha = 2^-inf = 0 then
      // multiplies the still-zero l and O); an all-masked tile (mx = -inf) never moves it.
      move[rb] = mx[rb] > m_run[rb] + lazy_thr;
    }
    // After a row's first tile its reference max rarely moves, so the factor alpha (two
    // exps), the new max and the rescale of l and of the 64 accumulators run in a
    // wave-uniform branch taken only when some row of the wave moved.
    if (__any(move[0] || move[1])) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const float alpha = move[rb] ? hx::fast_exp2((m_run[rb] - mx[rb]) * sl2) : 1.f;
        m_run[rb] = move[rb] ? mx[rb] : m_run[rb];
        l_run[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) oacc[db][rb] *= alpha;
      }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const float neg_m = m_run[rb] != -INFINITY ? -m_run[rb] * sl2 : 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sacc[kb][rb][i] = hx::fast_exp2(fmaf(sacc[kb][rb][i], sl2, neg_m));  // -inf -> 0
      // P in the MFMA's element type; the row sum adds the same rounded values (two per
      // dot2 against {1, 1}), so l matches the weights applied to V exactly.
      float psum = 0.f;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const hx::f32x4_t& x = sacc[2 * ks][rb];
        const hx::f32x4_t& y = sacc[2 * ks + 1][rb];
        const uint4 u = make_uint4(hx::pack2_round<T>(x[0], x[1]), hx::pack2_round<T>(x[2], x[3]),
                                   hx::pack2_round<T>(y[0], y[1]), hx::pack2_round<T>(y[2], y[3]));
        psum = hx::dot8<T>(u, hx::ones8<T>(), psum);
        pb[ks][rb] = hx::as_v8<T>(u);
      }
      l_run[rb] += psum;
    }

    // O^T += V^T P^T with the key order of pb: {4(lane>>4)+0..3, 16+4(lane>>4)+0..3}.
    // The first key step's V operands were read before the softmax.
    uint4 vf1[8];
    read_v(vl, 1, vf1);
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        oacc[db][rb] = E::mfma16x16x32(hx::as_v8<T>(vf0[db]), pb[0][rb], oacc[db][rb]);
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        oacc[db][rb] = E::mfma16x16x32(hx::as_v8<T>(vf1[db]), pb[1][rb], oacc[db][rb]);
    // The second key step's 16 V reads go out two per MFMA under the first step's
    // first 8 MFMAs (hipcc otherwise issues them four at a time between the second
    // step's MFMAs, each pair waiting for its reads).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 24, 1);
  };

  if (t_begin < t_end) load_tile(t_begin, k_lds0, v_lds0);
  for (int t = t_begin; t < t_end; t += 2) {
    tile_step(t, k_lds0, v_lds0, k_lds1, v_lds1);
    if (t + 1 < t_end) tile_step(t + 1, k_lds1, v_lds1, k_lds0, v_lds0);
  }

  if (bad_page && tid == 0) atomicOr(&a.hdr[H_ERR], HX_WERR_BAD_PAGE);

  // Normalise: lane holds dims 16db+4(lane>>4)+0..3 of row 16rb+(lane&15). The rows go
  // through this wave's LDS staging area and leave as whole 256-byte head rows, four per
  // store instruction (writing the fragment layout directly scatters 32-byte pieces of
  // 16 rows per instruction, about 2.5 us more per workgroup). A split writes its
  // partial (m in log2 units, l, o / l) to the row's slot instead of the output.
  const int64_t slot0 = S > 1 ? a.dec_cap + a.pf_base[item] + sp : 0;
  uint8_t* const stage = (w < 4 ? (w < 2 ? k_lds0 : k_lds1) : (w < 6 ? v_lds0 : v_lds1)) + (w & 1) * (32 * kTileRowBytes);
  __syncthreads();  // every wave is done with the tiles
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float l = hx::add_xor32(hx::add_xor16(l_run[rb]));
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int sr = 16 * rb + (lane & 15);
    uint8_t* const srow = stage + sr * kTileRowBytes + 8 * ((lane >> 4) & 1);
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<uint2*>(srow + 16 * k_chunk_pos(sr, 2 * db + (lane >> 5))) =
          make_uint2(hx::pack2_round<T>(oacc[db][rb][0] * inv, oacc[db][rb][1] * inv),
                     hx::pack2_round<T>(oacc[db][rb][2] * inv, oacc[db][rb][3] * inv));
    const int rr = wr0 + 16 * rb + (lane & 15);
    if (rr < n && (lane >> 4) == 0) {
      if (S > 1) {
        const int64_t slot = slot0 + (int64_t)(rr - row0) * S;
        if (slot < a.slot_cap) a.part_ml[slot * a.hq + qh] = make_float2(l > 0.f ? m_run[rb] * sl2 : -INFINITY, l);
      } else if (a.lse) {
        a.lse[(int64_t)qh * a.total_q + q0 + rr] = l > 0.f ? (m_run[rb] * sl2 + log2f(l)) * kLn2 : -INFINITY;
      }
    }
  }
  // Each wave reads back only the rows it staged, and one wave's LDS accesses complete in
  // order, so a wavefront-scope fence (no instruction, no barrier) orders the reads after
  // the writes. All eight reads go out before the first store; the stores carry the
  // non-temporal hint (C3 chunk 37.2 -> 35.4 us, the C5 tick's attention 0.08 ms less).
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  // Lane (r4, c) = (lane >> 4, lane & 15) stores the 16-byte chunk c of staged row 4i + r4.
  uint4 u[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int sr = 4 * i + (lane >> 4);
    u[i] = *reinterpret_cast<const uint4*>(stage + sr * kTileRowBytes + 16 * k_chunk_pos(sr, lane & 15));
  }
  if (S > 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = wr0 + 4 * i + (lane >> 4);
      const int64_t slot = slot0 + (int64_t)(rr - row0) * S;
      if (rr < n && slot < a.slot_cap) hx::st16_nt(a.part_o + (slot * a.hq + qh) * kD + 8 * (lane & 15), u[i]);
    }
    return;
  }
  // Output rows are 16-byte aligned unless the caller's strides or pointer are only
  // 8-byte aligned (allowed): then each chunk goes as two 8-byte stores.
  const bool out16 = a.o_row % 8 == 0 && a.o_head % 8 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0;
  uint16_t* const o0 = reinterpret_cast<uint16_t*>(a.out) + (int64_t)qh * a.o_head + 8 * (lane & 15);
  if (out16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = wr0 + 4 * i + (lane >> 4);
      if (rr < n) hx::st16_nt(o0 + (int64_t)(q0 + rr) * a.o_row, u[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = wr0 + 4 * i + (lane >> 4);
      if (rr < n) {
        uint16_t* o = o0 + (int64_t)(q0 + rr) * a.o_row;
        hx::st8_nt(o, u[i].x, u[i].y);
        hx::st8_nt(o + 4, u[i].z, u[i].w);
      }
    }
  }
}

template <typename T, int G>
__global__ __launch_bounds__(kChunkThreads, 2) void chunk_kernel(RunArgs a) {
  chunk_body<T, G>(a, hx::wg_x(), false);
}

// One launch for two plans' chunk items (a cascade's batch and its level batch, run in
// one call): workgroups [0, a0.grid_pf * hkv) take a0's items, the rest a1's, each
// through its own copy of the body, which reads that plan's arguments directly. a0's
// come first, so the level batch's short items fill the tail of a0's round.
template <typename T, int G>
__global__ __launch_bounds__(kChunkThreads, 2) void chunk_pair_kernel(RunArgs a0, RunArgs a1) {
  const int n0 = a0.grid_pf * a0.hkv;
  const int wg = hx::wg_x();
  if (wg < n0)
    chunk_body<T, G>(a0, wg, false);
  else
    chunk_body<T, G>(a1, wg - n0, true);
}

// ------------------------------------------------------------------ any head_dim
// Attention for shapes the tuned kernels do not cover: head_dim any multiple of 8 up to
// 256, and any group size G. One workgroup per (sequence, block of query rows, KV head
// g, block of up to kGenUnits of g's query heads); its (row, head) units share every K/V
// tile read. Keys go through LDS kGenTile at a time. Lane j scores key j of the tile for
// each of its wave's units, the softmax runs online per unit in fp32, and lane j
// accumulates O for dims j, j + 64, ... of every unit, reading each key's p from LDS.
// Decode and chunk rows alike, with no split-K: head_dim 128 with G in {1, 2, 4, 8}
// goes to the decode / chunk kernels instead.
constexpr int kGenUnits = 16;    // (row, head) units per workgroup, 4 per wave
constexpr int kGenTile = 64;     // keys per LDS tile: one per lane

struct GenericShape {
  int32_t head_dim, group, heads_per_item, rows_per_item, row_blocks, head_blocks;
};

inline GenericShape generic_shape(int max_q, int G, int head_dim) {
  GenericShape g;
  g.head_dim = head_dim;
  g.group = G;
  g.heads_per_item = G < kGenUnits ? G : kGenUnits;
  g.rows_per_item = kGenUnits / g.heads_per_item;
  g.row_blocks = (int)ceil_div(max_q > 0 ? max_q : 1, g.rows_per_item);
  g.head_blocks = (int)ceil_div(G, g.heads_per_item);
  return g;
}

template <typename T, int DMAX>
__global__ __launch_bounds__(256) void generic_kernel(RunArgs a, GenericShape gs) {
  typedef hx::Elem<T> E;
  constexpr int KS = DMAX + 8;                      // K tile row stride (elements)
  constexpr int NC = DMAX >= 64 ? DMAX / 64 : 1;    // O dims per lane and unit
  __shared__ __attribute__((aligned(16))) T k_lds[kGenTile * KS];
  __shared__ __attribute__((aligned(16))) T v_lds[kGenTile * DMAX];
  __shared__ __attribute__((aligned(16))) float q_lds[kGenUnits * DMAX];
  __shared__ float p_lds[kGenUnits][kGenTile];

  const int tid = hx::tid_x(), lane = tid & 63, w = tid >> 6;
  const int D = gs.head_dim;
  int x = hx::wg_x();
  const int hb = x % gs.head_blocks;
  x /= gs.head_blocks;
  const int g = x % a.hkv;
  x /= a.hkv;
  const int rb = x % gs.row_blocks;
  const int b = x / gs.row_blocks;
  const Header hd = read_header(a);
  if (!hd.ok || b >= a.batch) return;
  const int4 si = a.seq_info[b];
  const int q0 = si.x, n = si.y, L = si.z, kvb = si.w;
  const int row0 = rb * gs.rows_per_item;
  if (row0 >= n) return;
  const int rows = min(gs.rows_per_item, n - row0);
  const int h0 = hb * gs.heads_per_item;
  const int hcount = min(gs.heads_per_item, gs.group - h0);
  const int units = rows * hcount;  // unit u: row row0 + u / hcount, head g*G + h0 + u % hcount

  // The units' queries, widened to fp32.
  for (int idx = tid; idx < units * D; idx += 256) {
    const int u = idx / D, d = idx - (idx / D) * D;
    const int64_t qrow = query_row(a, q0 + row0 + u / hcount);
    const int qh = g * gs.group + h0 + u % hcount;
    q_lds[u * DMAX + d] = E::lo(reinterpret_cast<const uint16_t*>(a.q)[qrow * a.q_row + (int64_t)qh * a.q_head + d]);
  }
  // Keys any row of the block can see: [klo, khi].
  const int qfirst = L - n + row0, qlast = L - n + row0 + rows - 1;
  const int klo = a.win_left >= 0 ? max(0, qfirst - a.win_left) : 0;
  int khi = L - 1;
  if (a.win_right >= 0) khi = min(khi, qlast + a.win_right);

  float m[4], l[4], o[4][NC];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    m[k] = -INFINITY;
    l[k] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) o[k][c] = 0.f;
  }
  const int chunks = D / 8;  // 16-byte pieces of a head row
  const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)g * a.kv_head;
  const T* vbase = reinterpret_cast<const T*>(a.v) + (int64_t)g * a.kv_head;
  for (int t0 = khi >= klo ? (klo / kGenTile) * kGenTile : 0; khi >= klo && t0 <= khi; t0 += kGenTile) {
    __syncthreads();  // the previous tile's readers are done
    // K and V rows of keys t0 .. t0 + 63; keys past L - 1 re-read row L - 1 (masked).
    for (int idx = tid; idx < kGenTile * chunks; idx += 256) {
      const int key = idx / chunks, c8 = idx - (idx / chunks) * chunks;
      const int kk = min(t0 + key, L - 1);
      int64_t row;
      if (a.page_size > 0) {
        int page = a.bt[(int64_t)b * a.bt_stride + kk / a.page_size];
        if ((unsigned)page >= (unsigned)a.num_pages) {
          atomicOr(&a.hdr[H_ERR], HX_WERR_BAD_PAGE);
          page = 0;
        }
        row = (int64_t)page * a.page_size + kk % a.page_size;
      } else {
        row = (int64_t)kvb + kk;
      }
      *reinterpret_cast<uint4*>(&k_lds[key * KS + 8 * c8]) = ld16(kbase + row * a.kv_row + 8 * c8);
      *reinterpret_cast<uint4*>(&v_lds[key * DMAX + 8 * c8]) = ld16(vbase + row * a.kv_row + 8 * c8);
    }
    __syncthreads();
    // Scores and online softmax: lane j holds key t0 + j of each of the wave's units.
    const int kk = t0 + lane;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int c8 = 0; c8 < chunks; ++c8) {
      const uint4 kv = *reinterpret_cast<const uint4*>(&k_lds[lane * KS + 8 * c8]);
      const float kf[8] = {E::lo(kv.x), E::hi(kv.x), E::lo(kv.y), E::hi(kv.y),
                           E::lo(kv.z), E::hi(kv.z), E::lo(kv.w), E::hi(kv.w)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int u = w + 4 * k;
        if (u < units) {
          const float4 qa = *reinterpret_cast<const float4*>(&q_lds[u * DMAX + 8 * c8]);
          const float4 qb = *reinterpret_cast<const float4*>(&q_lds[u * DMAX + 8 * c8 + 4]);
          s[k] += qa.x * kf[0] + qa.y * kf[1] + qa.z * kf[2] + qa.w * kf[3] +
                  qb.x * kf[4] + qb.y * kf[5] + qb.z * kf[6] + qb.w * kf[7];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = w + 4 * k;
      if (u >= units) continue;  // wave-uniform
      const int qpos = L - n + row0 + u / hcount;
      const bool vis = kk <= L - 1 && (a.win_left < 0 || kk >= qpos - a.win_left) &&
                       (a.win_right < 0 || kk <= qpos + a.win_right);
      const float sc = vis ? s[k] * a.scale_log2 : -INFINITY;
      const float m_new = fmaxf(m[k], wave_max(sc));
      float p = 0.f, alpha = 1.f;
      if (m_new != -INFINITY) {
        p = vis ? hx::fast_exp2(sc - m_new) : 0.f;
        alpha = m[k] == -INFINITY ? 0.f : hx::fast_exp2(m[k] - m_new);
      }
      l[k] = l[k] * alpha + wave_sum(p);
      m[k] = m_new;
#pragma unroll
      for (int c = 0; c < NC; ++c) o[k][c] *= alpha;
      p_lds[u][lane] = p;
    }
    __syncthreads();
    // O += P V: lane owns dims lane + 64c.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = w + 4 * k;
      if (u >= units) continue;
      for (int j = 0; j < kGenTile; ++j) {
        const float pj = p_lds[u][j];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int d = lane + 64 * c;
          if (d < D) o[k][c] = fmaf(pj, E::lo(reinterpret_cast<const uint16_t*>(v_lds)[j * DMAX + d]), o[k][c]);
        }
      }
    }
  }
  // Normalise and store every unit of this wave.
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int u = w + 4 * k;
    if (u >= units) continue;
    const int64_t orow = q0 + row0 + u / hcount;
    const int qh = g * gs.group + h0 + u % hcount;
    const float inv = l[k] > 0.f ? 1.f / l[k] : 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = lane + 64 * c;
      if (d < D)
        reinterpret_cast<uint16_t*>(a.out)[orow * a.o_row + (int64_t)qh * a.o_head + d] = E::bits(o[k][c] * inv);
    }
    if (a.lse && lane == 0)
      a.lse[(int64_t)qh * a.total_q + orow] = l[k] > 0.f ? (m[k] + log2f(l[k])) * kLn2 : -INFINITY;
  }
}

// ------------------------------------------------------------------ host helpers
bool valid_group(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }

// Decode work items the launch covers: grid_dec rounded up to whole rounds of the XCDs.
int64_t decode_grid(int64_t grid_dec) { return (grid_dec + kXcds - 1) / kXcds * kXcds; }

template <typename T, int G>
int launch_run(const RunArgs& a, const RunArgs* side_pf, hipStream_t s) {
  // A second plan's chunk items (side_pf: a cascade's level batch, run in this call) share
  // one chunk launch with this plan's, first: the level batch's combine records below read
  // its partials. This call then appends nothing, so this plan's chunk rows need no
  // decode launch before them.
  if (side_pf != nullptr && (a.grid_pf > 0 || side_pf->grid_pf > 0))
    hipLaunchKernelGGL((chunk_pair_kernel<T, G>), dim3((unsigned)((a.grid_pf + side_pf->grid_pf) * a.hkv)),
                       dim3(kChunkThreads), 0, s, a, *side_pf);
  // The combine merges decode and chunk split partials, so it runs last. A second plan's
  // combine records (a.sc_wgs) follow the decode workgroups of the decode launch, as
  // 256-thread workgroups like that plan's own combine launch; when this call has no
  // decode launch, or that plan's rows want 512-thread workgroups, they get a combine
  // launch of their own first.
  const bool sc_wide = ceil_div(a.sc_max_k, kSplit) > kCombSmallSplits;
  const bool sc_in_decode = a.sc_wgs > 0 && a.grid_dec > 0 && !sc_wide;
  if (a.sc_wgs > 0 && !sc_in_decode) {
    if (sc_wide)
      hipLaunchKernelGGL((combine_kernel<T, G, 512>), dim3((unsigned)a.sc_wgs), dim3(512), 0, s, side_combine_args(a));
    else
      hipLaunchKernelGGL((combine_kernel<T, G, 256>), dim3((unsigned)a.sc_wgs), dim3(256), 0, s, side_combine_args(a));
  }
  const unsigned dec_wgs = (unsigned)(decode_grid(a.grid_dec) * a.hkv);
  if (sc_in_decode)
    hipLaunchKernelGGL((decode_kernel<T, G, kExtraCombine>), dim3(dec_wgs + (unsigned)(a.app_wgs + a.sc_wgs)),
                       dim3(kThreads), 0, s, a);
  else if (a.app_wgs > 0)
    hipLaunchKernelGGL((decode_kernel<T, G, kExtraAppend>), dim3(dec_wgs + (unsigned)a.app_wgs), dim3(kThreads), 0, s,
                       a);
  else if (a.grid_dec > 0)
    hipLaunchKernelGGL((decode_kernel<T, G, kExtraNone>), dim3(dec_wgs), dim3(kThreads), 0, s, a);
  if (a.grid_pf > 0 && side_pf == nullptr)
    hipLaunchKernelGGL((chunk_kernel<T, G>), dim3((unsigned)(a.grid_pf * a.hkv)), dim3(kChunkThreads), 0, s, a);
  // A cascade merge adds workgroups for its members whose rows have no combine record;
  // it runs in this launch whenever it is given (the call that holds the combine phase).
  const bool wide = ceil_div(a.max_k, kSplit) > kCombSmallSplits;
  const int64_t merge_wgs = a.mg_start != nullptr ? ceil_div((int64_t)a.mg_members * a.hq, (wide ? 512 : 256) / 16) : 0;
  if (a.grid_comb > 0 || merge_wgs > 0) {
    const unsigned grid = (unsigned)((int64_t)a.grid_comb * a.hkv + merge_wgs);
    if (wide)
      hipLaunchKernelGGL((combine_kernel<T, G, 512>), dim3(grid), dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((combine_kernel<T, G, 256>), dim3(grid), dim3(256), 0, s, a);
  }
  return hx::status_from_hip(hipGetLastError());
}

template <typename T>
int launch_run_g(const RunArgs& a, const RunArgs* side_pf, int G, hipStream_t s) {
  switch (G) {
    case 1: return launch_run<T, 1>(a, side_pf, s);
    case 2: return launch_run<T, 2>(a, side_pf, s);
    case 4: return launch_run<T, 4>(a, side_pf, s);
    case 8: return launch_run<T, 8>(a, side_pf, s);
    default: return HX_E_UNSUPPORTED;
  }
}

// head_dim 128 with G in {1, 2, 4, 8} runs the decode / chunk / combine kernels; every
// other supported shape runs generic_kernel.
bool tuned_shape(int G, int head_dim) { return head_dim == kD && valid_group(G); }

int check_shape(int batch, int max_q, int max_k, int hq, int hkv, int head_dim) {
  if (batch < 0 || max_q < 0 || max_k < 0 || hq < 1 || hkv < 1) return HX_E_INVALID_ARG;
  if (hq % hkv) return HX_E_INVALID_ARG;
  if (head_dim < 8 || head_dim > 256 || head_dim % 8) return HX_E_UNSUPPORTED;
  return HX_OK;
}

template <typename T>
int launch_generic(const RunArgs& a, const GenericShape& gs, hipStream_t s) {
  const int64_t grid = (int64_t)a.batch * gs.row_blocks * a.hkv * gs.head_blocks;
  if (grid > INT32_MAX) return HX_E_INVALID_ARG;
  if (grid == 0) return HX_OK;
  const dim3 g3((unsigned)grid), b3(256);
  if (gs.head_dim <= 32)
    hipLaunchKernelGGL((generic_kernel<T, 32>), g3, b3, 0, s, a, gs);
  else if (gs.head_dim <= 64)
    hipLaunchKernelGGL((generic_kernel<T, 64>), g3, b3, 0, s, a, gs);
  else if (gs.head_dim <= 128)
    hipLaunchKernelGGL((generic_kernel<T, 128>), g3, b3, 0, s, a, gs);
  else
    hipLaunchKernelGGL((generic_kernel<T, 256>), g3, b3, 0, s, a, gs);
  return hx::status_from_hip(hipGetLastError());
}

}  // namespace

extern "C" {

size_t hx_varlen_attn_workspace_bytes(int32_t batch, int32_t max_q, int32_t max_k,
                                      int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim) {
  if (check_shape(batch, max_q, max_k, n_q_heads, n_kv_heads, head_dim) != HX_OK) return 0;
  return make_layout(batch, max_q, max_k, n_q_heads, n_kv_heads).total;
}

size_t hx_varlen_attn_error_word_offset(void) { return H_ERR * sizeof(int32_t); }

int hx_varlen_attn_count_items(const int32_t* q_lens, const int32_t* k_lens, int32_t batch,
                               int32_t n_q_heads, int32_t n_kv_heads,
                               int32_t window_left, int32_t window_right,
                               int32_t* decode_items, int32_t* prefill_items,
                               int32_t* combine_seqs) {
  if (batch < 0 || n_q_heads < 1 || n_kv_heads < 1 || n_q_heads % n_kv_heads) return HX_E_INVALID_ARG;
  if (batch > 0 && (!q_lens || !k_lens)) return HX_E_INVALID_ARG;
  if (!decode_items || !prefill_items || !combine_seqs) return HX_E_INVALID_ARG;
  const Geometry geo = geometry(n_q_heads, n_kv_heads);
  // Same two passes as plan_kernel: chunk items and tiles unsplit, then the split.
  int64_t items0 = 0, tiles0 = 0;
  int max_tiles = 0;
  for (int b = 0; b < batch; ++b) {
    const int n = q_lens[b], L = k_lens[b];
    if (n < 0 || L < 0) return HX_E_INVALID_ARG;
    if (n < 2) continue;
    for (int row0 = 0; row0 < n; row0 += geo.rows_per_item) {
      int tb, te;
      chunk_tiles(n, L, row0, geo.rows_per_item, window_left, window_right, &tb, &te);
      tiles0 += (int64_t)(te - tb) * geo.head_quads;
      items0 += geo.head_quads;
      max_tiles = te - tb > max_tiles ? te - tb : max_tiles;
    }
  }
  auto chunk_wgs = [&](int st) -> int64_t {
    int64_t total = 0;
    for (int b = 0; b < batch; ++b) {
      const int n = q_lens[b], L = k_lens[b];
      if (n < 2) continue;
      for (int row0 = 0; row0 < n; row0 += geo.rows_per_item) {
        int tb, te;
        chunk_tiles(n, L, row0, geo.rows_per_item, window_left, window_right, &tb, &te);
        total += (int64_t)chunk_split_count(te - tb, st) * geo.head_quads;
      }
    }
    return total * n_kv_heads;
  };
  const int split_tiles = refine_split_tiles(chunk_split_tiles(tiles0, items0, n_kv_heads), max_tiles,
                                             chunk_keep_tiles(tiles0, n_kv_heads, 0), chunk_wgs);
  const int keep_tiles = chunk_keep_tiles(tiles0, n_kv_heads, split_tiles);
  int64_t nd = 0, np = 0, nc = 0;
  for (int b = 0; b < batch; ++b) {
    const int n = q_lens[b], L = k_lens[b];
    if (n == 1) {
      int first, count;
      decode_splits(L, window_left, &first, &count);
      nd += count;
      nc += count > 1;
    } else if (n >= 2) {
      for (int row0 = 0; row0 < n; row0 += geo.rows_per_item) {
        int tb, te;
        chunk_tiles(n, L, row0, geo.rows_per_item, window_left, window_right, &tb, &te);
        const int S = chunk_split_count(te - tb, split_tiles, keep_tiles);
        np += (int64_t)S * geo.head_quads;
        if (S > 1) nc += ceil_div(n - row0 < geo.rows_per_item ? n - row0 : geo.rows_per_item, kCombRows);
      }
    }
  }
  if (nd > INT32_MAX || np > INT32_MAX || nc > INT32_MAX) return HX_E_INVALID_ARG;
  *decode_items = (int32_t)nd;
  *prefill_items = (int32_t)np;
  *combine_seqs = (int32_t)nc;
  return HX_OK;
}

int hx_varlen_attn_plan(const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                        const int32_t* seqused_k, int32_t batch, int32_t total_q,
                        int32_t max_q, int32_t max_k, int64_t total_k_rows,
                        int32_t page_size, int32_t block_table_stride,
                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t window_left, int32_t window_right,
                        void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_shape(batch, max_q, max_k, n_q_heads, n_kv_heads, head_dim);
  if (st != HX_OK) return st;
  if (total_q < 0 || page_size < 0 || (page_size > 0 && page_size % kSplit)) return HX_E_INVALID_ARG;
  if (page_size > 0 && block_table_stride < 1) return HX_E_INVALID_ARG;
  if (page_size == 0 && (!cu_seq_k || total_k_rows < 0)) return HX_E_INVALID_ARG;
  if (batch > 0 && !cu_seq_q) return HX_E_INVALID_ARG;
  if (batch > 0 && !seqused_k && !cu_seq_k) return HX_E_INVALID_ARG;
  const Layout l = make_layout(batch, max_q, max_k, n_q_heads, n_kv_heads);
  if (!workspace || (uintptr_t)workspace % 256 || workspace_bytes < l.total) return HX_E_WORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const Geometry geo = geometry(n_q_heads, n_kv_heads);
  PlanArgs a;
  a.cu_q = cu_seq_q;
  a.cu_k = cu_seq_k;
  a.used_k = seqused_k;
  a.hdr = reinterpret_cast<int32_t*>(ws);
  a.seq_info = reinterpret_cast<int4*>(ws + l.seq_info);
  a.dec_items = reinterpret_cast<int4*>(ws + l.dec_items);
  a.comb_seqs = reinterpret_cast<int4*>(ws + l.comb_seqs);
  a.pf_items = reinterpret_cast<int4*>(ws + l.pf_items);
  a.pf_base = reinterpret_cast<int32_t*>(ws + l.pf_base);
  a.pf_seq = reinterpret_cast<int4*>(ws + l.pf_seq);
  a.total_k_rows = total_k_rows;
  a.max_dec = l.max_dec;
  a.max_pf = l.max_pf;
  a.max_comb = l.max_comb;
  a.cslot_cap = l.cslot_cap;
  a.batch = batch;
  a.total_q = total_q;
  a.max_q = max_q;
  a.max_k = max_k;
  a.page_size = page_size;
  a.bt_stride = block_table_stride;
  a.rows_per_item = geo.rows_per_item;
  a.head_quads = geo.head_quads;
  a.win_left = window_left;
  a.win_right = window_right;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, static_cast<hipStream_t>(stream), a);
  return hx::status_from_hip(hipGetLastError());
}

}  // extern "C"

namespace {

struct MergeSpec {
  const void* level_out;
  int64_t level_row, level_head;
  const float* level_lse;
  int64_t level_rows;
  const int32_t* member_seq;
  const int32_t* member_of_seq;
  int32_t n_members;
  const int32_t* part_start;
  const int32_t* part_idx;
  int32_t n_parts;
  // The level batch's own plan, when this call also runs that plan's combine phase
  // (level_ws == nullptr: it ran before; level_out / level_lse hold its results).
  void* level_ws;
  size_t level_ws_bytes;
  int32_t level_batch, level_max_q, level_max_k, level_comb_hint;
  // The level batch's chunk phase too, in this call's chunk launch (level_bt == nullptr:
  // it ran before): its block table, query row map and chunk-item hint.
  const int32_t* level_bt;
  int32_t level_bt_stride;
  const int64_t* level_q_rows;
  int64_t level_q_rows_total;
  int32_t level_pf_hint;
  int32_t level_win_left, level_win_right;
};

struct AppendSpec {
  const void* k_new;
  const void* v_new;
  int64_t kn_row, kn_head, vn_row, vn_head;
  const int64_t* write_slots;
  int64_t pool_rows;
};

int run_impl(const void* q, int64_t q_row_stride, int64_t q_head_stride,
             const int64_t* q_rows, int64_t q_rows_total,
             const void* k_cache, const void* v_cache,
             int64_t kv_row_stride, int64_t kv_head_stride,
             int32_t num_pages, int32_t page_size,
             const int32_t* block_table, int32_t block_table_stride,
             int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
             float scale, int32_t window_left, int32_t window_right,
             int32_t dtype,
             void* out, int64_t o_row_stride, int64_t o_head_stride,
             float* lse,
             int32_t decode_items_hint, int32_t prefill_items_hint,
             int32_t combine_seqs_hint,
             void* workspace, size_t workspace_bytes, void* stream, const AppendSpec* app,
             const MergeSpec* mg = nullptr) {
  int st = check_shape(batch, max_q, max_k, n_q_heads, n_kv_heads, head_dim);
  if (st != HX_OK) return st;
  if (dtype != HX_DTYPE_BF16 && dtype != HX_DTYPE_FP16) return HX_E_UNSUPPORTED;
  if (total_q < 0 || page_size < 0 || (page_size > 0 && page_size % kSplit)) return HX_E_INVALID_ARG;
  if (page_size > 0 && (num_pages < 1 || block_table_stride < 1 || !block_table)) return HX_E_INVALID_ARG;
  if (!(scale > 0.f) || !isfinite(scale)) return HX_E_INVALID_ARG;
  // 16-byte vector loads of q / K / V rows and 8-byte stores of output rows.
  if (!q || !k_cache || !v_cache || !out) return batch == 0 ? HX_OK : HX_E_INVALID_ARG;
  if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 || (uintptr_t)out % 8)
    return HX_E_INVALID_ARG;
  if (q_row_stride % 8 || q_head_stride % 8 || kv_row_stride % 8 || kv_head_stride % 8 ||
      o_row_stride % 4 || o_head_stride % 4)
    return HX_E_INVALID_ARG;
  if (q_row_stride < 0 || q_head_stride < 0 || kv_row_stride < 0 || kv_head_stride < 0 ||
      o_row_stride < 0 || o_head_stride < 0)
    return HX_E_INVALID_ARG;
  // Per-split row offsets are 32-bit: 256 rows of kv_row_stride must fit.
  if (kv_row_stride > (int64_t)(1 << 23)) return HX_E_INVALID_ARG;
  const Layout l = make_layout(batch, max_q, max_k, n_q_heads, n_kv_heads);
  if (!workspace || (uintptr_t)workspace % 256 || workspace_bytes < l.total) return HX_E_WORKSPACE;
  if (batch == 0) return HX_OK;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  RunArgs a;
  a.q = static_cast<const uint8_t*>(q);
  a.k = static_cast<const uint8_t*>(k_cache);
  a.v = static_cast<const uint8_t*>(v_cache);
  a.out = static_cast<uint8_t*>(out);
  a.lse = lse;
  a.bt = block_table;
  a.hdr = reinterpret_cast<int32_t*>(ws);
  a.seq_info = reinterpret_cast<const int4*>(ws + l.seq_info);
  a.dec_items = reinterpret_cast<const int4*>(ws + l.dec_items);
  a.comb_seqs = reinterpret_cast<const int4*>(ws + l.comb_seqs);
  a.pf_items = reinterpret_cast<const int4*>(ws + l.pf_items);
  a.pf_base = reinterpret_cast<const int32_t*>(ws + l.pf_base);
  a.pf_seq = reinterpret_cast<const int4*>(ws + l.pf_seq);
  a.part_ml = reinterpret_cast<float2*>(ws + l.part_ml);
  a.part_o = reinterpret_cast<uint16_t*>(ws + l.part_o);
  a.dec_cap = l.max_dec;
  a.slot_cap = l.max_dec + l.cslot_cap;
  a.q_row = q_row_stride;
  a.q_head = q_head_stride;
  a.kv_row = kv_row_stride;
  a.kv_head = kv_head_stride;
  a.o_row = o_row_stride;
  a.o_head = o_head_stride;
  a.num_pages = num_pages;
  a.page_size = page_size;
  a.bt_stride = block_table_stride;
  a.batch = batch;
  a.max_q = max_q;
  a.max_k = max_k;
  a.total_q = total_q;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.win_left = window_left;
  a.win_right = window_right;
  auto clamp_hint = [](int32_t hint, int64_t bound) -> int32_t {
    if (hint < 0 || hint > bound) return (int32_t)bound;
    return hint;
  };
  a.grid_dec = clamp_hint(decode_items_hint, l.max_dec);
  a.grid_pf = max_q >= 2 ? clamp_hint(prefill_items_hint, l.max_pf) : 0;
  a.grid_comb = clamp_hint(combine_seqs_hint, l.max_comb);
  if (decode_grid(a.grid_dec) * n_kv_heads + kAppendWGs > INT32_MAX || (int64_t)a.grid_pf * n_kv_heads > INT32_MAX)
    return HX_E_INVALID_ARG;
  a.k_new = nullptr;
  a.v_new = nullptr;
  a.write_slots = nullptr;
  a.kn_row = a.kn_head = a.vn_row = a.vn_head = 0;
  a.pool_rows = 0;
  a.app_wgs = 0;
  a.q_rows = q_rows;
  a.q_rows_total = q_rows_total;
  a.mg_o = nullptr;
  a.mg_o_row = a.mg_o_head = 0;
  a.mg_lse = nullptr;
  a.mg_lse_stride = a.mg_rows = 0;
  a.mg_seq = a.mg_of_seq = a.mg_start = a.mg_idx = nullptr;
  a.mg_members = a.mg_n_idx = 0;
  a.sc_hdr = nullptr;
  a.sc_comb_seqs = nullptr;
  a.sc_part_ml = nullptr;
  a.sc_part_o = nullptr;
  a.sc_out = nullptr;
  a.sc_lse = nullptr;
  a.sc_o_row = a.sc_o_head = a.sc_dec_cap = a.sc_slot_cap = 0;
  a.sc_batch = a.sc_max_q = a.sc_max_k = a.sc_total_q = a.sc_grid_comb = a.sc_wgs = 0;
  RunArgs side_pf;
  bool has_side_pf = false;
  if (mg != nullptr && mg->level_ws != nullptr) {
    // The level plan: same heads and pools, its own workspace, outputs level_out / level_lse
    // ([level_rows] rows, lse [n_q_heads, level_rows]). Its combine records run in this
    // call, before the merge reads their rows.
    if (!tuned_shape(n_q_heads / n_kv_heads, head_dim)) return HX_E_UNSUPPORTED;
    st = check_shape(mg->level_batch, mg->level_max_q, mg->level_max_k, n_q_heads, n_kv_heads, head_dim);
    if (st != HX_OK) return st;
    if (mg->level_rows < 0 || mg->level_rows > INT32_MAX || !mg->level_out || !mg->level_lse)
      return HX_E_INVALID_ARG;
    if ((uintptr_t)mg->level_out % 8 || mg->level_row % 4 || mg->level_head % 4 || mg->level_row < 0 ||
        mg->level_head < 0)
      return HX_E_INVALID_ARG;
    const Layout la = make_layout(mg->level_batch, mg->level_max_q, mg->level_max_k, n_q_heads, n_kv_heads);
    if ((uintptr_t)mg->level_ws % 256 || mg->level_ws_bytes < la.total) return HX_E_WORKSPACE;
    if (mg->level_batch > 0) {
      uint8_t* lw = static_cast<uint8_t*>(mg->level_ws);
      a.sc_hdr = reinterpret_cast<int32_t*>(lw);
      a.sc_comb_seqs = reinterpret_cast<const int4*>(lw + la.comb_seqs);
      a.sc_part_ml = reinterpret_cast<float2*>(lw + la.part_ml);
      a.sc_part_o = reinterpret_cast<uint16_t*>(lw + la.part_o);
      a.sc_out = static_cast<uint8_t*>(const_cast<void*>(mg->level_out));
      a.sc_lse = const_cast<float*>(mg->level_lse);
      a.sc_o_row = mg->level_row;
      a.sc_o_head = mg->level_head;
      a.sc_dec_cap = la.max_dec;
      a.sc_slot_cap = la.max_dec + la.cslot_cap;
      a.sc_batch = mg->level_batch;
      a.sc_max_q = mg->level_max_q;
      a.sc_max_k = mg->level_max_k;
      a.sc_total_q = (int32_t)mg->level_rows;
      a.sc_grid_comb = clamp_hint(mg->level_comb_hint, la.max_comb);
      const int64_t wgs = (int64_t)a.sc_grid_comb * n_kv_heads;
      if (wgs > INT32_MAX - decode_grid(a.grid_dec) * n_kv_heads - kAppendWGs) return HX_E_INVALID_ARG;
      a.sc_wgs = (int32_t)wgs;
    }
    if (mg->level_bt != nullptr && mg->level_batch > 0) {
      // The level plan's chunk items in this call's chunk launch: the same pools, heads
      // and scale, its own window, block table, row map, workspace and outputs. That
      // launch comes first (the level's combine records read its partials), so this call
      // appends nothing.
      if (app != nullptr) return HX_E_INVALID_ARG;
      if (page_size > 0 && mg->level_bt_stride < 1) return HX_E_INVALID_ARG;
      if (!mg->level_q_rows || mg->level_q_rows_total < 0) return HX_E_INVALID_ARG;
      uint8_t* lw = static_cast<uint8_t*>(mg->level_ws);
      side_pf = a;
      side_pf.out = static_cast<uint8_t*>(const_cast<void*>(mg->level_out));
      side_pf.lse = const_cast<float*>(mg->level_lse);
      side_pf.o_row = mg->level_row;
      side_pf.o_head = mg->level_head;
      side_pf.bt = mg->level_bt;
      side_pf.bt_stride = mg->level_bt_stride;
      side_pf.hdr = reinterpret_cast<int32_t*>(lw);
      side_pf.seq_info = reinterpret_cast<const int4*>(lw + la.seq_info);
      side_pf.dec_items = reinterpret_cast<const int4*>(lw + la.dec_items);
      side_pf.comb_seqs = reinterpret_cast<const int4*>(lw + la.comb_seqs);
      side_pf.pf_items = reinterpret_cast<const int4*>(lw + la.pf_items);
      side_pf.pf_base = reinterpret_cast<const int32_t*>(lw + la.pf_base);
      side_pf.pf_seq = reinterpret_cast<const int4*>(lw + la.pf_seq);
      side_pf.part_ml = reinterpret_cast<float2*>(lw + la.part_ml);
      side_pf.part_o = reinterpret_cast<uint16_t*>(lw + la.part_o);
      side_pf.dec_cap = la.max_dec;
      side_pf.slot_cap = la.max_dec + la.cslot_cap;
      side_pf.batch = mg->level_batch;
      side_pf.max_q = mg->level_max_q;
      side_pf.max_k = mg->level_max_k;
      side_pf.total_q = (int32_t)mg->level_rows;
      side_pf.grid_dec = 0;
      side_pf.grid_pf = mg->level_max_q >= 2 ? clamp_hint(mg->level_pf_hint, la.max_pf) : 0;
      side_pf.grid_comb = 0;
      side_pf.win_left = mg->level_win_left;
      side_pf.win_right = mg->level_win_right;
      side_pf.q_rows = mg->level_q_rows;
      side_pf.q_rows_total = mg->level_q_rows_total;
      side_pf.sc_wgs = 0;
      if (((int64_t)a.grid_pf + side_pf.grid_pf) * n_kv_heads > INT32_MAX) return HX_E_INVALID_ARG;
      has_side_pf = true;
    }
  }
  if (mg != nullptr && mg->n_members > 0) {
    // Tuned shapes only (the merge runs in the combine launch); 16-byte rows for the
    // merged stores and loads; the lse of every row (the unsplit members' merge reads it).
    if (!tuned_shape(n_q_heads / n_kv_heads, head_dim)) return HX_E_UNSUPPORTED;
    if (!lse || !mg->level_out || !mg->level_lse || !mg->member_seq || !mg->member_of_seq ||
        !mg->part_start || (mg->n_parts > 0 && !mg->part_idx))
      return HX_E_INVALID_ARG;
    if (mg->level_rows < 0 || mg->n_parts < 0 || mg->level_row < 0 || mg->level_head < 0)
      return HX_E_INVALID_ARG;
    if ((uintptr_t)out % 16 || o_row_stride % 8 || o_head_stride % 8 || (uintptr_t)mg->level_out % 16 ||
        mg->level_row % 8 || mg->level_head % 8)
      return HX_E_INVALID_ARG;
    a.mg_o = static_cast<const uint16_t*>(mg->level_out);
    a.mg_o_row = mg->level_row;
    a.mg_o_head = mg->level_head;
    a.mg_lse = mg->level_lse;
    a.mg_lse_stride = mg->level_rows;
    a.mg_rows = mg->level_rows;
    a.mg_seq = mg->member_seq;
    a.mg_of_seq = mg->member_of_seq;
    a.mg_start = mg->part_start;
    a.mg_idx = mg->part_idx;
    a.mg_members = mg->n_members;
    a.mg_n_idx = mg->n_parts;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int G = n_q_heads / n_kv_heads;
  const bool tuned = tuned_shape(G, head_dim);
  if (app != nullptr && total_q > 0) {
    if (!app->k_new || !app->v_new || !app->write_slots) return HX_E_INVALID_ARG;
    // Write slots index pool rows of n_kv_heads * head_dim contiguous elements (the pool
    // layout of the reference, [pages, page_size, n_kv_heads, head_dim] contiguous); the
    // append kernel and the attention kernels must agree on that row address.
    if (kv_row_stride != (int64_t)n_kv_heads * head_dim || kv_head_stride != head_dim) return HX_E_INVALID_ARG;
    if (page_size > 0 && app->pool_rows != (int64_t)num_pages * page_size) return HX_E_INVALID_ARG;
    if ((uintptr_t)app->k_new % 16 || (uintptr_t)app->v_new % 16 || app->kn_row % 8 ||
        app->kn_head % 8 || app->vn_row % 8 || app->vn_head % 8 || app->kn_row < 0 ||
        app->kn_head < 0 || app->vn_row < 0 || app->vn_head < 0 || app->pool_rows < 0)
      return HX_E_INVALID_ARG;
    // Chunk rows (and every row of generic_kernel) read their own new keys from the
    // pool. When the tick may hold chunk rows and a decode launch runs on the tuned path,
    // workgroups added to that launch write every row (the chunk kernel runs after it,
    // also in a later call); a decode-only tick's rows are written by their own decode
    // workgroups; otherwise (chunk rows run, the generic kernel runs, or this call
    // launches neither decode nor chunk work) every row is appended first, so that a
    // call given new rows always writes them.
    const bool append_in_decode = tuned && max_q >= 2 && a.grid_dec > 0;
    if (append_in_decode) {
      const int64_t wgs = ((int64_t)total_q * n_kv_heads * (head_dim / 8) + kThreads - 1) / kThreads;
      a.app_wgs = (int32_t)(wgs < kAppendWGs ? wgs : kAppendWGs);
    } else if (a.grid_pf > 0 || !tuned || a.grid_dec == 0) {
      const int elem = 2;
      const int st2 = hx_kv_append(const_cast<void*>(k_cache), const_cast<void*>(v_cache), app->pool_rows,
                                   app->k_new, app->kn_row, app->kn_head, app->v_new, app->vn_row,
                                   app->vn_head, app->write_slots, total_q, n_kv_heads, head_dim, elem,
                                   stream);
      if (st2 != HX_OK) return st2;
    }
    if (tuned) {
      a.k_new = static_cast<const uint8_t*>(app->k_new);
      a.v_new = static_cast<const uint8_t*>(app->v_new);
      a.write_slots = app->write_slots;
      a.kn_row = app->kn_row;
      a.kn_head = app->kn_head;
      a.vn_row = app->vn_row;
      a.vn_head = app->vn_head;
      a.pool_rows = app->pool_rows;
    }
  }
  if (!tuned) {
    // One kernel covers every row; a call whose hints launch neither decode nor chunk
    // work (the combine-only phase of a split run) launches nothing.
    if (decode_items_hint == 0 && prefill_items_hint == 0) return HX_OK;
    const GenericShape gs = generic_shape(max_q, G, head_dim);
    if (dtype == HX_DTYPE_BF16) return launch_generic<__bf16>(a, gs, s);
    return launch_generic<_Float16>(a, gs, s);
  }
  const RunArgs* side = has_side_pf ? &side_pf : nullptr;
  if (dtype == HX_DTYPE_BF16) return launch_run_g<__bf16>(a, side, G, s);
  return launch_run_g<_Float16>(a, side, G, s);
}

}  // namespace

extern "C" {

int hx_varlen_attn_run(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const void* k_cache, const void* v_cache,
                       int64_t kv_row_stride, int64_t kv_head_stride,
                       int32_t num_pages, int32_t page_size,
                       const int32_t* block_table, int32_t block_table_stride,
                       int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                       int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                       float scale, int32_t window_left, int32_t window_right,
                       int32_t dtype,
                       void* out, int64_t o_row_stride, int64_t o_head_stride,
                       float* lse,
                       int32_t decode_items_hint, int32_t prefill_items_hint,
                       int32_t combine_seqs_hint,
                       void* workspace, size_t workspace_bytes, void* stream) {
  return run_impl(q, q_row_stride, q_head_stride, nullptr, 0, k_cache, v_cache, kv_row_stride, kv_head_stride,
                  num_pages, page_size, block_table, block_table_stride, batch, total_q, max_q,
                  max_k, n_q_heads, n_kv_heads, head_dim, scale, window_left, window_right, dtype,
                  out, o_row_stride, o_head_stride, lse, decode_items_hint, prefill_items_hint,
                  combine_seqs_hint, workspace, workspace_bytes, stream, nullptr);
}

int hx_varlen_attn_run_rows(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                            const int64_t* query_rows, int64_t query_rows_total,
                            const void* k_cache, const void* v_cache,
                            int64_t kv_row_stride, int64_t kv_head_stride,
                            int32_t num_pages, int32_t page_size,
                            const int32_t* block_table, int32_t block_table_stride,
                            int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                            float scale, int32_t window_left, int32_t window_right,
                            int32_t dtype,
                            void* out, int64_t o_row_stride, int64_t o_head_stride,
                            float* lse,
                            int32_t decode_items_hint, int32_t prefill_items_hint,
                            int32_t combine_seqs_hint,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (total_q > 0 && batch > 0 && (!query_rows || query_rows_total < 1)) return HX_E_INVALID_ARG;
  return run_impl(q, q_row_stride, q_head_stride, query_rows, query_rows_total, k_cache, v_cache,
                  kv_row_stride, kv_head_stride, num_pages, page_size, block_table,
                  block_table_stride, batch, total_q, max_q, max_k, n_q_heads, n_kv_heads, head_dim,
                  scale, window_left, window_right, dtype, out, o_row_stride, o_head_stride, lse,
                  decode_items_hint, prefill_items_hint, combine_seqs_hint, workspace,
                  workspace_bytes, stream, nullptr);
}

int hx_varlen_attn_run_merged(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              const void* k_cache, const void* v_cache,
                              int64_t kv_row_stride, int64_t kv_head_stride,
                              int32_t num_pages, int32_t page_size,
                              const int32_t* block_table, int32_t block_table_stride,
                              int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                              int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                              float scale, int32_t window_left, int32_t window_right,
                              int32_t dtype,
                              void* out, int64_t o_row_stride, int64_t o_head_stride,
                              float* lse,
                              const void* level_out, int64_t level_row_stride, int64_t level_head_stride,
                              const float* level_lse, int64_t level_rows,
                              const int32_t* member_seq, const int32_t* member_of_seq, int32_t n_members,
                              const int32_t* part_start, const int32_t* part_idx, int32_t n_parts,
                              int32_t decode_items_hint, int32_t prefill_items_hint,
                              int32_t combine_seqs_hint,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (n_members < 0) return HX_E_INVALID_ARG;
  MergeSpec mg;
  mg.level_out = level_out;
  mg.level_row = level_row_stride;
  mg.level_head = level_head_stride;
  mg.level_lse = level_lse;
  mg.level_rows = level_rows;
  mg.member_seq = member_seq;
  mg.member_of_seq = member_of_seq;
  mg.n_members = n_members;
  mg.part_start = part_start;
  mg.part_idx = part_idx;
  mg.n_parts = n_parts;
  mg.level_ws = nullptr;
  mg.level_ws_bytes = 0;
  mg.level_batch = mg.level_max_q = mg.level_max_k = mg.level_comb_hint = 0;
  mg.level_bt = nullptr;
  mg.level_bt_stride = 0;
  mg.level_q_rows = nullptr;
  mg.level_q_rows_total = 0;
  mg.level_pf_hint = 0;
  mg.level_win_left = mg.level_win_right = -1;
  return run_impl(q, q_row_stride, q_head_stride, nullptr, 0, k_cache, v_cache, kv_row_stride,
                  kv_head_stride, num_pages, page_size, block_table, block_table_stride, batch,
                  total_q, max_q, max_k, n_q_heads, n_kv_heads, head_dim, scale, window_left,
                  window_right, dtype, out, o_row_stride, o_head_stride, lse, decode_items_hint,
                  prefill_items_hint, combine_seqs_hint, workspace, workspace_bytes, stream, nullptr, &mg);
}

int hx_varlen_attn_run_cascade(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache,
                               int64_t kv_row_stride, int64_t kv_head_stride,
                               int32_t num_pages, int32_t page_size,
                               const int32_t* block_table, int32_t block_table_stride,
                               int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                               int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                               float scale, int32_t window_left, int32_t window_right,
                               int32_t dtype,
                               void* out, int64_t o_row_stride, int64_t o_head_stride,
                               float* lse,
                               void* level_out, int64_t level_row_stride, int64_t level_head_stride,
                               float* level_lse, int64_t level_rows,
                               int32_t level_batch, int32_t level_max_q, int32_t level_max_k,
                               int32_t level_combine_hint, void* level_workspace, size_t level_workspace_bytes,
                               const int32_t* level_block_table, int32_t level_block_table_stride,
                               const int64_t* level_query_rows, int64_t level_query_rows_total,
                               int32_t level_prefill_hint, int32_t level_window_left, int32_t level_window_right,
                               const int32_t* member_seq, const int32_t* member_of_seq, int32_t n_members,
                               const int32_t* part_start, const int32_t* part_idx, int32_t n_parts,
                               int32_t decode_items_hint, int32_t prefill_items_hint,
                               int32_t combine_seqs_hint,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (n_members < 0 || !level_workspace) return HX_E_INVALID_ARG;
  MergeSpec mg;
  mg.level_out = level_out;
  mg.level_row = level_row_stride;
  mg.level_head = level_head_stride;
  mg.level_lse = level_lse;
  mg.level_rows = level_rows;
  mg.member_seq = member_seq;
  mg.member_of_seq = member_of_seq;
  mg.n_members = n_members;
  mg.part_start = part_start;
  mg.part_idx = part_idx;
  mg.n_parts = n_parts;
  mg.level_ws = level_workspace;
  mg.level_ws_bytes = level_workspace_bytes;
  mg.level_batch = level_batch;
  mg.level_max_q = level_max_q;
  mg.level_max_k = level_max_k;
  mg.level_comb_hint = level_combine_hint;
  mg.level_bt = level_block_table;
  mg.level_bt_stride = level_block_table_stride;
  mg.level_q_rows = level_query_rows;
  mg.level_q_rows_total = level_query_rows_total;
  mg.level_pf_hint = level_prefill_hint;
  mg.level_win_left = level_window_left;
  mg.level_win_right = level_window_right;
  return run_impl(q, q_row_stride, q_head_stride, nullptr, 0, k_cache, v_cache, kv_row_stride,
                  kv_head_stride, num_pages, page_size, block_table, block_table_stride, batch,
                  total_q, max_q, max_k, n_q_heads, n_kv_heads, head_dim, scale, window_left,
                  window_right, dtype, out, o_row_stride, o_head_stride, lse, decode_items_hint,
                  prefill_items_hint, combine_seqs_hint, workspace, workspace_bytes, stream, nullptr, &mg);
}

int hx_varlen_attn_append_run(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              void* k_cache, void* v_cache,
                              int64_t kv_row_stride, int64_t kv_head_stride,
                              int32_t num_pages, int32_t page_size,
                              const int32_t* block_table, int32_t block_table_stride,
                              int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                              int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                              float scale, int32_t window_left, int32_t window_right,
                              int32_t dtype,
                              void* out, int64_t o_row_stride, int64_t o_head_stride,
                              float* lse,
                              const void* k_new, int64_t k_new_row_stride, int64_t k_new_head_stride,
                              const void* v_new, int64_t v_new_row_stride, int64_t v_new_head_stride,
                              const int64_t* write_slots, int64_t pool_rows,
                              int32_t decode_items_hint, int32_t prefill_items_hint,
                              int32_t combine_seqs_hint,
                              void* workspace, size_t workspace_bytes, void* stream) {
  AppendSpec app;
  app.k_new = k_new;
  app.v_new = v_new;
  app.kn_row = k_new_row_stride;
  app.kn_head = k_new_head_stride;
  app.vn_row = v_new_row_stride;
  app.vn_head = v_new_head_stride;
  app.write_slots = write_slots;
  app.pool_rows = pool_rows;
  return run_impl(q, q_row_stride, q_head_stride, nullptr, 0, k_cache, v_cache, kv_row_stride, kv_head_stride,
                  num_pages, page_size, block_table, block_table_stride, batch, total_q, max_q,
                  max_k, n_q_heads, n_kv_heads, head_dim, scale, window_left, window_right, dtype,
                  out, o_row_stride, o_head_stride, lse, decode_items_hint, prefill_items_hint,
                  combine_seqs_hint, workspace, workspace_bytes, stream, &app);
}

int hx_varlen_attn(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                   const void* k_cache, const void* v_cache,
                   int64_t kv_row_stride, int64_t kv_head_stride,
                   int32_t num_pages, int32_t page_size,
                   const int32_t* block_table, int32_t block_table_stride,
                   const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                   const int32_t* seqused_k,
                   int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                   int64_t total_k_rows,
                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                   float scale, int32_t window_left, int32_t window_right,
                   int32_t dtype,
                   void* out, int64_t o_row_stride, int64_t o_head_stride,
                   float* lse,
                   void* workspace, size_t workspace_bytes, void* stream) {
  int st = hx_varlen_attn_plan(cu_seq_q, cu_seq_k, seqused_k, batch, total_q, max_q, max_k,
                               total_k_rows, page_size, block_table_stride, n_q_heads, n_kv_heads,
                               head_dim, window_left, window_right, workspace, workspace_bytes, stream);
  if (st != HX_OK) return st;
  return hx_varlen_attn_run(q, q_row_stride, q_head_stride, k_cache, v_cache, kv_row_stride,
                            kv_head_stride, num_pages, page_size, block_table, block_table_stride,
                            batch, total_q, max_q, max_k, n_q_heads, n_kv_heads, head_dim, scale,
                            window_left, window_right, dtype, out, o_row_stride, o_head_stride, lse,
                            -1, -1, -1, workspace, workspace_bytes, stream);
}

}  // extern "C"

// ------------------------------------------------------------------ no-allocation entry
// Workspace of hx_varlen_attn_noalloc: one array per GPU in the library's device memory,
// allocated with the code object when the library loads on that GPU and held until the
// process ends. Host code never passes `scratch` itself to a kernel (on the host it is
// only a stand-in for the symbol): it uses the device address hipGetSymbolAddress gives
// for the current GPU, looked up once per GPU and kept in g_scratch_ptr.
static constexpr size_t kNoallocScratchBytes = HX_NOALLOC_SCRATCH_BYTES;  // 128 MiB
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current GPU's scratch array (resolved at this GPU's first call).
int current_device_scratch(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hx::status_from_hip(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return HX_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hx::status_from_hip(e);
    if (p == nullptr || reinterpret_cast<uintptr_t>(p) % 256 != 0) return HX_E_WORKSPACE;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return HX_OK;
}

}  // namespace

extern "C" {

int hx_varlen_attn_noalloc(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache,
                           int64_t kv_row_stride, int64_t kv_head_stride,
                           int32_t num_pages, int32_t page_size,
                           const int32_t* block_table, int32_t block_table_stride,
                           const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                           const int32_t* seqused_k,
                           int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                           int64_t total_k_rows,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           float scale, int32_t window_left, int32_t window_right,
                           int32_t dtype,
                           void* out, int64_t o_row_stride, int64_t o_head_stride,
                           float* lse, void* stream) {
  const int st = check_shape(batch, max_q, max_k, n_q_heads, n_kv_heads, head_dim);
  if (st != HX_OK) return st;
  // The plan and the split partials of this call must fit the scratch array.
  if (make_layout(batch, max_q, max_k, n_q_heads, n_kv_heads).total > kNoallocScratchBytes)
    return HX_E_TOO_LARGE;
  void* ws = nullptr;
  const int sst = current_device_scratch(&ws);
  if (sst != HX_OK) return sst;
  // Every word the run kernels read is written by the plan kernel of this call first
  // (stream order), so nothing left in the array by an earlier call needs clearing.
  return hx_varlen_attn(q, q_row_stride, q_head_stride, k_cache, v_cache, kv_row_stride,
                        kv_head_stride, num_pages, page_size, block_table, block_table_stride,
                        cu_seq_q, cu_seq_k, seqused_k, batch, total_q, max_q, max_k, total_k_rows,
                        n_q_heads, n_kv_heads, head_dim, scale, window_left, window_right, dtype,
                        out, o_row_stride, o_head_stride, lse, ws, kNoallocScratchBytes, stream);
}

}  // extern "C"
