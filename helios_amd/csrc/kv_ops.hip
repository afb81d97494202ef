// KV append, page copy and page gather for the paged KV pool (gfx950).
//
// All three are bit copies bound by HBM bandwidth. Each thread moves whole
// 16-byte words where the sizes and alignments allow it (narrower words
// otherwise), so a wavefront reads and writes full 128-byte lines.

#include "hx_common.h"

namespace {

// ---------------------------------------------------------------- KV append
// Reference: PagedBatchCache._write (src/helios/runtime/qwen3/paged_cache.py:335-345),
// two index_copy_ calls along dim 0 of pool.view(-1, n_kv_heads, head_dim).
struct AppendArgs {
  uint8_t* k_pool;
  uint8_t* v_pool;
  const uint8_t* k;
  const uint8_t* v;
  const int64_t* slots;
  int64_t pool_rows;
  int64_t n_tokens;
  int64_t k_row_b, k_head_b, v_row_b, v_head_b;  // byte strides of the new rows
  int32_t n_kv;
  int32_t head_b;   // bytes of one head row (head_dim * elem_bytes)
  int32_t words;    // words of type W per head row
  int32_t n_wg;     // workgroups of the launch (the grid stride is n_wg * 256 threads)
  int32_t lw, lh;   // log2 of words and n_kv (the shift form only)
};

// Each thread moves one word of one head row. The slot, K and V loads of an iteration
// are all issued before the slot is tested (the new rows are always in range), so the
// iteration waits for memory once before its stores, not twice. SHIFT is the form for
// head rows of 2^lw words and 2^lh KV heads with every index and source offset below
// 2^31: the thread index splits by shifts and masks in 32-bit arithmetic.
template <typename W, bool SHIFT>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  const int64_t per_token = (int64_t)a.n_kv * a.words;
  const int64_t total = a.n_tokens * per_token;
  const int64_t pool_row_b = (int64_t)a.n_kv * a.head_b;
  for (int64_t idx = (int64_t)hx::wg_x() * 256 + hx::tid_x(); idx < total; idx += (int64_t)a.n_wg * 256) {
    int64_t t;
    int h, w;
    const uint8_t* ks;
    const uint8_t* vs;
    if constexpr (SHIFT) {
      const int i = (int)idx;
      w = i & ((1 << a.lw) - 1);
      h = (i >> a.lw) & ((1 << a.lh) - 1);
      const int ti = i >> (a.lw + a.lh);
      t = ti;
      ks = a.k + (uint32_t)(ti * (int)a.k_row_b + h * (int)a.k_head_b);
      vs = a.v + (uint32_t)(ti * (int)a.v_row_b + h * (int)a.v_head_b);
    } else {
      t = idx / per_token;
      const int rem = (int)(idx - t * per_token);
      h = rem / a.words;
      w = rem - h * a.words;
      ks = a.k + t * a.k_row_b + h * a.k_head_b;
      vs = a.v + t * a.v_row_b + h * a.v_head_b;
    }
    const int64_t slot = a.slots[t];
    const W kw = reinterpret_cast<const W*>(ks)[w];
    const W vw = reinterpret_cast<const W*>(vs)[w];
    hx::hold(kw);
    hx::hold(vw);
    if (slot < 0 || slot >= a.pool_rows) continue;
    const int64_t dst = slot * pool_row_b + (int64_t)h * a.head_b;
    if constexpr (sizeof(W) == 16) {
      // Non-temporal stores: the rows are read back by a later launch, and streamed
      // stores finish the launch sooner (2048 rows: 3.4-3.6 -> 3.0-3.1 us).
      hx::st16_nt(reinterpret_cast<W*>(a.k_pool + dst) + w, __builtin_bit_cast(uint4, kw));
      hx::st16_nt(reinterpret_cast<W*>(a.v_pool + dst) + w, __builtin_bit_cast(uint4, vw));
    } else {
      reinterpret_cast<W*>(a.k_pool + dst)[w] = kw;
      reinterpret_cast<W*>(a.v_pool + dst)[w] = vw;
    }
  }
}

// Largest word (16, 8, 4 or 2 bytes) dividing every size and address involved.
int word_bytes_for(std::initializer_list<uint64_t> values) {
  for (int w = 16; w >= 2; w >>= 1) {
    bool ok = true;
    for (uint64_t v : values) ok = ok && (v % (uint64_t)w == 0);
    if (ok) return w;
  }
  return 1;
}

// ---------------------------------------------------------------- page copy
// Reference semantics: KVCache.snapshot_block / restore_blocks
// (src/helios/runtime/qwen3/cache.py:109-147): a bit-exact copy of a token block
// for every layer, keys and values. Here the block is a set of whole pages.
constexpr int kCopyMaxTensors = 64;   // K and V tensors per launch (32 layers)
constexpr int kCopyMaxPages = 64;     // page pairs per launch
constexpr int kCopyThreads = 256;
constexpr int kCopyDepth = 4;         // 16-byte words in flight per thread per tile
constexpr int kCopyTileBytes = kCopyThreads * kCopyDepth * 16;  // 16 KiB
constexpr int kCopyMaxGrid = 8192;

struct CopyArgs {
  uint8_t* tensors[kCopyMaxTensors];
  int32_t src[kCopyMaxPages];
  int32_t dst[kCopyMaxPages];
  int64_t page_bytes;
  int32_t n_tensors;
  int32_t n_pages;
  int32_t tiles_per_page;
  int32_t n_wg;  // workgroups of the launch (the grid stride in tiles)
  // Strided form (strided != 0): tensor t is layer t / per_layer's K (t % per_layer == 0)
  // or V pool, at k0 / v0 + layer * layer_bytes; `tensors` is unused and n_tensors has
  // no limit.
  uint8_t* k0;
  uint8_t* v0;
  int64_t layer_bytes;
  int32_t per_layer;
  int32_t strided;
};

// Grid-stride over 16 KiB tiles of (tensor, page pair): each thread streams four
// 16-byte words with non-temporal loads and stores per tile. A steady stream of
// moderately deep tiles copies at ~5.7 TB/s on MI355X; one deep burst per workgroup
// (the first form of this kernel) reached only ~2.6 TB/s.
__global__ __launch_bounds__(kCopyThreads) void kv_copy_pages_kernel(CopyArgs a) {
  const int64_t total = (int64_t)a.n_tensors * a.n_pages * a.tiles_per_page;
  for (int64_t t = hx::wg_x(); t < total; t += a.n_wg) {
    const int tile = (int)(t % a.tiles_per_page);
    const int64_t rest = t / a.tiles_per_page;
    const int pair = (int)(rest % a.n_pages);
    const int tensor = (int)(rest / a.n_pages);
    uint8_t* base = a.strided ? (tensor % a.per_layer == 0 ? a.k0 : a.v0) + (int64_t)(tensor / a.per_layer) * a.layer_bytes
                              : a.tensors[tensor];
    const uint8_t* src = base + (int64_t)a.src[pair] * a.page_bytes;
    uint8_t* dst = base + (int64_t)a.dst[pair] * a.page_bytes;
    const int64_t t0 = (int64_t)tile * kCopyTileBytes;
    hx::u32x4_t buf[kCopyDepth];
#pragma unroll
    for (int i = 0; i < kCopyDepth; ++i) {
      const int64_t off = t0 + ((int64_t)i * kCopyThreads + hx::tid_x()) * 16;
      buf[i] = off < a.page_bytes
                   ? __builtin_nontemporal_load(reinterpret_cast<const hx::u32x4_t*>(src + off))
                   : hx::u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < kCopyDepth; ++i) {
      const int64_t off = t0 + ((int64_t)i * kCopyThreads + hx::tid_x()) * 16;
      if (off < a.page_bytes) __builtin_nontemporal_store(buf[i], reinterpret_cast<hx::u32x4_t*>(dst + off));
    }
  }
}

// ---------------------------------------------------------------- page gather
// Reference: _gather_cpu (src/helios/runtime/qwen3/paged_cache.py:405-414).
struct GatherArgs {
  const uint8_t* pool;
  const int32_t* pages;
  uint8_t* out;
  int64_t length;
  int32_t num_pool_pages;
  int32_t page_size;
  int32_t n_kv;
  int32_t head_b;
  int32_t words;
  int32_t n_wg;  // workgroups of the element-wise launch (its grid stride is n_wg * 256)
};

template <typename W>
__global__ __launch_bounds__(256) void kv_gather_kernel(GatherArgs a) {
  const int64_t per_head = a.length * a.words;
  const int64_t total = (int64_t)a.n_kv * per_head;
  for (int64_t idx = (int64_t)hx::wg_x() * 256 + hx::tid_x(); idx < total; idx += (int64_t)a.n_wg * 256) {
    const int h = (int)(idx / per_head);
    const int64_t rem = idx - (int64_t)h * per_head;
    const int64_t j = rem / a.words;
    const int w = (int)(rem - j * a.words);
    const int32_t page = a.pages[j / a.page_size];
    W value;
    if (page >= 0 && page < a.num_pool_pages) {
      const int64_t row = (int64_t)page * a.page_size + j % a.page_size;
      value = reinterpret_cast<const W*>(a.pool + (row * a.n_kv + h) * a.head_b)[w];
    } else {
      value = W{};
    }
    reinterpret_cast<W*>(a.out + idx / a.words * a.head_b)[w] = value;
  }
}

// The common case: 16-byte aligned head rows, a power-of-two number of 16-byte words per
// token row (RW = n_kv * head_b / 16) and per head row (HW), and pages holding a multiple
// of 32 tokens. Workgroup x copies tokens [32x, 32x + 32), which share one page (one
// page-id load); thread t moves words t + 256 i of that block, so every wave reads
// contiguous token rows (all heads) and writes whole 256-byte head pieces. Index math
// is shifts and masks.
constexpr int kGatherRows = 32;

template <int RW, int HW>
__global__ __launch_bounds__(256) void kv_gather_rows_kernel(GatherArgs a) {
  const int64_t tok0 = (int64_t)hx::wg_x() * kGatherRows;
  const int rows = (int)min((int64_t)kGatherRows, a.length - tok0);
  const int32_t page = a.pages[tok0 / a.page_size];
  const bool ok = page >= 0 && page < a.num_pool_pages;
  const int64_t row0 = (int64_t)(ok ? page : 0) * a.page_size + tok0 % a.page_size;
  const hx::u32x4_t* src = reinterpret_cast<const hx::u32x4_t*>(a.pool) + row0 * RW;
  hx::u32x4_t* out = reinterpret_cast<hx::u32x4_t*>(a.out);
  constexpr int kPer = kGatherRows * RW / 256;  // words per thread, all loaded before any store
  hx::u32x4_t v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int q = hx::tid_x() + 256 * i;
    v[i] = (ok && q / RW < rows) ? __builtin_nontemporal_load(src + q) : hx::u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int q = hx::tid_x() + 256 * i;
    const int jr = q / RW, wr = q & (RW - 1);
    if (jr < rows)
      __builtin_nontemporal_store(v[i], out + ((int64_t)(wr / HW) * a.length + tok0 + jr) * HW + (wr & (HW - 1)));
  }
}

int grid_for(int64_t items, int threads) {
  int64_t blocks = (items + threads - 1) / threads;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  return (int)blocks;
}

}  // namespace

extern "C" {

const char* hx_strerror(int code) {
  switch (code) {
    case HX_OK: return "success";
    case HX_E_INVALID_ARG: return "invalid argument";
    case HX_E_UNSUPPORTED: return "unsupported head_dim, group size or dtype";
    case HX_E_WORKSPACE: return "workspace missing, misaligned or too small";
    case HX_E_OVERLAP: return "page copy sources and destinations overlap";
    case HX_E_TOO_LARGE: return "the call needs more workspace than the no-allocation scratch holds";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown helios_paged status";
}

int hx_abi_version(void) { return 6; }

int hx_kv_append(void* k_pool, void* v_pool, int64_t pool_rows,
                 const void* k_new, int64_t k_row_stride, int64_t k_head_stride,
                 const void* v_new, int64_t v_row_stride, int64_t v_head_stride,
                 const int64_t* write_slots, int64_t n_tokens,
                 int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                 void* stream) {
  if (n_tokens < 0 || pool_rows < 0 || n_kv_heads < 1 || head_dim < 1) return HX_E_INVALID_ARG;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return HX_E_INVALID_ARG;
  if (n_tokens == 0) return HX_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !write_slots) return HX_E_INVALID_ARG;
  AppendArgs a;
  a.k_pool = static_cast<uint8_t*>(k_pool);
  a.v_pool = static_cast<uint8_t*>(v_pool);
  a.k = static_cast<const uint8_t*>(k_new);
  a.v = static_cast<const uint8_t*>(v_new);
  a.slots = write_slots;
  a.pool_rows = pool_rows;
  a.n_tokens = n_tokens;
  a.k_row_b = k_row_stride * elem_bytes;
  a.k_head_b = k_head_stride * elem_bytes;
  a.v_row_b = v_row_stride * elem_bytes;
  a.v_head_b = v_head_stride * elem_bytes;
  a.n_kv = n_kv_heads;
  a.head_b = head_dim * elem_bytes;
  const int wb = word_bytes_for({(uint64_t)a.head_b, (uint64_t)a.k_row_b, (uint64_t)a.k_head_b,
                                 (uint64_t)a.v_row_b, (uint64_t)a.v_head_b,
                                 (uint64_t)(uintptr_t)k_pool, (uint64_t)(uintptr_t)v_pool,
                                 (uint64_t)(uintptr_t)k_new, (uint64_t)(uintptr_t)v_new});
  a.words = a.head_b / wb;
  const int64_t items = n_tokens * n_kv_heads * (int64_t)a.words;
  const int grid = grid_for(items, 256);
  a.n_wg = grid;
  a.lw = 0;
  a.lh = 0;
  while ((1 << a.lw) < a.words) ++a.lw;
  while ((1 << a.lh) < n_kv_heads) ++a.lh;
  const int64_t lim = (int64_t)1 << 31;
  auto fits = [&](int64_t row_b, int64_t head_b) {
    return row_b >= 0 && head_b >= 0 && n_tokens * row_b + (int64_t)n_kv_heads * head_b < lim;
  };
  const bool shift = (1 << a.lw) == a.words && (1 << a.lh) == n_kv_heads && items + (int64_t)grid * 256 < lim &&
                     fits(a.k_row_b, a.k_head_b) && fits(a.v_row_b, a.v_head_b);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (wb) {
    case 16:
      if (shift) hipLaunchKernelGGL((kv_append_kernel<uint4, true>), dim3(grid), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((kv_append_kernel<uint4, false>), dim3(grid), dim3(256), 0, s, a);
      break;
    case 8: hipLaunchKernelGGL((kv_append_kernel<uint2, false>), dim3(grid), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((kv_append_kernel<uint32_t, false>), dim3(grid), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kv_append_kernel<uint16_t, false>), dim3(grid), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((kv_append_kernel<uint8_t, false>), dim3(grid), dim3(256), 0, s, a); break;
  }
  return hx::status_from_hip(hipGetLastError());
}

int hx_kv_copy_pages(void* const* k_pools, void* const* v_pools, int32_t n_layers,
                     const int32_t* src_pages, const int32_t* dst_pages, int32_t n_pages,
                     int32_t num_pool_pages, int64_t page_bytes, void* stream) {
  if (n_layers < 0 || n_pages < 0 || num_pool_pages < 1 || page_bytes < 16 || page_bytes % 16)
    return HX_E_INVALID_ARG;
  if (n_layers == 0 || n_pages == 0) return HX_OK;
  if (!k_pools || !src_pages || !dst_pages) return HX_E_INVALID_ARG;
  for (int i = 0; i < n_pages; ++i) {
    if (src_pages[i] < 0 || src_pages[i] >= num_pool_pages) return HX_E_INVALID_ARG;
    if (dst_pages[i] < 0 || dst_pages[i] >= num_pool_pages) return HX_E_INVALID_ARG;
  }
  for (int i = 0; i < n_pages; ++i)
    for (int j = 0; j < n_pages; ++j) {
      if (j > i && dst_pages[i] == dst_pages[j]) return HX_E_OVERLAP;
      if (dst_pages[i] == src_pages[j]) return HX_E_OVERLAP;
    }
  const int per_layer = v_pools ? 2 : 1;
  for (int l = 0; l < n_layers; ++l) {
    if (!k_pools[l] || (v_pools && !v_pools[l])) return HX_E_INVALID_ARG;
    if ((uintptr_t)k_pools[l] % 16 || (v_pools && (uintptr_t)v_pools[l] % 16)) return HX_E_INVALID_ARG;
  }
  const int tiles = (int)((page_bytes + kCopyTileBytes - 1) / kCopyTileBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int total_tensors = n_layers * per_layer;
  // Pools of one allocation (every layer's K, and V, at one stride from the first, as a
  // [2, layers, pages, ...] store lays them out) go in one launch whatever the layer
  // count; other pointer lists go kCopyMaxTensors tensors per launch.
  int64_t layer_bytes = 0;
  bool strided = n_layers >= 2;
  if (strided) {
    layer_bytes = static_cast<uint8_t*>(k_pools[1]) - static_cast<uint8_t*>(k_pools[0]);
    for (int l = 1; l < n_layers && strided; ++l) {
      strided = static_cast<uint8_t*>(k_pools[l]) - static_cast<uint8_t*>(k_pools[0]) == (int64_t)l * layer_bytes &&
                (!v_pools || static_cast<uint8_t*>(v_pools[l]) - static_cast<uint8_t*>(v_pools[0]) == (int64_t)l * layer_bytes);
    }
  }
  const int per_launch = strided ? total_tensors : kCopyMaxTensors;
  for (int t0 = 0; t0 < total_tensors; t0 += per_launch) {
    const int nt = total_tensors - t0 < per_launch ? total_tensors - t0 : per_launch;
    for (int p0 = 0; p0 < n_pages; p0 += kCopyMaxPages) {
      const int np = n_pages - p0 < kCopyMaxPages ? n_pages - p0 : kCopyMaxPages;
      CopyArgs a;
      a.strided = strided ? 1 : 0;
      a.per_layer = per_layer;
      a.k0 = static_cast<uint8_t*>(k_pools[0]);
      a.v0 = v_pools ? static_cast<uint8_t*>(v_pools[0]) : nullptr;
      a.layer_bytes = layer_bytes;
      if (!strided) {
        for (int t = 0; t < nt; ++t) {
          const int flat = t0 + t;
          const int layer = flat / per_layer;
          a.tensors[t] = static_cast<uint8_t*>((flat % per_layer == 0) ? k_pools[layer] : v_pools[layer]);
        }
      }
      for (int p = 0; p < np; ++p) {
        a.src[p] = src_pages[p0 + p];
        a.dst[p] = dst_pages[p0 + p];
      }
      a.page_bytes = page_bytes;
      a.n_tensors = nt;
      a.n_pages = np;
      a.tiles_per_page = tiles;
      int64_t grid = (int64_t)nt * np * tiles;
      if (grid > kCopyMaxGrid) grid = kCopyMaxGrid;
      a.n_wg = (int32_t)grid;
      hipLaunchKernelGGL(kv_copy_pages_kernel, dim3((unsigned)grid), dim3(kCopyThreads), 0, s, a);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return (int)e;
    }
  }
  return HX_OK;
}

int hx_kv_gather(const void* pool, int32_t num_pool_pages, int32_t page_size,
                 int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                 const int32_t* pages, int32_t n_pages, int64_t length,
                 void* out, void* stream) {
  if (num_pool_pages < 1 || page_size < 1 || n_kv_heads < 1 || head_dim < 1 || n_pages < 0 ||
      length < 0)
    return HX_E_INVALID_ARG;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return HX_E_INVALID_ARG;
  if (length > (int64_t)n_pages * page_size) return HX_E_INVALID_ARG;
  if (length == 0) return HX_OK;
  if (!pool || !pages || !out) return HX_E_INVALID_ARG;
  GatherArgs a;
  a.pool = static_cast<const uint8_t*>(pool);
  a.pages = pages;
  a.out = static_cast<uint8_t*>(out);
  a.length = length;
  a.num_pool_pages = num_pool_pages;
  a.page_size = page_size;
  a.n_kv = n_kv_heads;
  a.head_b = head_dim * elem_bytes;
  const int wb = word_bytes_for({(uint64_t)a.head_b, (uint64_t)(uintptr_t)pool, (uint64_t)(uintptr_t)out});
  a.words = a.head_b / wb;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (wb == 16 && page_size % kGatherRows == 0 && length / kGatherRows < 0x7fffffff) {
    const int rw = n_kv_heads * a.head_b / 16, hw = a.head_b / 16;
    const unsigned blocks = (unsigned)((length + kGatherRows - 1) / kGatherRows);
    bool launched = true;
    if (rw == 128 && hw == 16)
      hipLaunchKernelGGL((kv_gather_rows_kernel<128, 16>), dim3(blocks), dim3(256), 0, s, a);
    else if (rw == 64 && hw == 16)
      hipLaunchKernelGGL((kv_gather_rows_kernel<64, 16>), dim3(blocks), dim3(256), 0, s, a);
    else if (rw == 256 && hw == 16)
      hipLaunchKernelGGL((kv_gather_rows_kernel<256, 16>), dim3(blocks), dim3(256), 0, s, a);
    else
      launched = false;
    if (launched) return hx::status_from_hip(hipGetLastError());
  }
  const int grid = grid_for((int64_t)n_kv_heads * length * a.words, 256);
  a.n_wg = grid;
  switch (wb) {
    case 16: hipLaunchKernelGGL(kv_gather_kernel<uint4>, dim3(grid), dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(kv_gather_kernel<uint2>, dim3(grid), dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(kv_gather_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(kv_gather_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, a); break;
  }
  return hx::status_from_hip(hipGetLastError());
}

}  // extern "C"
