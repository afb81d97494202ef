// Final RMSNorm + lm_head + greedy argmax over the logit rows of a tick (gfx950).
//
// Reference: Qwen3Model.forward_packed ends with x.index_select(1, logit_indices), the
// final RMSNorm (layers.py:29-39) cast to the model dtype, and self.output, the tied
// embedding as a bias-free Linear (model.py:108-110), which writes bf16 logits
// [rows, vocab]. The engine then takes heads.argmax(dim=-1) for greedy rows
// (engine.py:470-473) and copies the token ids to the host.
//
// Here three launches produce the token ids and never write the logits to HBM unless
// asked to:
//   1. final_norm_kernel: gather each logit row, RMSNorm it with the reference's op
//      order, round to the model dtype, store [rows_pad, hidden] in the workspace.
//   2. logits_argmax_kernel: one workgroup per 128 vocab rows streams its slice of the
//      embedding once (the 778 MB weight read is the roofline: HBM), stages weight and
//      row chunks in LDS, runs 16x16x32 MFMAs for up to 160 rows, rounds every logit to
//      the model dtype like the Linear's output, and reduces a (value, first index) key
//      per row over its vocab rows.
//   3. argmax_reduce_kernel: per row, the maximum key over the vocab tiles.
// A key orders first by the rounded logit and then by the smaller vocab index, which is
// torch.argmax's rule for ties (the first maximal element).

#include "hx_common.h"

namespace {

constexpr int kLgThreads = 256;
constexpr int kLgVocabTile = 128;            // vocab rows per workgroup: 4 waves x 32
constexpr int kLgKChunk = 128;               // hidden elements per LDS stage
constexpr int kLgRowBytes = kLgKChunk * 2;   // one staged row: 256 B = 16 chunks of 16 B
constexpr int kLgMaxTokenTiles = 10;         // 16-row tiles per launch: 160 logit rows
constexpr int kLgMaxRows = 16 * kLgMaxTokenTiles;

// 16-byte chunk c of staged row r sits at chunk c ^ (r & 15). A fragment read (16 rows,
// one chunk each per 16 lanes) and a row store (one row, 16 chunks per 16 lanes) then
// both touch 16 distinct 16-byte bank groups, i.e. all 64 banks once.
__device__ __forceinline__ int lg_off(int r, int c) { return r * kLgRowBytes + ((c ^ (r & 15)) << 4); }

// Orderable key of a logit and its vocab index: larger value first, then smaller index.
// -0 counts as +0, as torch's comparison does.
__device__ __forceinline__ uint64_t argmax_key(float f, uint32_t idx) {
  if (f == 0.f) f = 0.f;
  const uint32_t b = __float_as_uint(f);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t ord = (uint32_t)(key >> 32);
  return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

// ------------------------------------------------------------------------ final norm
// One workgroup per padded row j. Rows past n (or with an index outside the hidden
// rows) become zeros and row_ok[j] = 0.
template <typename T>
__global__ __launch_bounds__(kLgThreads) void final_norm_kernel(
    const uint16_t* x, int64_t x_row, int64_t total_rows, const int64_t* idx, int64_t n,
    const float* w, float eps, int hidden, uint16_t* xn, int32_t* row_ok) {
  __shared__ float s_part[kLgThreads / 64];
  const int j = hx::wg_x(), tid = hx::tid_x();
  const int nv = hidden >> 3;
  uint4* dst = reinterpret_cast<uint4*>(xn + (int64_t)j * hidden);
  int64_t src = -1;
  if (j < n) {
    const int64_t s = idx[j];
    if (s >= 0 && s < total_rows) src = s;
  }
  if (tid == 0) row_ok[j] = src >= 0 ? 1 : 0;
  if (src < 0) {
    for (int v = tid; v < nv; v += kLgThreads) dst[v] = hx::zero4();
    return;
  }
  const uint4* p = reinterpret_cast<const uint4*>(x + src * x_row);
  // mean(x^2): squares rounded to fp32, then summed (x.pow(2).mean(dim=-1)).
  float ss = 0.f;
  for (int v = tid; v < nv; v += kLgThreads) {
    const uint4 u = p[v];
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float a = hx::Elem<T>::lo(wd[q]), b = hx::Elem<T>::hi(wd[q]);
      ss = __fadd_rn(ss, __fmul_rn(a, a));
      ss = __fadd_rn(ss, __fmul_rn(b, b));
    }
  }
  ss = hx::wave_sum_xor(ss, 1, 32);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  ss = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float r = rsqrtf(__fadd_rn(__fdiv_rn(ss, (float)hidden), eps));
  for (int v = tid; v < nv; v += kLgThreads) {
    const uint4 u = p[v];
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 8 * v + 2 * q;
      const float a = __fmul_rn(__fmul_rn(hx::Elem<T>::lo(wd[q]), r), w[e]);
      const float b = __fmul_rn(__fmul_rn(hx::Elem<T>::hi(wd[q]), r), w[e + 1]);
      o[q] = hx::pack2_round<T>(a, b);
    }
    dst[v] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One chunk's loads into registers: eight 16-byte weight pieces (non-temporal: the
// embedding is streamed once per call) and NT pieces of the normalised rows.
template <int NT>
__device__ __forceinline__ void lg_load(uint4 (&rw)[8], uint4 (&rx)[NT], const uint16_t* emb,
                                        const int64_t (&wrow)[8], const uint16_t* xsrc,
                                        int64_t xstep, int k0) {
#pragma unroll
  for (int i = 0; i < 8; ++i) rw[i] = hx::ld16_stream(emb + wrow[i] + k0);
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const hx::u32x4_t v = *reinterpret_cast<const hx::u32x4_t*>(xsrc + i * xstep + k0);
    rx[i] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// ------------------------------------------------------------------- logits + argmax
// Workgroup g owns vocab rows [128 g, 128 g + 128); wave w of it owns 32 of them as two
// 16-row MFMA tiles, against all NT 16-row tiles of the normalised logit rows. The
// hidden dimension is walked in 128-element chunks: every thread loads its share of the
// next chunk into registers while the MFMAs consume the current one from LDS.
//   weights: load i of a wave covers 4 rows x 256 B (16 lanes per row, coalesced);
//   rows:    load i of the workgroup covers 16 rows x 256 B.
// MFMA operand A is 16 vocab rows x 32 hidden, B is 32 hidden x 16 logit rows; lane l
// holds row (l & 15), hidden elements 8 (l >> 4) .. +7 of each 32-wide step, and its
// accumulator holds vocab rows 4 (l >> 4) .. +3 for logit row (l & 15).
template <typename T, int NT>
__global__ __launch_bounds__(kLgThreads) void logits_argmax_kernel(
    const uint16_t* __restrict__ emb, int64_t ld_emb, int64_t vocab, int hidden,
    const uint16_t* __restrict__ xn, int n, int32_t tiles, uint64_t* __restrict__ partial,
    uint16_t* __restrict__ logits, int64_t ld_logits) {
  __shared__ __attribute__((aligned(16))) unsigned char s_w[kLgVocabTile * kLgRowBytes];
  __shared__ __attribute__((aligned(16))) unsigned char s_x[NT * 16 * kLgRowBytes];
  __shared__ uint64_t s_key[kLgThreads / 64][NT * 16];

  const int tid = hx::tid_x(), lane = tid & 63, wave = tid >> 6;
  const int64_t v0 = (int64_t)hx::wg_x() * kLgVocabTile;

  // Global source of this thread's weight loads: rows past the vocab re-read the last
  // row (their logits are never used).
  int64_t wrow[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = v0 + 32 * wave + 4 * i + (lane >> 4);
    wrow[i] = (row < vocab ? row : vocab - 1) * ld_emb + 8 * (lane & 15);
  }
  const uint16_t* xsrc = xn + (int64_t)(tid >> 4) * hidden + 8 * (tid & 15);

  uint4 rw[8], rx[NT];
  const int64_t xstep = (int64_t)16 * hidden;

  hx::f32x4_t acc[2][NT];
#pragma unroll
  for (int v = 0; v < 2; ++v)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[v][t] = (hx::f32x4_t){0.f, 0.f, 0.f, 0.f};

  const int chunks = hidden / kLgKChunk;
  lg_load<NT>(rw, rx, emb, wrow, xsrc, xstep, 0);
  for (int c = 0; c < chunks; ++c) {
    __syncthreads();  // the previous chunk's fragments have been read
#pragma unroll
    for (int i = 0; i < 8; ++i)
      *reinterpret_cast<uint4*>(s_w + lg_off(32 * wave + 4 * i + (lane >> 4), lane & 15)) = rw[i];
#pragma unroll
    for (int i = 0; i < NT; ++i)
      *reinterpret_cast<uint4*>(s_x + lg_off(16 * i + (tid >> 4), tid & 15)) = rx[i];
    __syncthreads();
    if (c + 1 < chunks) lg_load<NT>(rw, rx, emb, wrow, xsrc, xstep, (c + 1) * kLgKChunk);
#pragma unroll
    for (int s = 0; s < kLgKChunk / 32; ++s) {
      const int ch = 4 * s + (lane >> 4);
      const uint4 a0 = *reinterpret_cast<const uint4*>(s_w + lg_off(32 * wave + (lane & 15), ch));
      const uint4 a1 = *reinterpret_cast<const uint4*>(s_w + lg_off(32 * wave + 16 + (lane & 15), ch));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint4 b = *reinterpret_cast<const uint4*>(s_x + lg_off(16 * t + (lane & 15), ch));
        acc[0][t] = hx::Elem<T>::mfma16x16x32(hx::as_v8<T>(a0), hx::as_v8<T>(b), acc[0][t]);
        acc[1][t] = hx::Elem<T>::mfma16x16x32(hx::as_v8<T>(a1), hx::as_v8<T>(b), acc[1][t]);
      }
    }
  }

  // Round each logit to the model dtype, then reduce keys: over this lane's 8 vocab rows,
  // over the 4 lanes of the same logit row, over the 4 waves.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tok = 16 * t + (lane & 15);
    uint64_t best = 0;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int64_t vr0 = v0 + 32 * wave + 16 * v + 4 * (lane >> 4);
      uint16_t bits[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bits[i] = hx::Elem<T>::bits(acc[v][t][i]);
        const float f = hx::Elem<T>::lo((uint32_t)bits[i]);
        if (vr0 + i < vocab) best = max_u64(best, argmax_key(f, (uint32_t)(vr0 + i)));
      }
      if (logits != nullptr && tok < n) {
        uint16_t* dst = logits + (int64_t)tok * ld_logits + vr0;
        if (vr0 + 3 < vocab && ((reinterpret_cast<uintptr_t>(dst) & 7) == 0)) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(hx::pack2(bits[0], bits[1]), hx::pack2(bits[2], bits[3]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (vr0 + i < vocab) dst[i] = bits[i];
        }
      }
    }
    best = max_u64(best, shfl_xor_u64(best, 16));
    best = max_u64(best, shfl_xor_u64(best, 32));
    if (lane < 16) s_key[wave][16 * t + lane] = best;
  }
  __syncthreads();
  for (int j = tid; j < n; j += kLgThreads) {
    const uint64_t m = max_u64(max_u64(s_key[0][j], s_key[1][j]), max_u64(s_key[2][j], s_key[3][j]));
    partial[(int64_t)j * tiles + hx::wg_x()] = m;
  }
}

// One workgroup per logit row: the maximum key over the vocab tiles.
__global__ __launch_bounds__(kLgThreads) void argmax_reduce_kernel(
    const uint64_t* partial, int32_t tiles, const int32_t* row_ok, int64_t* token_ids,
    float* max_logits) {
  __shared__ uint64_t s_best[kLgThreads / 64];
  const int j = hx::wg_x(), tid = hx::tid_x();
  const uint64_t* p = partial + (int64_t)j * tiles;
  uint64_t best = 0;
  for (int t = tid; t < tiles; t += kLgThreads) best = max_u64(best, p[t]);
  for (int m = 1; m < 64; m <<= 1) best = max_u64(best, shfl_xor_u64(best, m));
  if ((tid & 63) == 0) s_best[tid >> 6] = best;
  __syncthreads();
  if (tid == 0) {
    best = max_u64(max_u64(s_best[0], s_best[1]), max_u64(s_best[2], s_best[3]));
    const bool ok = row_ok[j] != 0 && best != 0;
    token_ids[j] = ok ? (int64_t)(0xFFFFFFFFu - (uint32_t)best) : -1;
    // The quiet-NaN bits, stored as data: device code is built without NaN semantics,
    // under which a NaN literal would be undefined.
    if (max_logits != nullptr) max_logits[j] = ok ? key_value(best) : __uint_as_float(0x7FC00000u);
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct LogitsLayout {
  int rows_pad;
  int tiles;
  size_t xn, ok, partial, total;
};

LogitsLayout logits_layout(int64_t n_rows, int64_t vocab, int32_t hidden) {
  LogitsLayout l;
  const int64_t group = n_rows < kLgMaxRows ? n_rows : kLgMaxRows;
  l.rows_pad = (int)((group + 15) / 16 * 16);
  if (l.rows_pad < 16) l.rows_pad = 16;
  l.tiles = (int)((vocab + kLgVocabTile - 1) / kLgVocabTile);
  l.xn = 0;
  l.ok = align256((size_t)l.rows_pad * hidden * 2);
  l.partial = l.ok + align256((size_t)l.rows_pad * 4);
  l.total = l.partial + align256((size_t)l.rows_pad * l.tiles * 8);
  return l;
}

template <typename T, int NT>
void launch_argmax(int tiles, hipStream_t s, const uint16_t* emb, int64_t ld_emb, int64_t vocab,
                   int hidden, const uint16_t* xn, int n, uint64_t* partial, uint16_t* logits,
                   int64_t ld_logits) {
  hipLaunchKernelGGL((logits_argmax_kernel<T, NT>), dim3(tiles), dim3(kLgThreads), 0, s, emb, ld_emb,
                     vocab, hidden, xn, n, tiles, partial, logits, ld_logits);
}

template <typename T>
void launch_group(int nt, int tiles, hipStream_t s, const uint16_t* emb, int64_t ld_emb,
                  int64_t vocab, int hidden, const uint16_t* xn, int n, uint64_t* partial,
                  uint16_t* logits, int64_t ld_logits) {
  switch (nt) {
#define HX_LG_CASE(K) \
  case K: launch_argmax<T, K>(tiles, s, emb, ld_emb, vocab, hidden, xn, n, partial, logits, ld_logits); break;
    HX_LG_CASE(1) HX_LG_CASE(2) HX_LG_CASE(3) HX_LG_CASE(4) HX_LG_CASE(5)
    HX_LG_CASE(6) HX_LG_CASE(7) HX_LG_CASE(8) HX_LG_CASE(9) HX_LG_CASE(10)
#undef HX_LG_CASE
    default: break;
  }
}

}  // namespace

extern "C" size_t hx_logits_workspace_bytes(int64_t n_rows, int64_t vocab, int32_t hidden) {
  if (n_rows < 0 || vocab < 1 || hidden < 1) return 0;
  return logits_layout(n_rows, vocab, hidden).total;
}

extern "C" int hx_final_norm_logits_argmax(
    const void* hidden_states, int64_t hidden_row_stride, int64_t total_rows,
    const int64_t* logit_indices, int64_t n_rows, const float* norm_weight, float eps,
    const void* embedding, int64_t embedding_row_stride, int64_t vocab, int32_t hidden,
    int32_t dtype, int64_t* token_ids, float* max_logits, void* logits, int64_t logits_row_stride,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype != HX_DTYPE_BF16 && dtype != HX_DTYPE_FP16) return HX_E_UNSUPPORTED;
  if (hidden < kLgKChunk || hidden % kLgKChunk != 0 || hidden > 65536) return HX_E_UNSUPPORTED;
  if (n_rows < 0 || total_rows < 0 || vocab < 1 || vocab > 0x7FFFFFFF) return HX_E_INVALID_ARG;
  if (n_rows == 0) return HX_OK;
  if (!hidden_states || !logit_indices || !norm_weight || !embedding || !token_ids || !workspace)
    return HX_E_INVALID_ARG;
  if (hidden_row_stride < hidden || embedding_row_stride < hidden || hidden_row_stride % 8 != 0 ||
      embedding_row_stride % 8 != 0)
    return HX_E_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(hidden_states) | reinterpret_cast<uintptr_t>(embedding) |
       reinterpret_cast<uintptr_t>(workspace)) & 15)
    return HX_E_INVALID_ARG;
  if (logits != nullptr && logits_row_stride < vocab) return HX_E_INVALID_ARG;
  const LogitsLayout lay = logits_layout(n_rows, vocab, hidden);
  if (workspace_bytes < lay.total) return HX_E_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  uint16_t* xn = reinterpret_cast<uint16_t*>(ws + lay.xn);
  int32_t* ok = reinterpret_cast<int32_t*>(ws + lay.ok);
  uint64_t* partial = reinterpret_cast<uint64_t*>(ws + lay.partial);
  const uint16_t* x = static_cast<const uint16_t*>(hidden_states);
  const uint16_t* emb = static_cast<const uint16_t*>(embedding);
  uint16_t* lg = static_cast<uint16_t*>(logits);
  // Groups of up to 160 rows; each group streams the embedding once.
  for (int64_t r0 = 0; r0 < n_rows; r0 += kLgMaxRows) {
    const int n = (int)(n_rows - r0 < kLgMaxRows ? n_rows - r0 : kLgMaxRows);
    const int pad = (n + 15) / 16 * 16;
    if (dtype == HX_DTYPE_BF16)
      hipLaunchKernelGGL(final_norm_kernel<__bf16>, dim3(pad), dim3(kLgThreads), 0, s, x, hidden_row_stride,
                         total_rows, logit_indices + r0, (int64_t)n, norm_weight, eps, (int)hidden, xn, ok);
    else
      hipLaunchKernelGGL(final_norm_kernel<_Float16>, dim3(pad), dim3(kLgThreads), 0, s, x, hidden_row_stride,
                         total_rows, logit_indices + r0, (int64_t)n, norm_weight, eps, (int)hidden, xn, ok);
    uint16_t* lg_group = lg != nullptr ? lg + r0 * logits_row_stride : nullptr;
    if (dtype == HX_DTYPE_BF16)
      launch_group<__bf16>(pad / 16, lay.tiles, s, emb, embedding_row_stride, vocab, hidden, xn, n, partial,
                           lg_group, logits_row_stride);
    else
      launch_group<_Float16>(pad / 16, lay.tiles, s, emb, embedding_row_stride, vocab, hidden, xn, n, partial,
                             lg_group, logits_row_stride);
    hipLaunchKernelGGL(argmax_reduce_kernel, dim3(n), dim3(kLgThreads), 0, s, partial, lay.tiles, ok,
                       token_ids + r0, max_logits != nullptr ? max_logits + r0 : nullptr);
  }
  return hx::status_from_hip(hipGetLastError());
}
