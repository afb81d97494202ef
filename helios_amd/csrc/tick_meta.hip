// Per-tick attention metadata built on the device (gfx950).
//
// Reference: PagedBatchCache.prepare (src/helios/runtime/qwen3/paged_cache.py:221-270)
// and PackedBatchCache.prepare_packed (:418-494) build cu_seq_q, cu_seq_k, seqused_k,
// positions, logit_indices and write_slots as Python lists, one entry per token, and
// copy each to the device through `metadata` (:272-288). Here the host uploads three
// int32 values per sequence (length before the tick, tokens this tick, logit rows) and
// one launch derives every array: workgroup 0 writes the per-sequence arrays and the
// logit indices, workgroups 1.. write one token row per thread.

#include "hx_common.h"

namespace {

constexpr int kMetaThreads = 256;
constexpr int kMetaMaxBatch = 4096;

struct MetaArgs {
  const int32_t* seq;  // lengths[B], counts[B], logit_counts[B]
  int32_t batch;
  int32_t total_q;
  int32_t n_logits;
  const int32_t* bt;
  int32_t bt_stride;
  int32_t page_size;
  int32_t* cu_q;
  int32_t* cu_k;
  int32_t* used_k;
  int64_t* positions;
  int64_t* slots;
  int64_t* logit_idx;
};

// Exclusive prefix sum of in[0..n) into out[0..n] (out[n] = total) by one workgroup.
// Each thread sums a contiguous run of ceil(n / 256) values; the 256 run totals are
// scanned in LDS (Hillis-Steele); then each thread writes its run.
__device__ void block_scan(const int32_t* in, int32_t* out, int n, int32_t* part) {
  const int tid = hx::tid_x();
  const int per = (n + kMetaThreads - 1) / kMetaThreads;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  int32_t run = 0;
  for (int i = lo; i < hi; ++i) run += in[i];
  part[tid] = run;
  __syncthreads();
  for (int d = 1; d < kMetaThreads; d <<= 1) {
    const int32_t add = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int32_t acc = part[tid] - run;  // exclusive prefix of this run
  for (int i = lo; i < hi; ++i) {
    out[i] = acc;
    acc += in[i];
  }
  if (tid == kMetaThreads - 1) out[n] = part[tid];
  __syncthreads();
}

__global__ __launch_bounds__(kMetaThreads) void tick_meta_kernel(MetaArgs a) {
  __shared__ int32_t s_len[kMetaMaxBatch];
  __shared__ int32_t s_cnt[kMetaMaxBatch];
  __shared__ int32_t s_cuq[kMetaMaxBatch + 1];
  __shared__ int32_t s_aux[kMetaMaxBatch + 1];
  __shared__ int32_t s_part[kMetaThreads];
  const int B = a.batch, tid = hx::tid_x();
  for (int b = tid; b < B; b += kMetaThreads) {
    s_len[b] = a.seq[b];
    s_cnt[b] = a.seq[B + b];
  }
  __syncthreads();
  block_scan(s_cnt, s_cuq, B, s_part);

  if (hx::wg_x() == 0) {
    for (int b = tid; b <= B; b += kMetaThreads) a.cu_q[b] = s_cuq[b];
    // Sequence ends E_b = length + count, their prefix sums, and seqused_k.
    for (int b = tid; b < B; b += kMetaThreads) {
      const int32_t e = s_len[b] + s_cnt[b];
      a.used_k[b] = e;
      s_len[b] = e;  // s_len now holds the ends
    }
    __syncthreads();
    block_scan(s_len, s_aux, B, s_part);
    for (int b = tid; b <= B; b += kMetaThreads) a.cu_k[b] = s_aux[b];
    if (a.logit_idx != nullptr) {
      __syncthreads();
      for (int b = tid; b < B; b += kMetaThreads) s_len[b] = a.seq[2 * B + b];  // logit rows
      __syncthreads();
      block_scan(s_len, s_aux, B, s_part);
      for (int b = tid; b < B; b += kMetaThreads) {
        const int tail = s_len[b];
        const int end = s_cuq[b + 1];
        for (int i = 0; i < tail; ++i) {
          const int o = s_aux[b] + i;
          if (o < a.n_logits) a.logit_idx[o] = (int64_t)(end - tail + i);
        }
      }
    }
    return;
  }

  // Token rows: row t belongs to the last sequence b with cu_q[b] <= t.
  const int t = (int)(hx::wg_x() - 1) * kMetaThreads + tid;
  if (t >= a.total_q) return;
  int64_t pos = -1, slot = -1;
  if (t < s_cuq[B]) {
    int lo = 0, hi = B - 1;  // invariant: s_cuq[lo] <= t < s_cuq[hi + 1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cuq[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    pos = (int64_t)s_len[b] + (t - s_cuq[b]);
    const int64_t pi = pos / a.page_size;
    if (pi < a.bt_stride) {
      const int32_t page = a.bt[(int64_t)b * a.bt_stride + pi];
      slot = (int64_t)page * a.page_size + (pos - pi * a.page_size);
    }
  }
  if (a.positions != nullptr) a.positions[t] = pos;
  a.slots[t] = slot;
}

}  // namespace

extern "C" int hx_tick_metadata(const int32_t* seq, int32_t batch, int32_t total_q,
                                int32_t n_logits, const int32_t* block_table,
                                int32_t block_table_stride, int32_t page_size,
                                int32_t* cu_seq_q, int32_t* cu_seq_k, int32_t* seqused_k,
                                int64_t* positions, int64_t* write_slots,
                                int64_t* logit_indices, void* stream) {
  if (batch < 1 || batch > kMetaMaxBatch || total_q < 0 || n_logits < 0 || page_size < 1 ||
      block_table_stride < 1)
    return HX_E_INVALID_ARG;
  if (!seq || !block_table || !cu_seq_q || !cu_seq_k || !seqused_k || !write_slots)
    return HX_E_INVALID_ARG;
  if (n_logits > 0 && !logit_indices) return HX_E_INVALID_ARG;
  MetaArgs a;
  a.seq = seq;
  a.batch = batch;
  a.total_q = total_q;
  a.n_logits = n_logits;
  a.bt = block_table;
  a.bt_stride = block_table_stride;
  a.page_size = page_size;
  a.cu_q = cu_seq_q;
  a.cu_k = cu_seq_k;
  a.used_k = seqused_k;
  a.positions = positions;
  a.slots = write_slots;
  a.logit_idx = n_logits > 0 ? logit_indices : nullptr;
  const unsigned grid = 1u + (unsigned)((total_q + kMetaThreads - 1) / kMetaThreads);
  hipLaunchKernelGGL(tick_meta_kernel, dim3(grid), dim3(kMetaThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return hx::status_from_hip(hipGetLastError());
}

// ---------------------------------------------------------------- attention merge
// Attention results over disjoint key sets of the same query row, each normalised with
// its own log-sum-exp, combine exactly into the result over the union:
//   o = (sum_i o_i e^(lse_i - m)) / (sum_i e^(lse_i - m)),  lse = m + log(sum_i e^(lse_i - m)),
// m = max_i lse_i. Entry j merges its parts (rows of o_a) into packed row rows[j] of
// (out, lse_out) in place: parts part_idx[part_start[j]] .. part_idx[part_start[j+1]-1],
// or o_a row j alone when part_start is null. The parts are folded in list order, two
// at a time as in the formula above with one of them the running result.
namespace {

template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(uint16_t* out, int64_t o_row, int64_t o_head,
                                                    float* lse_out, int64_t total_out,
                                                    const uint16_t* oa, int64_t a_row, int64_t a_head,
                                                    const float* lse_a, int64_t total_a,
                                                    const int64_t* rows, const int32_t* part_start,
                                                    const int32_t* part_idx, int64_t n_parts,
                                                    int64_t n_rows, int hq) {
  // One wave per (entry j, head h); lane l owns dims l and l + 64. Every lane reads the old
  // lse before lane 0 stores the merged one, in program order within the wave.
  const int64_t item = (int64_t)hx::wg_x() * 4 + (hx::tid_x() >> 6);
  const int lane = hx::tid_x() & 63;
  if (item >= n_rows * hq) return;
  const int64_t j = item / hq;
  const int h = (int)(item - j * hq);
  const int64_t r = rows[j];
  if (r < 0 || r >= total_out) return;
  int64_t p0 = j, p1 = j + 1;
  if (part_start != nullptr) {  // a range outside the part list is clipped to it
    p0 = max((int64_t)part_start[j], (int64_t)0);
    p1 = min((int64_t)part_start[j + 1], n_parts);
  }
  float* lb_p = lse_out + (int64_t)h * total_out + r;
  float m = *lb_p;  // the running result is normalised, with log-sum-exp m
  uint16_t* po = out + r * o_row + (int64_t)h * o_head;
  float acc[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) acc[k] = (float)__builtin_bit_cast(T, po[lane + 64 * k]);
  bool changed = false;
  for (int64_t p = p0; p < p1; ++p) {
    const int64_t ja = part_start != nullptr ? (int64_t)part_idx[p] : p;
    if (ja < 0 || ja >= total_a) continue;
    const float la = lse_a[(int64_t)h * total_a + ja];
    const float mn = fmaxf(m, la);
    if (mn == -INFINITY) continue;  // neither side saw a key yet
    const float wa = expf(la - mn), wb = expf(m - mn);
    const uint16_t* pa = oa + ja * a_row + (int64_t)h * a_head;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float xa = (float)__builtin_bit_cast(T, pa[lane + 64 * k]);
      acc[k] = fmaf(xa, wa, acc[k] * wb) / (wa + wb);  // one rounding order in both kernels
    }
    m = mn + logf(wa + wb);
    changed = true;
  }
  if (!changed) return;
#pragma unroll
  for (int k = 0; k < 2; ++k) po[lane + 64 * k] = __builtin_bit_cast(uint16_t, (T)acc[k]);
  if (lane == 0) *lb_p = m;
}

// merge_kernel's arithmetic with a short dependency chain: 16 lanes per (entry j, head h),
// lane i owning dims 8i..8i+7 (16-byte loads; rows 16-byte aligned, checked on the host),
// and the part indices, part log-sum-exps and part rows of up to four parts loaded
// together before they are folded, in list order, exactly as merge_kernel folds them.
template <typename T>
__global__ __launch_bounds__(256) void merge_vec_kernel(uint16_t* out, int64_t o_row, int64_t o_head,
                                                        float* lse_out, int64_t total_out,
                                                        const uint16_t* oa, int64_t a_row, int64_t a_head,
                                                        const float* lse_a, int64_t total_a,
                                                        const int64_t* rows, const int32_t* part_start,
                                                        const int32_t* part_idx, int64_t n_parts,
                                                        int64_t n_rows, int hq) {
  const int64_t item = (int64_t)hx::wg_x() * 16 + (hx::tid_x() >> 4);
  const int li = hx::tid_x() & 15;
  if (item >= n_rows * hq) return;
  const int64_t j = item / hq;
  const int h = (int)(item - j * hq);
  const int64_t r = rows[j];
  int64_t p0 = j, p1 = j + 1;
  if (part_start != nullptr) {  // a range outside the part list is clipped to it
    p0 = max((int64_t)part_start[j], (int64_t)0);
    p1 = min((int64_t)part_start[j + 1], n_parts);
  }
  if (r < 0 || r >= total_out) return;
  float* lb_p = lse_out + (int64_t)h * total_out + r;
  uint16_t* po = out + r * o_row + (int64_t)h * o_head + 8 * li;
  float m = *lb_p;  // the running result is normalised, with log-sum-exp m
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
  // Parts outside [0, total_a) are skipped (o_a holds total_a rows).
  const bool changed = hx::fold_parts<T>(acc, m, oa, a_row, a_head, lse_a, total_a, total_a, h, li,
                                         part_start != nullptr ? part_idx : nullptr, p0, p1);
  if (!changed) return;
  uint4 u;
  u.x = hx::pack2_round<T>(acc[0], acc[1]);
  u.y = hx::pack2_round<T>(acc[2], acc[3]);
  u.z = hx::pack2_round<T>(acc[4], acc[5]);
  u.w = hx::pack2_round<T>(acc[6], acc[7]);
  // Every lane of the entry has read the old lse (above, before any fold) before lane 0
  // of the entry stores the merged one: all 16 lanes sit in one wave, in program order.
  *reinterpret_cast<uint4*>(po) = u;
  if (li == 0) *lb_p = m;
}

}  // namespace

extern "C" int hx_attn_merge(void* out, int64_t out_row_stride, int64_t out_head_stride,
                             float* lse_out, int64_t total_out,
                             const void* o_a, int64_t a_row_stride, int64_t a_head_stride,
                             const float* lse_a, int64_t total_a,
                             const int64_t* rows, const int32_t* part_start, const int32_t* part_idx,
                             int64_t n_parts, int64_t n_rows, int32_t n_heads, int32_t head_dim,
                             int32_t dtype, void* stream) {
  if (head_dim != 128 || (dtype != HX_DTYPE_BF16 && dtype != HX_DTYPE_FP16)) return HX_E_UNSUPPORTED;
  if (n_rows < 0 || n_heads < 1 || total_out < 0 || total_a < 0) return HX_E_INVALID_ARG;
  if (part_start == nullptr && total_a < n_rows) return HX_E_INVALID_ARG;
  if ((part_start == nullptr) != (part_idx == nullptr) || n_parts < 0) return HX_E_INVALID_ARG;
  if (n_rows == 0) return HX_OK;
  if (!out || !lse_out || !o_a || !lse_a || !rows) return HX_E_INVALID_ARG;
  const int64_t items = n_rows * n_heads;
  if ((items + 3) / 4 > 0x7fffffff) return HX_E_INVALID_ARG;
  const unsigned grid = (unsigned)((items + 3) / 4);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint16_t* o = static_cast<uint16_t*>(out);
  const uint16_t* a = static_cast<const uint16_t*>(o_a);
  const bool vec = out_row_stride % 8 == 0 && out_head_stride % 8 == 0 && a_row_stride % 8 == 0 &&
                   a_head_stride % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(o_a) % 16 == 0;
  if (vec) {
    const unsigned vgrid = (unsigned)((items + 15) / 16);
    if (dtype == HX_DTYPE_BF16)
      hipLaunchKernelGGL(merge_vec_kernel<__bf16>, dim3(vgrid), dim3(256), 0, s, o, out_row_stride,
                         out_head_stride, lse_out, total_out, a, a_row_stride, a_head_stride, lse_a, total_a,
                         rows, part_start, part_idx, n_parts, n_rows, n_heads);
    else
      hipLaunchKernelGGL(merge_vec_kernel<_Float16>, dim3(vgrid), dim3(256), 0, s, o, out_row_stride,
                         out_head_stride, lse_out, total_out, a, a_row_stride, a_head_stride, lse_a, total_a,
                         rows, part_start, part_idx, n_parts, n_rows, n_heads);
    return hx::status_from_hip(hipGetLastError());
  }
  if (dtype == HX_DTYPE_BF16)
    hipLaunchKernelGGL(merge_kernel<__bf16>, dim3(grid), dim3(256), 0, s, o, out_row_stride, out_head_stride,
                       lse_out, total_out, a, a_row_stride, a_head_stride, lse_a, total_a, rows, part_start,
                       part_idx, n_parts, n_rows, n_heads);
  else
    hipLaunchKernelGGL(merge_kernel<_Float16>, dim3(grid), dim3(256), 0, s, o, out_row_stride, out_head_stride,
                       lse_out, total_out, a, a_row_stride, a_head_stride, lse_a, total_a, rows, part_start,
                       part_idx, n_parts, n_rows, n_heads);
  return hx::status_from_hip(hipGetLastError());
}
