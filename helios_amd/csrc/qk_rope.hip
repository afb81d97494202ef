// Per-head RMSNorm + RoPE of the new queries and keys, fused with the KV append (gfx950).
//
// Reference: GroupedQueryAttention.forward (src/helios/runtime/qwen3/layers.py:131-164)
// applies q_norm / k_norm (RMSNorm over head_dim in fp32, layers.py:30-40), then
// apply_rope (layers.py:54-72: x * cos + cat(-x2, x1) * sin in fp32, cast back), then
// PagedBatchCache.attend appends K and V into the pool (_write, paged_cache.py:335-345).
// Here one launch reads the projections once: queries come out normalised and rotated,
// keys are normalised, rotated and stored straight into their pool rows, and values are
// copied into theirs; the rotated keys never make a round trip through HBM.
//
// One workgroup per packed row. The 16-byte-access kernel (aligned rows) gives each head
// 16 lanes of 8 dims; the 2-byte-access kernel gives each head a wave, lane l owning dims
// l and l + 64, which are exactly the pair that RoPE mixes. The arithmetic follows the reference's op order with no fused
// multiply-adds: n = bf16((x * rsqrt(mean(x^2) + eps)) * w), then
// out = bf16(n * cos + (-n') * sin).

#include "hx_common.h"

namespace {

constexpr int kRopeD = 128;
constexpr int kRopeThreads = 256;

struct RopeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_row, q_head, k_row, k_head, v_row, v_head;
  const float* q_scale;
  const float* k_scale;
  const float* cos;
  const float* sin;
  int64_t rope_rows;
  const int64_t* positions;
  int64_t n_rows;
  int32_t hq, hkv;
  float eps;
  uint16_t* q_out;
  int64_t qo_row, qo_head;
  uint16_t* k_pool;
  uint16_t* v_pool;
  int64_t pool_rows;
  const int64_t* slots;
};

template <typename T>
__device__ __forceinline__ float to_f(uint16_t b) {
  return (float)__builtin_bit_cast(T, b);
}
template <typename T>
__device__ __forceinline__ uint16_t from_f(float f) {
  return __builtin_bit_cast(uint16_t, (T)f);
}

template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_append_kernel(RopeArgs a) {
  // One workgroup per packed row: the row's position, slot, RoPE factors and norm
  // weights are read once and reused by every head; wave w takes heads w, w + 4, ...
  const int lane = hx::tid_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(hx::tid_x() >> 6);
  const int64_t row = hx::wg_x();
  const int heads = a.hq + 2 * a.hkv;
  const int64_t slot = a.slots[row];
  const bool slot_ok = slot >= 0 && slot < a.pool_rows;
  int64_t pos = a.positions[row];
  pos = pos < 0 ? 0 : (pos >= a.rope_rows ? a.rope_rows - 1 : pos);
  const float c0 = a.cos[pos * kRopeD + lane], c1 = a.cos[pos * kRopeD + lane + 64];
  const float s0 = a.sin[pos * kRopeD + lane], s1 = a.sin[pos * kRopeD + lane + 64];
  const float wq0 = a.q_scale[lane], wq1 = a.q_scale[lane + 64];
  const float wk0 = a.k_scale[lane], wk1 = a.k_scale[lane + 64];
  for (int h = wave; h < heads; h += kRopeThreads / 64) {
    if (h >= a.hq + a.hkv) {  // value head: plain copy into the pool
      if (!slot_ok) continue;
      const int hv = h - a.hq - a.hkv;
      const uint16_t* src = a.v + row * a.v_row + hv * a.v_head;
      uint16_t* dst = a.v_pool + (slot * a.hkv + hv) * kRopeD;
      const uint16_t e0 = src[lane], e1 = src[lane + 64];
      dst[lane] = e0;
      dst[lane + 64] = e1;
      continue;
    }
    const bool is_q = h < a.hq;
    const int hh = is_q ? h : h - a.hq;
    if (!is_q && !slot_ok) continue;
    const uint16_t* src = is_q ? a.q + row * a.q_row + hh * a.q_head : a.k + row * a.k_row + hh * a.k_head;
    const float x0 = to_f<T>(src[lane]), x1 = to_f<T>(src[lane + 64]);
    float ss = __fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1));
    for (int m = 32; m >= 1; m >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, m));
    const float r = rsqrtf(__fadd_rn(__fdiv_rn(ss, (float)kRopeD), a.eps));
    const float n0 = to_f<T>(from_f<T>(__fmul_rn(__fmul_rn(x0, r), is_q ? wq0 : wk0)));
    const float n1 = to_f<T>(from_f<T>(__fmul_rn(__fmul_rn(x1, r), is_q ? wq1 : wk1)));
    const float o0 = __fadd_rn(__fmul_rn(n0, c0), __fmul_rn(-n1, s0));
    const float o1 = __fadd_rn(__fmul_rn(n1, c1), __fmul_rn(n0, s1));
    uint16_t* dst = is_q ? a.q_out + row * a.qo_row + hh * a.qo_head
                         : a.k_pool + (slot * a.hkv + hh) * kRopeD;
    dst[lane] = from_f<T>(o0);
    dst[lane + 64] = from_f<T>(o1);
  }
}

// The same computation with 16-byte accesses, for 16-byte aligned rows (the common case):
// a head row is 16 lanes x 8 dims, so each wave takes four heads at a time. Lane j of a
// head owns dims 8j .. 8j + 7; the RoPE partner of dim d (d +- 64) sits in lane j ^ 8 at
// the same position and comes over in four packed 32-bit shuffles. The sum of squares is
// reduced over the 16 lanes of the head; the element arithmetic is the scalar kernel's.
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_append_vec_kernel(RopeArgs a) {
  const int lane = hx::tid_x() & 63;
  const int wave = __builtin_amdgcn_readfirstlane(hx::tid_x() >> 6);
  const int sub = lane >> 4, j = lane & 15;
  const int64_t row = hx::wg_x();
  const int heads = a.hq + 2 * a.hkv;
  const int64_t slot = a.slots[row];
  const bool slot_ok = slot >= 0 && slot < a.pool_rows;
  int64_t pos = a.positions[row];
  pos = pos < 0 ? 0 : (pos >= a.rope_rows ? a.rope_rows - 1 : pos);
  float c[8], sn[8], wq[8], wk[8];
  {
    const float4* cp = reinterpret_cast<const float4*>(a.cos + pos * kRopeD + 8 * j);
    const float4* sp = reinterpret_cast<const float4*>(a.sin + pos * kRopeD + 8 * j);
    const float4* qp = reinterpret_cast<const float4*>(a.q_scale + 8 * j);
    const float4* kp = reinterpret_cast<const float4*>(a.k_scale + 8 * j);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4 c4 = cp[h], s4 = sp[h], q4 = qp[h], k4 = kp[h];
      c[4 * h] = c4.x; c[4 * h + 1] = c4.y; c[4 * h + 2] = c4.z; c[4 * h + 3] = c4.w;
      sn[4 * h] = s4.x; sn[4 * h + 1] = s4.y; sn[4 * h + 2] = s4.z; sn[4 * h + 3] = s4.w;
      wq[4 * h] = q4.x; wq[4 * h + 1] = q4.y; wq[4 * h + 2] = q4.z; wq[4 * h + 3] = q4.w;
      wk[4 * h] = k4.x; wk[4 * h + 1] = k4.y; wk[4 * h + 2] = k4.z; wk[4 * h + 3] = k4.w;
    }
  }
  for (int h0 = 4 * wave; h0 < heads; h0 += kRopeThreads / 16) {
    const int h = h0 + sub;
    if (h >= heads) continue;  // whole 16-lane groups drop out together
    if (h >= a.hq + a.hkv) {   // value head: plain copy into the pool
      if (!slot_ok) continue;
      const int hv = h - a.hq - a.hkv;
      const uint4 val = *reinterpret_cast<const uint4*>(a.v + row * a.v_row + hv * a.v_head + 8 * j);
      // Non-temporal stores here and below: the rows are read by later launches, and
      // streamed stores finish this one sooner (2048 rows: 11.8-12.0 -> 10.0-10.1 us).
      hx::st16_nt(a.v_pool + (slot * a.hkv + hv) * kRopeD + 8 * j, val);
      continue;
    }
    const bool is_q = h < a.hq;
    const int hh = is_q ? h : h - a.hq;
    if (!is_q && !slot_ok) continue;
    const uint4 raw = *reinterpret_cast<const uint4*>(
        is_q ? a.q + row * a.q_row + hh * a.q_head + 8 * j : a.k + row * a.k_row + hh * a.k_head + 8 * j);
    const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
    float x[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[2 * q] = hx::Elem<T>::lo(rw[q]);
      x[2 * q + 1] = hx::Elem<T>::hi(rw[q]);
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(x[e], x[e]));
#pragma unroll
    for (int m = 1; m <= 8; m <<= 1) ss = __fadd_rn(ss, __shfl_xor(ss, m));
    const float r = rsqrtf(__fadd_rn(__fdiv_rn(ss, (float)kRopeD), a.eps));
    uint32_t np[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      np[q] = hx::pack2_round<T>(__fmul_rn(__fmul_rn(x[2 * q], r), is_q ? wq[2 * q] : wk[2 * q]),
                                 __fmul_rn(__fmul_rn(x[2 * q + 1], r), is_q ? wq[2 * q + 1] : wk[2 * q + 1]));
    const bool low = j < 8;  // dims < 64: out = n c - n' s; else out = n c + n' s
    uint32_t op[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t pp = (uint32_t)__shfl_xor((int)np[q], 8);
      float o[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float n = e ? hx::Elem<T>::hi(np[q]) : hx::Elem<T>::lo(np[q]);
        const float np_ = e ? hx::Elem<T>::hi(pp) : hx::Elem<T>::lo(pp);
        o[e] = __fadd_rn(__fmul_rn(n, c[2 * q + e]), __fmul_rn(low ? -np_ : np_, sn[2 * q + e]));
      }
      op[q] = hx::pack2_round<T>(o[0], o[1]);
    }
    uint16_t* dst = is_q ? a.q_out + row * a.qo_row + hh * a.qo_head + 8 * j
                         : a.k_pool + (slot * a.hkv + hh) * kRopeD + 8 * j;
    hx::st16_nt(dst, make_uint4(op[0], op[1], op[2], op[3]));
  }
}

}  // namespace

extern "C" int hx_qk_norm_rope_append(
    const void* q, int64_t q_row_stride, int64_t q_head_stride,
    const void* k, int64_t k_row_stride, int64_t k_head_stride,
    const void* v, int64_t v_row_stride, int64_t v_head_stride,
    const float* q_norm_weight, const float* k_norm_weight,
    const float* cos, const float* sin, int64_t rope_rows,
    const int64_t* positions, int64_t n_rows,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float eps, int32_t dtype,
    void* q_out, int64_t q_out_row_stride, int64_t q_out_head_stride,
    void* k_pool, void* v_pool, int64_t pool_rows, const int64_t* write_slots,
    void* stream) {
  if (head_dim != kRopeD || (dtype != HX_DTYPE_BF16 && dtype != HX_DTYPE_FP16)) return HX_E_UNSUPPORTED;
  if (n_rows < 0 || n_q_heads < 1 || n_kv_heads < 1 || rope_rows < 1 || !(eps >= 0.f)) return HX_E_INVALID_ARG;
  if (n_rows == 0) return HX_OK;
  if (!q || !k || !v || !q_norm_weight || !k_norm_weight || !cos || !sin || !positions || !q_out ||
      !k_pool || !v_pool || !write_slots)
    return HX_E_INVALID_ARG;
  RopeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.q_row = q_row_stride;
  a.q_head = q_head_stride;
  a.k_row = k_row_stride;
  a.k_head = k_head_stride;
  a.v_row = v_row_stride;
  a.v_head = v_head_stride;
  a.q_scale = q_norm_weight;
  a.k_scale = k_norm_weight;
  a.cos = cos;
  a.sin = sin;
  a.rope_rows = rope_rows;
  a.positions = positions;
  a.n_rows = n_rows;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.eps = eps;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.qo_row = q_out_row_stride;
  a.qo_head = q_out_head_stride;
  a.k_pool = static_cast<uint16_t*>(k_pool);
  a.v_pool = static_cast<uint16_t*>(v_pool);
  a.pool_rows = pool_rows;
  a.slots = write_slots;
  if (n_rows > 0x7fffffff) return HX_E_INVALID_ARG;
  const unsigned grid = (unsigned)n_rows;  // one workgroup per packed row
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // 16-byte path when every row, head and table start is 16-byte aligned.
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(q_out) |
                         reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool) |
                         reinterpret_cast<uintptr_t>(cos) | reinterpret_cast<uintptr_t>(sin) |
                         reinterpret_cast<uintptr_t>(q_norm_weight) | reinterpret_cast<uintptr_t>(k_norm_weight);
  const int64_t strides = q_row_stride | q_head_stride | k_row_stride | k_head_stride | v_row_stride |
                          v_head_stride | q_out_row_stride | q_out_head_stride;
  const bool vec = (ptrs & 15) == 0 && (strides & 7) == 0;
  if (dtype == HX_DTYPE_BF16) {
    if (vec) hipLaunchKernelGGL(qk_norm_rope_append_vec_kernel<__bf16>, dim3(grid), dim3(kRopeThreads), 0, s, a);
    else hipLaunchKernelGGL(qk_norm_rope_append_kernel<__bf16>, dim3(grid), dim3(kRopeThreads), 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL(qk_norm_rope_append_vec_kernel<_Float16>, dim3(grid), dim3(kRopeThreads), 0, s, a);
    else hipLaunchKernelGGL(qk_norm_rope_append_kernel<_Float16>, dim3(grid), dim3(kRopeThreads), 0, s, a);
  }
  return hx::status_from_hip(hipGetLastError());
}
