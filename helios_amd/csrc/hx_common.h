// Shared device helpers for the gfx950 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/helios_paged.h"

namespace hx {

// Work-item and workgroup indices and the workgroup size along x, read with the
// intrinsics. HIP's threadIdx / blockIdx / blockDim / gridDim go through device-library
// functions built for IEEE mode, which the inliner keeps out of these non-IEEE kernels:
// every use was a real call, and a kernel that calls gives up registers to the calling
// convention. The workgroup count is not read on the device: the grid size intrinsic
// loads it from the dispatch packet in the queue's host-visible memory, an uncached read
// per workgroup that made a 2048-row append 4x slower; grid-stride kernels take their
// workgroup count as an argument instead.
__device__ __forceinline__ int tid_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int wg_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int wg_size_x() { return (int)__builtin_amdgcn_workgroup_size_x(); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Element-type traits: 8-wide MFMA operand, the 16x16x32 MFMA, and conversions.
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  typedef bf16x8_t v8;
  static __device__ __forceinline__ f32x4_t mfma16x16x32(v8 a, v8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // Low / high 16-bit halves of a packed pair, widened to fp32 exactly.
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ uint16_t bits(float f) {
    __bf16 h = (__bf16)f;  // round to nearest even
    return __builtin_bit_cast(uint16_t, h);
  }
  // c + a.lo*b.lo + a.hi*b.hi for two packed pairs (v_dot2_f32_bf16).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
};

template <>
struct Elem<_Float16> {
  typedef f16x8_t v8;
  static __device__ __forceinline__ f32x4_t mfma16x16x32(v8 a, v8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static __device__ __forceinline__ uint16_t bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
  }
};

// 2^x with the raw v_exp_f32 (exp2f adds denormal-range fix-ups around it). Softmax
// arguments are <= 0; results below 2^-126 flush to zero and 2^-inf is 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two floats rounded to nearest-even and packed as {lo, hi} 16-bit elements.
template <typename T>
__device__ __forceinline__ uint32_t pack2_round(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2_round<__bf16>(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
}
template <>
__device__ __forceinline__ uint32_t pack2_round<_Float16>(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, h2));
}

// Eight packed 1.0 values of element type T.
template <typename T>
__device__ __forceinline__ uint4 ones8();
template <>
__device__ __forceinline__ uint4 ones8<__bf16>() { return make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u); }
template <>
__device__ __forceinline__ uint4 ones8<_Float16>() { return make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u); }

template <typename T>
__device__ __forceinline__ typename Elem<T>::v8 as_v8(uint4 u) {
  return __builtin_bit_cast(typename Elem<T>::v8, u);
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// 16-byte load with the non-temporal hint: K/V rows are streamed once per tick, and
// streaming them past the caches leaves L2 to the split partials and metadata.
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Raw buffer resource over `bytes` bytes from `base` (stride 0: byte addressing, reads
// past `bytes` return zeros), for loads whose per-lane part is a 32-bit offset and whose
// per-load part is a scalar offset: no per-load vector address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16-byte buffer load at byte offset voff + soff with the non-temporal hint (aux bit 1).
__device__ __forceinline__ uint4 ld16_stream(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// a.lo*b.lo + a.hi*b.hi in fp32 with a zero accumulator, as the three-operand dot2 with an
// inline 0: the two-operand form ties the accumulator to the destination and needs a
// v_mov of 0 first.
template <typename T>
__device__ __forceinline__ float dot2_zero(uint32_t a, uint32_t b);
template <>
__device__ __forceinline__ float dot2_zero<__bf16>(uint32_t a, uint32_t b) {
  float r;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <>
__device__ __forceinline__ float dot2_zero<_Float16>(uint32_t a, uint32_t b) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// 8 packed elements . 8 packed elements, in fp32 (four dot2 steps from zero).
template <typename T>
__device__ __forceinline__ float dot8_zero(uint4 a, uint4 b) {
  float c = dot2_zero<T>(a.x, b.x);
  c = Elem<T>::dot2(a.y, b.y, c);
  c = Elem<T>::dot2(a.z, b.z, c);
  return Elem<T>::dot2(a.w, b.w, c);
}

// s_waitcnt immediate for vmcnt(0), other counters unconstrained (gfx9 encoding).
constexpr unsigned kWaitVm0 = 0x0f70;

// 16-byte buffer load at byte offset voff straight into LDS: lane l's bytes land at
// lds_base + 16 l (lds_base wave-uniform). Completion is counted by vmcnt.
__device__ __forceinline__ void ld16_to_lds(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, (int)voff, 0, 0, 0);
}

// ds_read_b64_tr_b16 at LDS byte address p. Within each 16-lane group the lanes' 8-byte
// reads form a 4 x 16 block of 16-bit values (lane i supplies elements 4i..4i+3, row-major);
// lane j of the group receives column j, i.e. elements j, 16 + j, 32 + j, 48 + j.
__device__ __forceinline__ uint2 ld8_lds_tr16(const void* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Stores with the non-temporal hint (global_store ... nt): the chunk kernel's output rows
// and split partials are written once at a workgroup's end and read by a later launch;
// streamed this way the workgroups of a launch finish sooner.
__device__ __forceinline__ void st16_nt(void* p, uint4 v) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4u{v.x, v.y, v.z, v.w}, static_cast<v4u*>(p));
}
__device__ __forceinline__ void st8_nt(void* p, uint32_t x, uint32_t y) {
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(v2u{x, y}, static_cast<v2u*>(p));
}

// Holds a loaded value in registers at this point of the program, so that the
// compiler cannot sink its load below a later branch (a load issued before a test
// shares the memory round trip of the loads the test waits for).
template <typename W>
__device__ __forceinline__ void hold(const W& v) {
  if constexpr (sizeof(W) >= 4) {
    struct Words { uint32_t d[sizeof(W) / 4]; };
    const Words u = __builtin_bit_cast(Words, v);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(W) / 4); ++i) asm volatile("" ::"v"(u.d[i]));
  } else {
    asm volatile("" ::"v"((uint32_t)v));
  }
}

// 16-byte buffer load at byte offset voff (default cache policy).
__device__ __forceinline__ uint4 ld16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// 8 packed elements . 8 packed elements + c, in fp32 (four dot2 steps).
template <typename T>
__device__ __forceinline__ float dot8(uint4 a, uint4 b, float c) {
  c = Elem<T>::dot2(a.x, b.x, c);
  c = Elem<T>::dot2(a.y, b.y, c);
  c = Elem<T>::dot2(a.z, b.z, c);
  return Elem<T>::dot2(a.w, b.w, c);
}

// Per-lane select by a wave-uniform 64-bit lane mask held in scalar registers: lanes whose
// mask bit is set take a, the others b. Written as the three-operand v_cndmask_b32 so the
// mask stays in an SGPR pair: the compiler otherwise picks the two-operand form that
// reads VCC, which issues about 4x slower on gfx950.
__device__ __forceinline__ float lane_sel(uint64_t mask, float a, float b) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(mask));
  return r;
}
__device__ __forceinline__ uint32_t lane_sel(uint64_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(mask));
  return r;
}
// Lanes whose index within their 16-lane row has `bit` set.
__device__ __forceinline__ constexpr uint64_t row_bit_lanes(int bit) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((l & 15) >> bit & 1) m |= 1ull << l;
  return m;
}

// Cross-lane moves within a 16-lane row (DPP). Each pairing is an involution:
// xor1 / xor2 within quads, half-mirror (lane ^ 7 within 8), mirror (lane ^ 15).
enum : int {
  kDppXor1 = 0xB1,        // quad_perm [1,0,3,2]
  kDppXor2 = 0x4E,        // quad_perm [2,3,0,1]
  kDppHalfMirror = 0x141, // row_half_mirror
  kDppMirror = 0x140,     // row_mirror
};
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Combine with the lane 16 (32) apart using the gfx950 permlane swaps: a VALU exchange
// instead of an LDS permute. Swapping a value with itself leaves lane l holding
// {x[l], x[l ^ 16]} (for 32: {x[l], x[l ^ 32]}) with the lower lane's value first in
// both lanes of a pair, so both get the identical result.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// Interleave the low (sel=0) or high (sel=1) 16-bit halves of x and y: {x.h, y.h}.
__device__ __forceinline__ uint32_t interleave_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t interleave_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask_lo, int mask_hi) {
  for (int m = mask_lo; m <= mask_hi; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum_xor(float v, int mask_lo, int mask_hi) {
  for (int m = mask_lo; m <= mask_hi; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

inline int status_from_hip(hipError_t e) { return e == hipSuccess ? HX_OK : (int)e; }

// Log-sum-exp fold of attention results over disjoint key sets of one query row and head
// h, for the 8 dims 8li..8li+7 a lane owns: parts p0..p1-1 are rows part_idx[p] (or p when
// part_idx is null) of oa (element type T, 16-byte aligned rows) with natural-log
// log-sum-exps lse_a[h * lse_stride + row]; rows outside [0, a_rows) are skipped. Each
// part folds into the running (acc, m) in list order:
//   o = fma(o_a, w_a, o * w_b) / (w_a + w_b),  m = max + log(w_a + w_b),
// w = e^(lse - max). Up to four parts' indices, lse and rows are loaded together before
// they are folded. Returns whether any part was folded.
template <typename T>
__device__ __forceinline__ bool fold_parts(float (&acc)[8], float& m, const uint16_t* oa, int64_t a_row,
                                           int64_t a_head, const float* lse_a, int64_t lse_stride,
                                           int64_t a_rows, int h, int li, const int32_t* part_idx,
                                           int64_t p0, int64_t p1) {
  bool changed = false;
  for (int64_t pb = p0; pb < p1; pb += 4) {
    int64_t ja[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      ja[k] = -1;
      if (pb + k < p1) ja[k] = part_idx != nullptr ? (int64_t)part_idx[pb + k] : pb + k;
    }
    float la[4];
    uint4 pv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool ok = ja[k] >= 0 && ja[k] < a_rows;
      la[k] = ok ? lse_a[(int64_t)h * lse_stride + ja[k]] : -INFINITY;
      pv[k] = ok ? *reinterpret_cast<const uint4*>(oa + ja[k] * a_row + (int64_t)h * a_head + 8 * li)
                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (!(ja[k] >= 0 && ja[k] < a_rows)) continue;
      const float mn = fmaxf(m, la[k]);
      if (mn == -INFINITY) continue;  // neither side saw a key yet
      const float wa = expf(la[k] - mn), wb = expf(m - mn);
      const uint32_t w4[4] = {pv[k].x, pv[k].y, pv[k].z, pv[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xa0 = Elem<T>::lo(w4[e]), xa1 = Elem<T>::hi(w4[e]);
        acc[2 * e] = fmaf(xa0, wa, acc[2 * e] * wb) / (wa + wb);
        acc[2 * e + 1] = fmaf(xa1, wa, acc[2 * e + 1] * wb) / (wa + wb);
      }
      m = mn + logf(wa + wb);
      changed = true;
    }
  }
  return changed;
}

}  // namespace hx
