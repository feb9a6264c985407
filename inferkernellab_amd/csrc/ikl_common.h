// Shared device helpers for the gfx950 paged-decode kernels: element
// traits for fp16 / bf16 / fp32, 16-byte vector loads, dot products on
// packed halves, wave-level DPP reductions and the thread-local error slot
// of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/ikl_paged.h"

namespace ikl {

// ---------------------------------------------------------------- errors
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int check_launch(const char *what);

// ---------------------------------------------------------- element types
struct f16_tag {};
struct bf16_tag {};
struct f32_tag {};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

template <typename Tag> struct elem;

template <> struct elem<f16_tag> {
  static constexpr int bytes = 2;
  static constexpr int vec = 8;  // elements per 16-byte chunk
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(half2_t, w)[0];
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(half2_t, w)[1];
  }
  // fp32 accumulate of a.lo*b.lo + a.hi*b.hi + c.
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                  c, false);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    half2_t h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
};

__device__ inline uint32_t f32_to_bf16_bits(float f) {
  // Round to nearest even, NaN kept quiet (matches torch's float->bfloat16).
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

template <> struct elem<bf16_tag> {
  static constexpr int bytes = 2;
  static constexpr int vec = 8;
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                           __builtin_bit_cast(bf162_t, b), c, false);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
  }
};

template <> struct elem<f32_tag> {
  static constexpr int bytes = 4;
  static constexpr int vec = 4;
};

// ------------------------------------------------------------ wave helpers
// DPP controls (gfx9 encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i <-> 7-i within 8
constexpr int DPP_ROW_MIRROR = 0x140;       // lane i <-> 15-i within 16

template <int CTRL>
__device__ inline float dpp_mov(float v) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N contiguous lanes (N in 1,2,4,8,16); every lane
// of the group receives the group sum. Uses pairings (xor1, xor2, half
// mirror, mirror) whose composition covers each group exactly once.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 2) v += dpp_mov<DPP_QUAD_XOR1>(v);
  if constexpr (N >= 4) v += dpp_mov<DPP_QUAD_XOR2>(v);
  if constexpr (N >= 8) v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
  if constexpr (N >= 16) v += dpp_mov<DPP_ROW_MIRROR>(v);
  static_assert(N <= 16, "group_sum supports up to 16 lanes");
  return v;
}

__device__ inline float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// gfx950 v_permlane16_swap / v_permlane32_swap with both operands = v: the
// two results hold, per lane l, v[l] and v[l ^ 16] (resp. v[l ^ 32]) in some
// order, so a symmetric op of the pair is the xor-16 (xor-32) butterfly step
// without the LDS round trip of ds_bpermute.
__device__ inline float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct alignas(16) u32x4 {
  uint32_t x, y, z, w;
};

__device__ inline u32x4 load16(const void *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}

// 16-byte load through the global address space (global_load_dwordx4,
// counted by vmcnt only — a generic pointer would become a flat load that
// also holds lgkmcnt).
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) v4u32 *global_v4u32_ptr;
__device__ inline u32x4 load16_global(const void *p) {
  const v4u32 v = *(global_v4u32_ptr)(p);
  return u32x4{v.x, v.y, v.z, v.w};
}
__device__ inline v4u32 load16v_global(const void *p) { return *(global_v4u32_ptr)(p); }

// Streaming (non-temporal) 16-byte load for K/V rows that are read exactly
// once per launch: keeps them from displacing reusable lines in L2 / MALL.
__device__ inline v4u32 load16v_stream(const void *p) {
  return __builtin_nontemporal_load((global_v4u32_ptr)(p));
}
__device__ inline u32x4 load16_stream(const void *p) {
  const v4u32 v = load16v_stream(p);
  return u32x4{v.x, v.y, v.z, v.w};
}
__device__ inline void store16(void *p, const u32x4 &v) {
  *reinterpret_cast<u32x4 *>(p) = v;
}
__device__ inline uint32_t u32x4_at(const u32x4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// FP8 KV rows: the power-of-two scale 2^ceil(log2(amax / 448)) (at least
// 2^-126) of a row whose largest magnitude is amax, read off the bits of the
// correctly rounded amax / 448; 1 for a zero or non-finite amax. Codes are
// e4m3(x / scale): the division by a power of two is exact.
__device__ inline float e4m3_row_scale(float amax) {
  if (!(amax > 0.f) || amax == INFINITY) return 1.0f;
  const uint32_t bits = __float_as_uint(amax / 448.0f);
  int e = (int)((bits >> 23) & 0xffu) - 127 + ((bits & 0x7fffffu) != 0u ? 1 : 0);
  e = e < -126 ? -126 : (e > 127 ? 127 : e);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

template <typename IdxT>
__device__ inline int64_t load_index(const void *base, int64_t i) {
  return (int64_t)(reinterpret_cast<const IdxT *>(base)[i]);
}

}  // namespace ikl
