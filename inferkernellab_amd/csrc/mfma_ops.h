// gfx950 matrix-core building blocks shared by the paged attention kernels
// (decode in paged_decode_mfma.hip, prefill in paged_prefill.hip): operand
// vector types and, per 16-bit element type, the two MFMA shapes used and
// the rounding pack of fp32 probabilities into the P operand.
//
// MFMA operand layouts (gfx950; 16x16x32 checked by a lane-layout probe):
//   16x16x32: lane l supplies A[l%16][8(l/16)+j], B[8(l/16)+j][l%16], j < 8;
//   16x16x16: lane l supplies A[l%16][4(l/16)+j], B[4(l/16)+j][l%16], j < 4;
//   both:     lane l receives D[4(l/16)+i][l%16], i < 4.
// ds_read_b64_tr_b16: in each 16-lane group, lane i receives element i%4 of
//   the 8-byte chunks supplied by lanes 4k + i/4, k < 4.
#pragma once

#include "ikl_common.h"

namespace ikl {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <typename Tag>
struct mfma_ops;

template <>
struct mfma_ops<bf16_tag> {
  // D[16 x 16] += A[16 x 32] . B[32 x 16]
  __device__ static inline f32x4_t mma_k32(v4u32 a, v4u32 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // D[16 x 16] += A[16 x 16] . B[16 x 16]
  __device__ static inline f32x4_t mma_k16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two probabilities (v_cvt_pk_bf16_f32).
  __device__ static inline uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x, y}, bf16x2_t));
  }
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // A 16-bit P keeps 8 significant bits: worth splitting into two MFMAs.
  static constexpr bool NARROW_P = true;
  static constexpr uint32_t ONE2 = 0x3f803f80u;  // two 1.0 elements
};

template <>
struct mfma_ops<f16_tag> {
  __device__ static inline f32x4_t mma_k32(v4u32 a, v4u32 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4_t mma_k16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                                 __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x, y}, f16x2_t));
  }
  __device__ static inline float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[0]; }
  __device__ static inline float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2_t, w)[1]; }
  static constexpr bool NARROW_P = false;  // fp16 P (<= 2^8) already keeps 11 bits
  static constexpr uint32_t ONE2 = 0x3c003c00u;  // two 1.0 elements
};

__device__ inline v4u32 zero4() { return v4u32{0u, 0u, 0u, 0u}; }

// Orders the wave's LDS accesses on either side of it for every lane. Lanes
// of one wave exchange tiles through LDS (one lane stores what another
// loads); without a fence the compiler may treat LDS as memory private to
// each thread and move or forward a load across another lane's store (it did
// for a store guarded to half the lanes: the other half kept the previous
// tile's value). Wavefront scope: no instruction beyond the ordering.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef __attribute__((address_space(3))) s16x4_t *lds_s4_ptr;

// ds_read_b64_tr_b16 of the 8-byte chunk this lane supplies (see above).
__device__ inline u32x2_t lds_read_tr(const char *p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_ptr)(p)));
}

}  // namespace
}  // namespace ikl
