// FP8 (OCP E4M3) row quantisation shared by the KV append kernel
// (append_kv.hip) and the decode step's append carried by the split reduce
// kernel (paged_decode.hip), so both write the same codes and scales: one
// wave per (token, head) row, lane l holding elements 4l .. 4l + 3
// (head_dim <= 256). The row maximum gives the power-of-two scale
// e4m3_row_scale(amax); the codes are e4m3(x / scale) clamped to +-448,
// rounded to nearest even by v_cvt_pk_fp8_f32.
#pragma once

#include "ikl_common.h"

namespace ikl {

template <typename Tag>
__device__ inline void load4(const char *p, float *x);
template <>
__device__ inline void load4<bf16_tag>(const char *p, float *x) {
  const uint2 w = *reinterpret_cast<const uint2 *>(p);
  x[0] = elem<bf16_tag>::lo(w.x);
  x[1] = elem<bf16_tag>::hi(w.x);
  x[2] = elem<bf16_tag>::lo(w.y);
  x[3] = elem<bf16_tag>::hi(w.y);
}
template <>
__device__ inline void load4<f16_tag>(const char *p, float *x) {
  const uint2 w = *reinterpret_cast<const uint2 *>(p);
  x[0] = elem<f16_tag>::lo(w.x);
  x[1] = elem<f16_tag>::hi(w.x);
  x[2] = elem<f16_tag>::lo(w.y);
  x[3] = elem<f16_tag>::hi(w.y);
}
template <>
__device__ inline void load4<f32_tag>(const char *p, float *x) {
  const float4 w = *reinterpret_cast<const float4 *>(p);
  x[0] = w.x;
  x[1] = w.y;
  x[2] = w.z;
  x[3] = w.w;
}

__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_mov<DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_mov<DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
  return max_xor32(max_xor16(v));
}

// Quantises one row (every lane of the wave calls it; lanes with on == false
// hold no elements) and stores its codes at row + 4 lane and its scale at
// *scale (lane 0).
__device__ inline void store_fp8_row(char *row, float *scale, int lane, bool on, const float *x) {
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = on ? x[i] : 0.f;
  const float amax = wave_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  const float s = e4m3_row_scale(amax);
  float y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] = fminf(fmaxf(v[i] / s, -448.0f), 448.0f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w, true);
  if (on) *reinterpret_cast<int *>(row + 4 * lane) = w;
  if (lane == 0) *scale = s;
}

}  // namespace ikl
