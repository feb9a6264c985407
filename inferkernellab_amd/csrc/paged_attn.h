// Shared definitions of the paged decode attention kernel families
// (VALU "scalar" kernels in paged_decode.hip, MFMA kernels in
// paged_decode_mfma.hip): launch parameters, softmax constants and small
// device helpers.
#pragma once

#include <math.h>

#include "ikl_common.h"

namespace ikl {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_SENTINEL = -1.0e30f;  // finite "minus infinity" for running maxima
constexpr float RESCALE_LOG2 = 8.0f;      // lazy-rescale threshold (factor 256)

struct AttnParams {
  const char *q;
  int64_t q_sb, q_sh;  // elements
  const char *kc;
  const char *vc;
  int64_t k_sb, k_st, k_sh;  // elements
  int64_t v_sb, v_st, v_sh;  // elements
  const void *tables;
  int64_t t_sb;
  int64_t table_width;
  const void *lens;
  char *out;
  int64_t o_sb, o_sh;  // elements
  float *part_o;       // [B, NP, H, D] fp32 (split only): a partition's heads are contiguous
  float *part_lse;     // [B, NP, H] fp32, log2 domain (split only)
  int64_t num_blocks;
  int32_t num_heads;
  int32_t heads_per_kv;
  int32_t group_size;
  int32_t groups_per_kv;
  int32_t block_size;
  int32_t bs_shift;        // log2(block_size) or -1
  int32_t partition_size;  // tokens per grid.x slot
  int32_t num_parts;       // NP (grid.x)
  int32_t split;           // write partials instead of the output
  int32_t table_i64;
  int32_t lens_i64;
  float scale_log2;        // scale * log2(e)
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 512 zero bytes: masked lanes (positions past the context, or blocks
// outside the cache) load from here, so every tile load is unconditional
// and the wave never branches around its memory operations.
static __device__ __attribute__((aligned(16))) uint32_t g_zero_row[128] = {0};

template <typename Tag>
__device__ inline void store_out_chunk(char *dst, const float *v);

template <>
__device__ inline void store_out_chunk<bf16_tag>(char *dst, const float *v) {
  u32x4 w;
  w.x = elem<bf16_tag>::pack2(v[0], v[1]);
  w.y = elem<bf16_tag>::pack2(v[2], v[3]);
  w.z = elem<bf16_tag>::pack2(v[4], v[5]);
  w.w = elem<bf16_tag>::pack2(v[6], v[7]);
  store16(dst, w);
}
template <>
__device__ inline void store_out_chunk<f16_tag>(char *dst, const float *v) {
  u32x4 w;
  w.x = elem<f16_tag>::pack2(v[0], v[1]);
  w.y = elem<f16_tag>::pack2(v[2], v[3]);
  w.z = elem<f16_tag>::pack2(v[4], v[5]);
  w.w = elem<f16_tag>::pack2(v[6], v[7]);
  store16(dst, w);
}
template <>
__device__ inline void store_out_chunk<f32_tag>(char *dst, const float *v) {
  u32x4 w;
  w.x = __float_as_uint(v[0]);
  w.y = __float_as_uint(v[1]);
  w.z = __float_as_uint(v[2]);
  w.w = __float_as_uint(v[3]);
  store16(dst, w);
}

// Loads the window of 64 block-table entries starting at logical block
// `base`; entries outside the table or naming a block outside the cache
// become -1 (masked).
__device__ inline int load_table_window(const AttnParams &p, int64_t b, int64_t base, int lane) {
  const int64_t lb = base + lane;
  int phys = -1;
  if (lb < p.table_width) {
    const int64_t e = p.table_i64 ? load_index<int64_t>(p.tables, b * p.t_sb + lb)
                                  : load_index<int32_t>(p.tables, b * p.t_sb + lb);
    if (e >= 0 && e < p.num_blocks) phys = (int)e;
  }
  return phys;
}

// MFMA kernel family (paged_decode_mfma.hip). mfma_supported() tells whether
// a (dtype, head_dim, block_size, group) launch has a compiled MFMA kernel;
// launch_mfma_attention() enqueues it (grid as for the scalar family).
bool mfma_supported(int dtype, int head_dim, int block_size, int group_size);
hipError_t launch_mfma_attention(int dtype, int head_dim, const AttnParams &p, dim3 grid, hipStream_t s);

}  // namespace ikl
