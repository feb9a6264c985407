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

// KV append carried by the split reduce kernel (ikl_paged_decode_step): its
// workgroups also scatter `rows` (token, kv head) rows of new K/V into the
// cache, as ikl_append_kv does: plain copies in 16-byte chunks (16-bit or
// fp32 caches, aligned rows of at most 32 chunks), or (fp8) rows quantised
// into an FP8 cache, one workgroup per (token, head, K or V) row.
struct FusedAppend {
  const char *key;
  const char *value;
  int64_t key_st, key_sh, value_st, value_sh;  // bytes
  const void *slots;
  char *kc;
  char *vc;
  int64_t kc_sb, kc_st, kc_sh, vc_sb, vc_st, vc_sh;  // bytes
  int64_t rows;       // tokens x kv heads; 0 = nothing to append
  int64_t num_slots;  // num_blocks * block_size
  int32_t kv_heads;
  int32_t chunks;     // 16-byte chunks per head row, <= 32
  int32_t block_size;
  int32_t slots_i64;
  // FP8 cache: codes into kc / vc, one fp32 scale per row into k_scale /
  // v_scale [blocks, kv heads, block_size] (strides in elements)
  int32_t fp8;
  int32_t src_dtype;  // enum ikl_dtype of key / value
  int32_t head_dim;
  float *k_scale;
  float *v_scale;
  int64_t s_sb, s_sh;
};

// Fills `f` from the arguments of an ikl_append_kv call: IKL_OK when the
// append can ride on the reduce kernel, 1 when it is valid but must run as
// its own launch (rows not 16-byte aligned or longer than 512 bytes), an
// IKL_E* code when the arguments are invalid (message set).
int prepare_fused_append(const ikl_append_args *a, FusedAppend &f);

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
  // Balanced ("stream-K") split of the MFMA family; sk_waves == 0 selects
  // the fixed partitions above. With sk_waves = W, the global sequence of
  // 16-token tiles — request-major, then (kv head, query group) unit, then
  // position — is cut into W equal runs, one per workgroup; the piece of
  // unit s (= b * units + u) that run w covers lands in partial slot s + w
  // (the pairs (s, w) met along the sequence are ordered in both s and w, so
  // the slots are distinct and each unit's pieces are consecutive).
  int32_t sk_waves;
  int32_t units;           // kv heads x query groups per request
  // Units per workgroup of the unit-parallel balanced split (1 = one-unit
  // runs, as above). With sk_unitw = UW > 1 the sequence is request-major,
  // then unit group (UW consecutive units), then position: the run's
  // workgroup has UW waves, wave i attends unit ug * UW + i, and the piece
  // of (request b, group ug) that run w covers lands in slots ((b * units /
  // UW + ug) + w) * UW + i.
  int32_t sk_unitw;
  // Entries each (request, unit group) segment of the sequence counts
  // before its first tile (0 = none): a run pays a restart at every
  // segment it enters, so runs that cross into a segment get that many
  // fewer tiles. Segment of a request with n > 0 tiles: n + sk_seg_cost
  // entries, tile t at entry sk_seg_cost + t.
  int32_t sk_seg_cost;
  int32_t grid_spread;     // fixed-partition MFMA grid is request-fastest (spread_grid)
  int32_t fixed_waves;     // waves per fixed-partition MFMA workgroup (4, or 8 for 32-head units over FP8)
  int64_t batch;
  int64_t cap_tokens;      // table_width * block_size: positions a table can map
  // FP8 KV cache (MFMA family): E4M3 codes with one fp32 scale per (token,
  // head) row in k_scale / v_scale [blocks, kv heads, block_size].
  int32_t kv_fp8;
  const float *k_scale;
  const float *v_scale;
  int64_t s_sb, s_sh;      // elements
  FusedAppend app;         // rows == 0 unless a decode step fuses its append
};

// Order of the fixed-partition MFMA kernel's grid. Consecutive workgroups
// are dealt round-robin over the 8 XCDs. The default is unit-fastest (unit,
// partition, request). When the units are not a multiple of 8 but units x
// partitions is, that order puts partition i of every request on the same
// XCD (one unit and 8 partitions: XCD = partition), so ragged context
// lengths leave the XCDs of the last partitions idle; the grid is then
// request-fastest (request, unit, partition) with the request rotated by
// the partition index. Grids of at most 256 workgroups keep the default
// (request-fastest measured the same or slower there).
inline bool spread_grid(int64_t units, int64_t parts, int64_t batch) {
  return (units & 7) != 0 && ((units * parts) & 7) == 0 && units * parts * batch > 256 && units <= 65535;
}

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

// ---------------------------------------------------- balanced split helpers
// Context length clamped to [0, cap_tokens] (positions past the table are
// masked anyway, so they are not scheduled).
__device__ inline int64_t clamped_ctx(const AttnParams &p, int64_t b) {
  int64_t c = p.lens_i64 ? load_index<int64_t>(p.lens, b) : load_index<int32_t>(p.lens, b);
  c = c < 0 ? 0 : c;
  return c < p.cap_tokens ? c : p.cap_tokens;
}

// Inclusive prefix sum over the 64 lanes of a wave, in DPP moves (no LDS
// round trips): a Hillis-Steele scan inside each 16-lane row (row_shr 1, 2,
// 4, 8; lanes without a source add 0), then lane 15 of rows 0 and 2 into
// rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3 (row_bcast:31).
__device__ inline int wave_incl_scan(int x, int lane) {
  (void)lane;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
  return x;
}

// Request-level tile totals of the balanced split: tiles of all requests
// before b (*before), of b itself (*own) and of the whole batch (return),
// in request-tile units (multiply by p.units for global tiles). The host
// bounds cap_tokens so that a 64-request chunk sum fits in 32 bits.
// Segment entries of a request with n tiles in the balanced split's
// sequence (see AttnParams::sk_seg_cost).
__device__ inline int seg_len(const AttnParams &p, int n) { return n > 0 ? n + p.sk_seg_cost : 0; }

// Balanced split: segment entries of all requests (returned), of the
// requests before b (*before) and request b's tiles (*own).
__device__ inline int64_t request_tiles(const AttnParams &p, int64_t b, int lane, int64_t *before,
                                        int *own) {
  int64_t base = 0, total = 0;
  *before = 0;
  *own = 0;
  for (int64_t c0 = 0; c0 < p.batch; c0 += 64) {
    const int64_t r = c0 + lane;
    const int n = r < p.batch ? (int)((clamped_ctx(p, r) + 15) >> 4) : 0;
    const int incl = wave_incl_scan(seg_len(p, n), lane);
    if (b >= c0 && b < c0 + 64) {
      const int l = (int)(b - c0);
      *own = __shfl(n, l, 64);
      *before = base + __shfl(incl, l, 64) - seg_len(p, *own);
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  total = base;
  return total;
}

// The run of a balanced split over T tiles and W runs (W <= T),
// [floor(w T / W), floor((w + 1) T / W)), that holds global tile g.
__device__ inline int64_t wave_of_tile(int64_t g, int64_t T, int64_t W) { return ((g + 1) * W - 1) / T; }

// MFMA kernel family (paged_decode_mfma.hip). mfma_supported() tells whether
// a (dtype, head_dim, block_size, group) launch has a compiled MFMA kernel;
// launch_mfma_attention() enqueues it (grid as for the scalar family, or
// p.sk_waves workgroups for the balanced split).
bool mfma_supported(int dtype, int head_dim, int block_size, int group_size);
hipError_t launch_mfma_attention(int dtype, int head_dim, const AttnParams &p, dim3 grid, hipStream_t s);
// Static launch shape of the MFMA family (fixed partitions or balanced split).
struct MfmaShape {
  int tile_tokens, waves_per_workgroup, stages;
};
// fixed_waves: the plan's waves per fixed-partition workgroup (0: the default).
MfmaShape mfma_launch_shape(bool balanced, int group_size, int unitw = 1, int fixed_waves = 0);

// Workgroups of the balanced-split MFMA kernel (for units of `group_size`
// heads; `unitw` units per workgroup for the unit-parallel form) resident at
// once on the current device.
int mfma_streamk_capacity(int dtype, int head_dim, int group_size, bool kv_fp8, int unitw = 1);

// Workgroups of the fixed-partition MFMA kernel (units of `group_size`
// heads) resident at once on the current device.
int mfma_fixed_capacity(int dtype, int head_dim, int group_size, bool kv_fp8);

// Workgroups of its 8-wave form for 32-head units over the FP8 cache
// resident at once on the current device.
int mfma_fixed8_capacity(int dtype, int head_dim);

// Compute units of the current device (256 when no device answers).
int mfma_cu_count();

// Units per workgroup the balanced split uses for `units` units of
// `group_size` heads per request: the largest of 8, 4, 2 dividing `units`
// for units of up to 16 heads, else 1 (one-unit runs).
int mfma_streamk_unitw(int64_t units, int group_size);

}  // namespace ikl
