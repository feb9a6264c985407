// Paged decode attention for gfx950: VALU ("scalar") kernel family, the
// split-context reduce kernel and the ikl_paged_attention entry point.
//
// Computes, per request b and query head h (kv head = h / (H/Hkv), the map
// of attention.py:9-15 and triton_ops.py:123):
//   out[b,h,:] = softmax(scale * q[b,h,:] . K[b,:ctx_b,kvh,:]) @ V[b,:ctx_b,kvh,:]
// where token p of request b lives at cache[table[b, p / bs], p % bs]
// (cache.py:113-129, 191-200), like paged_reference (attention.py:134-175).
//
// Launch geometry (one wave64 per workgroup; 2 or 4 when up to 4 partitions
// of a request are folded into one unsplit workgroup):
//   grid.x = split-context partition (1 when not split)
//   grid.y = kv_head * groups_per_kv + query_group
//   grid.z = request
// Each workgroup streams the K/V rows of its partition ONCE and applies them
// to all G query heads of its group (G = H/Hkv for GQA; the reference's
// per-head kernel re-reads K/V G times, triton_ops.py:465).
//
// Lane layout: TPT lanes share one token; lane `sub` of the token owns the
// 16-byte chunks c*TPT+sub (c < CPL) of the head_dim row, so the TPT lanes
// of a token read TPT*16 contiguous bytes per load instruction. A wave
// covers ROWS = 64/TPT tokens per row-step and R row-steps per tile.
// QK^T: packed-half dot products (v_dot2_f32_{f16,bf16}) + DPP group sum.
// Softmax: every token row keeps its own online (max, sum, acc) in the
// log2 domain, rescaled lazily (only when the max grows by more than
// RESCALE_LOG2); rows merge once at the end of the partition.
// PV: fp32 FMAs on converted V.
#include <math.h>

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <mutex>
#include <string>

#include "fp8_row.h"
#include "ikl_common.h"
#include "paged_attn.h"

namespace ikl {
namespace {

constexpr int pow2_divisor(int n, int cap) {
  int t = 1;
  while (t * 2 <= cap && n % (t * 2) == 0) t *= 2;
  return t;
}

constexpr int cmin(int a, int b) { return a < b ? a : b; }

// Lanes per token: at most 8 for groups of <= 4 heads, 16 for groups of 8
// and for fp32 4-head groups of 128 dims (more lanes per token keep the
// per-lane query and accumulator registers of a large group in budget: the
// fp32 hd128 4-head kernel goes from 256 VGPRs at one wave per SIMD to 172 at
// two, GQA 32/8 B32 x U[1024, 4096] 149.7 -> 139.9 us; fp32 hd64 4-head
// groups, 2-head groups and one head stay at 8, where 16 measured slower or
// equal); 16-byte K (and V) loads per lane per tile.
constexpr int TPT_CAP_SMALL_GROUP = 8;
constexpr int TPT_CAP_LARGE_GROUP = 16;
constexpr int LOADS_PER_LANE = 4;

template <typename Tag, int D, int G>
struct ScalarCfg {
  static constexpr int EB = elem<Tag>::bytes;
  static constexpr int VEC = 16 / EB;              // elements per 16-byte chunk
  static constexpr int NCHUNK = D / VEC;           // chunks per head_dim row
  static_assert(D % VEC == 0, "head_dim must be a multiple of a 16-byte chunk");
  static constexpr int TPT =
      pow2_divisor(NCHUNK, (G >= 8 || (EB == 4 && D >= 128 && G >= 4)) ? TPT_CAP_LARGE_GROUP : TPT_CAP_SMALL_GROUP);
  static constexpr int CPL = NCHUNK / TPT;         // chunks per lane
  static constexpr int LD = CPL * VEC;             // dims per lane
  static constexpr int ROWS = 64 / TPT;            // tokens per row-step
  // Row-steps per tile: LOADS_PER_LANE chunks of K per lane, and never
  // more than 64 tokens so one 64-entry block-table window covers a tile.
  static constexpr int R0 = CPL >= LOADS_PER_LANE ? 1 : LOADS_PER_LANE / CPL;
  static constexpr int R = cmin(R0, 64 / ROWS);
  static constexpr int TI = ROWS * R;              // tokens per tile (<= 64)
  static_assert(TI <= 64, "a tile must fit one table window");
};

// W waves per workgroup share one partition: wave w takes tiles
// [w n / W, (w + 1) n / W) of its n tiles, and the waves' (m, l, o) merge in
// LDS before wave 0 writes, so a launch that needs W times the waves of its
// (partition, unit, request) count gets them without W times the partials.
template <typename Tag, int D, int G, int W>
__global__ __launch_bounds__(64 * W) void paged_decode_scalar_kernel(const AttnParams p) {
  using C = ScalarCfg<Tag, D, G>;
  constexpr int TPT = C::TPT, CPL = C::CPL, LD = C::LD, ROWS = C::ROWS, R = C::R, TI = C::TI;
  constexpr int VEC = C::VEC, EB = C::EB;
  constexpr bool F32 = (EB == 4);

  const int lane = threadIdx.x & 63;
  const int wave = W > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
  const int row = lane / TPT;
  const int sub = lane % TPT;
  // Grid (partition, unit, request), partition fastest. Consecutive
  // workgroups are dealt round-robin over the 8 XCDs, so with a multiple of
  // 8 partitions per request the XCD would be the partition index for every
  // request, and ragged context lengths would leave the XCDs of the last,
  // mostly empty partitions idle. The partition index is then rotated by
  // (unit + request) % 8, which deals each request's partitions over all 8
  // (MHA 32 hd128 bf16 B32 x U[1024, 4096]: 304 -> 239 us for the whole
  // operation; fp32 GQA 32/8 B32 x U[1024, 4096]: 158 -> 147 us; uniform
  // batches unchanged).
  int part = blockIdx.x;
  if ((gridDim.x & 7u) == 0u) {
    part += (int)((blockIdx.y + blockIdx.z) & 7u);
    if (part >= (int)gridDim.x) part -= (int)gridDim.x;
  }
  const int kvh = blockIdx.y / p.groups_per_kv;
  const int qg = blockIdx.y % p.groups_per_kv;
  const int64_t b = blockIdx.z;

  const int64_t ctx = p.lens_i64 ? load_index<int64_t>(p.lens, b) : load_index<int32_t>(p.lens, b);
  const int64_t part_start = (int64_t)part * p.partition_size;
  if (part > 0 && part_start >= ctx) return;  // no tokens for this partition
  const int64_t part_end = ctx < part_start + p.partition_size ? ctx : part_start + p.partition_size;
  const int wg_tiles = part_end > part_start ? (int)((part_end - part_start + TI - 1) / TI) : 0;
  // this wave's run of the partition's tiles: positions [w_start, w_end)
  const int t_lo = wave * wg_tiles / W, t_hi = (wave + 1) * wg_tiles / W;
  const int n_tiles = t_hi - t_lo;
  const int64_t w_start = part_start + (int64_t)t_lo * TI;
  const int64_t w_end = part_end < part_start + (int64_t)t_hi * TI ? part_end : part_start + (int64_t)t_hi * TI;

  // ---- query heads of this group, kept packed (two halves per word)
  const int head0 = qg * p.group_size;  // index among the kv head's query heads
  uint32_t qw[G][CPL][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const bool hv = (g < p.group_size) && (head0 + g < p.heads_per_kv);
    const int64_t hq = (int64_t)kvh * p.heads_per_kv + head0 + g;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (hv) v = load16(p.q + (b * p.q_sb + hq * p.q_sh + (int64_t)(c * TPT + sub) * VEC) * EB);
      qw[g][c][0] = v.x;
      qw[g][c][1] = v.y;
      qw[g][c][2] = v.z;
      qw[g][c][3] = v.w;
    }
  }

  float m[G], l[G], acc[G][LD];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = NEG_SENTINEL;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < LD; ++i) acc[g][i] = 0.f;
  }

  const char *kbase = p.kc + (int64_t)kvh * p.k_sh * EB;
  const char *vbase = p.vc + (int64_t)kvh * p.v_sh * EB;
  const char *zero_row = reinterpret_cast<const char *>(g_zero_row);
  const int bs = p.block_size;
  const int lane_off = sub * 16;

  // Block-table window: lane j holds table[b, win_base + j] (or -1).
  int64_t win_base = p.bs_shift >= 0 ? (w_start >> p.bs_shift) : w_start / bs;
  int win = load_table_window(p, b, win_base, lane);

  // Issues the K/V loads of tile `t` (unconditionally: masked lanes read
  // the zero row) and returns the lane's valid-token mask.
  auto issue_tile = [&](int t, u32x4 (&kr)[R][CPL], u32x4 (&vr)[R][CPL]) -> uint32_t {
    const int64_t tile_base = w_start + (int64_t)t * TI;
    const int64_t last = tile_base + TI - 1;
    const int64_t lb_hi = p.bs_shift >= 0 ? (last >> p.bs_shift) : last / bs;
    if (lb_hi >= win_base + 64) {  // wave-uniform: move the window forward
      win_base = p.bs_shift >= 0 ? (tile_base >> p.bs_shift) : tile_base / bs;
      win = load_table_window(p, b, win_base, lane);
    }
    uint32_t valid = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t pos = tile_base + r * ROWS + row;
      const int64_t lb = p.bs_shift >= 0 ? (pos >> p.bs_shift) : pos / bs;
      const int off = (int)(pos - lb * bs);
      const int idx = (int)(lb - win_base);  // 0..63 by construction of the window
      const int phys = __builtin_amdgcn_ds_bpermute((idx & 63) * 4, win);
      const bool ok = (pos < w_end) && (phys >= 0);
      valid |= (ok ? 1u : 0u) << r;
      const char *krow = ok ? kbase + ((int64_t)phys * p.k_sb + (int64_t)off * p.k_st) * EB : zero_row;
      const char *vrow = ok ? vbase + ((int64_t)phys * p.v_sb + (int64_t)off * p.v_st) * EB : zero_row;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        kr[r][c] = load16_stream(krow + c * TPT * 16 + lane_off);
        vr[r][c] = load16_stream(vrow + c * TPT * 16 + lane_off);
      }
    }
    return valid;
  };

  auto compute_tile = [&](const u32x4 (&kr)[R][CPL], const u32x4 (&vr)[R][CPL], uint32_t valid) {
    float s[R][G];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t kw = u32x4_at(kr[r][c], w);
            if constexpr (F32) {
              d = fmaf(__uint_as_float(kw), __uint_as_float(qw[g][c][w]), d);
            } else {
              d = elem<Tag>::dot2(kw, qw[g][c][w], d);
            }
          }
        }
        d = group_sum<TPT>(d) * p.scale_log2;
        s[r][g] = ((valid >> r) & 1u) ? d : -INFINITY;
      }
    }
    // Lazy online-softmax rescale: only when a row's max grows by more
    // than RESCALE_LOG2 (results are unchanged; weights stay <= 2^8).
    bool need_any = false;
    float tmax[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float t = s[0][g];
#pragma unroll
      for (int r = 1; r < R; ++r) t = fmaxf(t, s[r][g]);
      tmax[g] = t;
      need_any |= t > m[g] + RESCALE_LOG2;
    }
    if (__builtin_amdgcn_ballot_w64(need_any) != 0ull) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const bool need = tmax[g] > m[g] + RESCALE_LOG2;
        const float alpha = need ? fast_exp2(m[g] - tmax[g]) : 1.f;
        m[g] = need ? tmax[g] : m[g];
        l[g] *= alpha;
#pragma unroll
        for (int i = 0; i < LD; ++i) acc[g][i] *= alpha;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float pr[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        pr[g] = fast_exp2(s[r][g] - m[g]);
        l[g] += pr[g];
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t vw = u32x4_at(vr[r][c], w);
          if constexpr (F32) {
            const float v0 = __uint_as_float(vw);
#pragma unroll
            for (int g = 0; g < G; ++g) acc[g][c * VEC + w] = fmaf(pr[g], v0, acc[g][c * VEC + w]);
          } else {
            const float v0 = elem<Tag>::lo(vw);
            const float v1 = elem<Tag>::hi(vw);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              acc[g][c * VEC + 2 * w] = fmaf(pr[g], v0, acc[g][c * VEC + 2 * w]);
              acc[g][c * VEC + 2 * w + 1] = fmaf(pr[g], v1, acc[g][c * VEC + 2 * w + 1]);
            }
          }
        }
      }
    }
  };

  // ---- software pipeline, two register buffers: the loads of the next
  // tile are in flight while the current one computes. Loads past the last
  // tile are fully masked (zero row) so the issue pattern is straight-line.
  u32x4 ka[R][CPL], va[R][CPL], kb[R][CPL], vb[R][CPL];
  uint32_t valid_a = issue_tile(0, ka, va);
  for (int t = 0; t < n_tiles; t += 2) {
    const uint32_t valid_b = issue_tile(t + 1, kb, vb);
    compute_tile(ka, va, valid_a);
    valid_a = issue_tile(t + 2, ka, va);
    if (t + 1 < n_tiles) compute_tile(kb, vb, valid_b);
  }

  // ---- merge the token rows of the wave (same sub, different row)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = m[g];
#pragma unroll
    for (int mask = TPT; mask < 64; mask <<= 1) mx = fmaxf(mx, shfl_xor_f(mx, mask));
    const float w = fast_exp2(m[g] - mx);
    l[g] *= w;
#pragma unroll
    for (int mask = TPT; mask < 64; mask <<= 1) l[g] += shfl_xor_f(l[g], mask);
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      float a = acc[g][i] * w;
#pragma unroll
      for (int mask = TPT; mask < 64; mask <<= 1) a += shfl_xor_f(a, mask);
      acc[g][i] = a;
    }
    m[g] = mx;
  }

  // ---- merge the workgroup's waves; wave 0 writes
  if constexpr (W > 1) {
    __shared__ float lds_ml[W][2][G];
    __shared__ float lds_o[W][G][D];
    if (row == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int c = 0; c < CPL; ++c)
#pragma unroll
          for (int e = 0; e < VEC; ++e) lds_o[wave][g][(c * TPT + sub) * VEC + e] = acc[g][c * VEC + e];
        if (sub == 0) {
          lds_ml[wave][0][g] = m[g];
          lds_ml[wave][1][g] = l[g];
        }
      }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = lds_ml[0][0][g];
#pragma unroll
      for (int w = 1; w < W; ++w) mx = fmaxf(mx, lds_ml[w][0][g]);
      float f[W];
      float lt = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        f[w] = fast_exp2(lds_ml[w][0][g] - mx);
        lt = fmaf(lds_ml[w][1][g], f[w], lt);
      }
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          float a = 0.f;
#pragma unroll
          for (int w = 0; w < W; ++w) a = fmaf(lds_o[w][g][(c * TPT + sub) * VEC + e], f[w], a);
          acc[g][c * VEC + e] = a;
        }
      m[g] = mx;
      l[g] = lt;
    }
  }

  // ---- write: row r writes the heads g with g % ROWS == r
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if ((g % ROWS) != row) continue;
    if (!(g < p.group_size && head0 + g < p.heads_per_kv)) continue;
    const int64_t hq = (int64_t)kvh * p.heads_per_kv + head0 + g;
    if (p.split) {
      const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
      const int64_t prow = (b * p.num_parts + part) * p.num_heads + hq;
      float *po = p.part_o + prow * D;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
          u32x4 w;
          w.x = __float_as_uint(acc[g][c * VEC + e] * inv);
          w.y = __float_as_uint(acc[g][c * VEC + e + 1] * inv);
          w.z = __float_as_uint(acc[g][c * VEC + e + 2] * inv);
          w.w = __float_as_uint(acc[g][c * VEC + e + 3] * inv);
          store16(po + (c * TPT + sub) * VEC + e, w);
        }
      }
      if (sub == 0) p.part_lse[prow] = l[g] > 0.f ? m[g] + log2f(l[g]) : -INFINITY;
    } else {
      const float inv = 1.f / l[g];  // l == 0 (no valid token) gives NaN, like the reference
      char *dst = p.out + (b * p.o_sb + hq * p.o_sh) * EB;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        float v[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = acc[g][c * VEC + e] * inv;
        store_out_chunk<Tag>(dst + (int64_t)(c * TPT + sub) * 16, v);
      }
    }
  }
}

// Fused KV append of a decode step: the reduce workgroups, flattened to
// wg in [0, nwg), take rows (token t, kv head h) of the new K/V; a pass
// covers R = 64 / (2 chunks) rows per workgroup, and lane l copies K chunk
// l % (2 chunks) (V chunk when >= chunks) of row wg R + l / (2 chunks). The
// loads are issued when the kernel starts and the stores placed after the
// partials are read, so the copy's round trip overlaps the reduce's.
struct FusedRow {
  v4u32 data;
  int64_t slot, t;
  int h, c;
  bool on, is_v;
};

__device__ inline FusedRow fused_append_load(const FusedAppend &f, int64_t row0, int lane) {
  FusedRow r{};
  const int per_row = 2 * f.chunks;
  const int sub = lane % per_row;
  const int64_t row = row0 + lane / per_row;
  r.on = lane / per_row < 64 / per_row && row < f.rows;
  if (!r.on) return r;
  r.is_v = sub >= f.chunks;
  r.c = r.is_v ? sub - f.chunks : sub;
  r.t = row / f.kv_heads;
  r.h = (int)(row - r.t * f.kv_heads);
  r.slot = f.slots_i64 ? load_index<int64_t>(f.slots, r.t) : load_index<int32_t>(f.slots, r.t);
  const char *src = r.is_v ? f.value + r.t * f.value_st + r.h * f.value_sh : f.key + r.t * f.key_st + r.h * f.key_sh;
  r.data = load16v_global(src + r.c * 16);
  return r;
}

// FP8 cache: row r of the 2 x rows (token, head, K or V) rows, one wave per
// row, loaded when the kernel starts and quantised after the partials are
// read (store_fp8_row, as ikl_append_kv writes it).
struct Fp8FusedRow {
  float x[4];
  int64_t slot, t;
  int h, which;
  bool valid, on;
};

template <typename Tag>
__device__ inline Fp8FusedRow fused_fp8_load(const FusedAppend &f, int64_t r, int lane) {
  constexpr int EB = elem<Tag>::bytes;
  Fp8FusedRow row{};
  row.valid = r < 2 * f.rows;
  if (!row.valid) return row;
  row.which = (int)(r & 1);
  const int64_t tr = r >> 1;
  row.t = tr / f.kv_heads;
  row.h = (int)(tr - row.t * f.kv_heads);
  row.on = 4 * lane < f.head_dim;
  const char *src = row.which ? f.value + row.t * f.value_st + row.h * f.value_sh
                              : f.key + row.t * f.key_st + row.h * f.key_sh;
  load4<Tag>(src + (row.on ? 4 * lane * EB : 0), row.x);  // lanes past the row re-read its start
  row.slot = f.slots_i64 ? load_index<int64_t>(f.slots, row.t) : load_index<int32_t>(f.slots, row.t);
  return row;
}

// Every lane of the wave calls it (the row and its slot are the wave's).
__device__ inline void fused_fp8_store(const FusedAppend &f, const Fp8FusedRow &r, int lane) {
  if (!r.valid || r.slot < 0 || r.slot >= f.num_slots) return;  // slots outside the cache are skipped
  const int64_t blk = r.slot / f.block_size, off = r.slot - blk * f.block_size;
  char *dst = r.which ? f.vc + blk * f.vc_sb + off * f.vc_st + r.h * f.vc_sh
                      : f.kc + blk * f.kc_sb + off * f.kc_st + r.h * f.kc_sh;
  float *scale = (r.which ? f.v_scale : f.k_scale) + blk * f.s_sb + r.h * f.s_sh + off;
  store_fp8_row(dst, scale, lane, r.on, r.x);
}

__device__ inline void fused_append_store(const FusedAppend &f, const FusedRow &r) {
  if (!r.on || r.slot < 0 || r.slot >= f.num_slots) return;  // slots outside the cache are skipped
  const int64_t blk = r.slot / f.block_size, off = r.slot - blk * f.block_size;
  char *dst = r.is_v ? f.vc + blk * f.vc_sb + off * f.vc_st + r.h * f.vc_sh
                     : f.kc + blk * f.kc_sb + off * f.kc_st + r.h * f.kc_sh;
  *reinterpret_cast<v4u32 *>(dst + r.c * 16) = r.data;
}

// Combines the split partials of one (request, head):
//   out = sum_p 2^(lse_p - M) o_p / sum_p 2^(lse_p - M),  M = max_p lse_p.
// Lanes split into GROUPS groups of D/4 lanes; group j takes partitions
// j, j+GROUPS, ... with 16-byte loads (the log-sum-exp and the row of a
// partition are loaded together, several partitions in flight), keeping its
// own running maximum; the groups then combine through LDS.
template <typename Tag, int D>
__global__ __launch_bounds__(64) void paged_decode_reduce_kernel(const AttnParams p) {
  constexpr int EB = elem<Tag>::bytes;
  constexpr int CH = D / 4;           // float4 chunks per row
  constexpr int GROUPS = 64 / CH;     // partition groups
  __shared__ float4 part_sum[GROUPS][CH];
  __shared__ float part_z[GROUPS], part_m[GROUPS];
  const int lane = threadIdx.x;
  const int64_t hq = blockIdx.x;
  const int64_t b = blockIdx.y;
  // fused append: first pass loaded now, stored once the partials are in
  const int64_t wg = b * gridDim.x + hq, nwg = (int64_t)gridDim.x * gridDim.y;
  const bool app8 = p.app.rows > 0 && p.app.fp8;
  const int64_t app_rpp = p.app.rows > 0 && !app8 ? 64 / (2 * p.app.chunks) : 0;
  const FusedRow first_row = app_rpp > 0 ? fused_append_load(p.app, wg * app_rpp, lane) : FusedRow{};
  const Fp8FusedRow first_row8 = app8 ? fused_fp8_load<Tag>(p.app, wg, lane) : Fp8FusedRow{};
  int np;
  int64_t prow, pstride;
  if (p.sk_waves > 0) {
    // balanced split: the pieces of unit u (group ug = u / UW, member i) sit
    // in consecutive slots (b NUG + ug + w) UW + i for the runs w that cover
    // its group's tiles (UW = 1: one-unit runs); rows slot * group_size + head.
    int64_t before;
    int own;
    const int64_t total = request_tiles(p, b, lane, &before, &own);
    const int64_t UW = p.sk_unitw;
    const int64_t NUG = p.units / UW;
    const int64_t T = NUG * total;
    const int64_t W = (int64_t)p.sk_waves < T ? (int64_t)p.sk_waves : T;
    const int kvh = (int)(hq / p.heads_per_kv), r = (int)(hq % p.heads_per_kv);
    const int64_t u = (int64_t)kvh * p.groups_per_kv + r / p.group_size;
    const int64_t ug = u / UW, ui = u - ug * UW;
    const int64_t s = NUG * before + ug * seg_len(p, own) + p.sk_seg_cost;  // the group's first tile's entry
    const int64_t w_lo = own > 0 ? wave_of_tile(s, T, W) : 0;
    const int64_t w_hi = own > 0 ? wave_of_tile(s + own - 1, T, W) : -1;
    np = (int)(w_hi - w_lo + 1);
    prow = ((b * NUG + ug + w_lo) * UW + ui) * p.group_size + r % p.group_size;
    pstride = UW * p.group_size;
  } else {
    const int64_t ctx = p.lens_i64 ? load_index<int64_t>(p.lens, b) : load_index<int32_t>(p.lens, b);
    np = ctx > 0 ? (int)((ctx + p.partition_size - 1) / p.partition_size) : 0;
    if (np > p.num_parts) np = p.num_parts;
    // partial rows of this (request, head): (b * NP + i) * H + hq
    prow = b * p.num_parts * p.num_heads + hq;
    pstride = p.num_heads;
  }
  // One pass over the partials: each group keeps its own running maximum
  // (online softmax over its partitions), and the groups meet in LDS. The
  // partials load in batches of GROUPS * K (16) with their loads issued
  // together: indices past np read partial np - 1 again and weigh 0, so a
  // head with up to 16 partials waits on one memory round trip (a loop of
  // 4-way unrolled steps plus a remainder took two or three for the 9 or so
  // of a balanced split).
  constexpr int K = GROUPS >= 16 ? 1 : 16 / GROUPS;
  const int grp = lane / CH;
  const int ch = lane % CH;
  if (grp < GROUPS) {
    float4 a = {0.f, 0.f, 0.f, 0.f};
    float z = 0.f, m = -INFINITY;
    for (int i0 = grp; i0 < np; i0 += GROUPS * K) {
      float lk[K];
      float4 ok[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int i = i0 + k * GROUPS;
        const int64_t row = prow + (int64_t)(i < np ? i : np - 1) * pstride;
        lk[k] = p.part_lse[row];
        ok[k] = reinterpret_cast<const float4 *>(p.part_o + row * D)[ch];
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const float l = i0 + k * GROUPS < np ? lk[k] : -INFINITY;
        const float4 o = ok[k];
        const float mn = fmaxf(m, l);
        const float c = mn == -INFINITY ? 1.f : fast_exp2(m - mn);  // rescale of what is summed so far
        const float w = mn == -INFINITY ? 0.f : fast_exp2(l - mn);  // empty partitions (-inf) weigh 0
        z = fmaf(z, c, w);
        a.x = fmaf(w, o.x, a.x * c);
        a.y = fmaf(w, o.y, a.y * c);
        a.z = fmaf(w, o.z, a.z * c);
        a.w = fmaf(w, o.w, a.w * c);
        m = mn;
      }
    }
    part_sum[grp][ch] = a;
    if (ch == 0) {
      part_z[grp] = z;
      part_m[grp] = m;
    }
  }
  if (app8) {
    fused_fp8_store(p.app, first_row8, lane);
    for (int64_t r = wg + nwg; r < 2 * p.app.rows; r += nwg) fused_fp8_store(p.app, fused_fp8_load<Tag>(p.app, r, lane), lane);
  } else if (p.app.rows > 0) {
    fused_append_store(p.app, first_row);
    for (int64_t row0 = (wg + nwg) * app_rpp; row0 < p.app.rows; row0 += nwg * app_rpp)
      fused_append_store(p.app, fused_append_load(p.app, row0, lane));
  }
  __syncthreads();
  if (lane >= CH) return;
  float mx = part_m[0];
#pragma unroll
  for (int j = 1; j < GROUPS; ++j) mx = fmaxf(mx, part_m[j]);
  float4 t = {0.f, 0.f, 0.f, 0.f};
  float zt = 0.f;
#pragma unroll
  for (int j = 0; j < GROUPS; ++j) {
    const float f = part_m[j] == -INFINITY ? 0.f : fast_exp2(part_m[j] - mx);
    const float4 u = part_sum[j][lane];
    t.x = fmaf(f, u.x, t.x);
    t.y = fmaf(f, u.y, t.y);
    t.z = fmaf(f, u.z, t.z);
    t.w = fmaf(f, u.w, t.w);
    zt = fmaf(f, part_z[j], zt);
  }
  const float inv = 1.f / zt;
  const float v[4] = {t.x * inv, t.y * inv, t.z * inv, t.w * inv};
  char *dst = p.out + (b * p.o_sb + hq * p.o_sh) * EB + (int64_t)lane * 4 * EB;
  if constexpr (EB == 4) {
    store16(dst, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                       __float_as_uint(v[3])});
  } else {
    uint2 w;
    w.x = elem<Tag>::pack2(v[0], v[1]);
    w.y = elem<Tag>::pack2(v[2], v[3]);
    *reinterpret_cast<uint2 *>(dst) = w;
  }
}

// ------------------------------------------------------------ host side

struct Plan {
  int eb = 0;
  int path = IKL_PATH_SCALAR_GROUPED;
  int heads_per_kv = 0;
  int group_size = 0;
  int gmax = 0;
  int groups_per_kv = 0;
  int partition = 0;  // tokens per grid.x slot
  int num_parts = 1;
  bool split = false;
  int sk_waves = 0;  // balanced split (MFMA family): runs (workgroups) sharing the batch's tiles
  int sk_unitw = 1;  // units per balanced-split workgroup (unit-parallel form when > 1)
  int sk_seg_cost = 0;  // leading entries per (request, unit group) segment of the balanced split
  int64_t units = 0;  // kv heads x query groups per request
  int64_t ws_o_bytes = 0;
  int64_t ws_bytes = 0;
  bool kv_fp8 = false;  // E4M3 cache with per-row scales (MFMA family only)
  int scalar_waves = 1;  // waves per workgroup of the VALU family (1, 2 or 4)
  int fixed_waves = 4;   // waves per fixed-partition MFMA workgroup (8: 32-head units over the FP8 cache)
};

int elem_bytes(int dtype) {
  switch (dtype) {
    case IKL_F16:
    case IKL_BF16: return 2;
    case IKL_F32: return 4;
    default: return 0;
  }
}

bool head_dim_supported(int d) { return d == 16 || d == 32 || d == 64 || d == 96 || d == 128; }

int next_pow2(int x) {
  int v = 1;
  while (v < x) v *= 2;
  return v;
}

constexpr int SCALAR_MAX_GROUP = 8;
constexpr int MFMA_MAX_GROUP = 32;

// Kernel family of a launch shape: one query head per KV head -> the
// one-head scalar kernel; fp16/bf16 with an MFMA-compatible head_dim and
// block size -> matrix cores; everything else -> the grouped scalar kernel.
int select_path(int dtype, int head_dim, int block_size, int heads_per_kv, int query_group_size) {
  if (heads_per_kv == 1) return IKL_PATH_MHA_FALLBACK;
  int gs = query_group_size <= 0 || query_group_size > heads_per_kv ? heads_per_kv : query_group_size;
  if (gs > MFMA_MAX_GROUP) gs = MFMA_MAX_GROUP;
  if (mfma_supported(dtype, head_dim, block_size, gs)) return IKL_PATH_MFMA_GROUPED;
  return IKL_PATH_SCALAR_GROUPED;
}

// fold_waves: let the automatic VALU split fold up to 4 partitions of a
// request into one unsplit multi-wave workgroup (false for the decode step's
// alternative plan, which keeps the split so the reduce carries the append).
int make_plan(const ikl_paged_attention_args *a, Plan &pl, bool fold_waves = true) {
  if (!a) return fail(IKL_EINVAL, "attention: null argument struct");
  pl.eb = elem_bytes(a->dtype);
  if (!pl.eb) return fail(IKL_EINVAL, "attention: unsupported dtype");
  if (a->batch <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0)
    return fail(IKL_EINVAL, "query dimensions must be positive");
  if (a->num_heads % a->num_kv_heads != 0)
    return fail(IKL_EINVAL, "num_heads must be divisible by num_kv_heads");
  if (a->block_size <= 0 || a->num_blocks <= 0)
    return fail(IKL_EINVAL, "cache dimensions must be positive");
  if (a->num_blocks > 0x7fffffffLL) return fail(IKL_EINVAL, "num_blocks must fit in int32");
  if (a->table_width <= 0) return fail(IKL_EINVAL, "block_tables must contain at least one logical block");
  if (a->table_type != IKL_I32 && a->table_type != IKL_I64)
    return fail(IKL_EINVAL, "block_tables must use int32 or int64");
  if (a->lens_type != IKL_I32 && a->lens_type != IKL_I64)
    return fail(IKL_EINVAL, "context_lens must use int32 or int64");
  if (!head_dim_supported(a->head_dim))
    return fail(IKL_EUNSUPPORTED, "head_dim " + std::to_string(a->head_dim) +
                                      " is not compiled (supported: 16, 32, 64, 96, 128)");
  if (a->batch > 65535) return fail(IKL_EINVAL, "batch exceeds the grid limit (65535)");
  if (a->query_group_size < 0) return fail(IKL_EINVAL, "query_group_size must be non-negative");
  pl.heads_per_kv = a->num_heads / a->num_kv_heads;
  const int requested_gs = a->query_group_size;
  if (a->cache_dtype != 0 && a->cache_dtype != a->dtype && a->cache_dtype != IKL_FP8_E4M3)
    return fail(IKL_EINVAL, "attention: cache_dtype must be 0, the query dtype or IKL_FP8_E4M3");
  pl.kv_fp8 = a->cache_dtype == IKL_FP8_E4M3;
  if (pl.kv_fp8) {
    // the FP8 cache is read by the MFMA family only (any heads per KV head)
    if (a->path != -1 && a->path != IKL_PATH_MFMA_GROUPED)
      return fail(IKL_EUNSUPPORTED, "attention: the FP8 cache is read by the MFMA family only");
    pl.path = IKL_PATH_MFMA_GROUPED;
  } else if (a->path == -1) {
    pl.path = select_path(a->dtype, a->head_dim, a->block_size, pl.heads_per_kv, requested_gs);
    // partition_size -2 asks for the balanced split, which the MFMA family
    // runs: an MHA launch left to the library moves there from the per-head
    // kernel when the family supports its shape. On ragged batches the
    // balanced split is slightly ahead of the per-head kernel's fixed
    // partitions (whole operation, MALL flushed: MHA 32 hd128 bf16 B32 x
    // U[1024, 4096] 239 -> 228 us); on uniform ones the per-head kernel,
    // which partition_size 0 keeps, is 6-10 % faster.
    //
    // Small MHA launches move there too: with at most 32 MiB of K/V at the
    // longest context they are latency-bound, and the MFMA kernel's 4-wave
    // workgroups (a partition's tiles split over 4 waves, merged in LDS)
    // take fewer dependent steps than the per-head kernel's one wave.
    // Whole operation, MALL flushed, MHA 32 hd64 fp16: B1 x 128 16.1 ->
    // 13.6 us, B4 x 128 16.0 -> 13.4, B1 x 512 17.6 -> 15.2, B4 x 512 18.0
    // -> 17.0, B16 x 128 16.3 -> 15.5; at 64 MiB and above the per-head
    // kernel is as fast or faster (B16 x 512 25.3 vs 25.6, B4 x 2048 25.6 vs
    // 27.1, B16 x 2048 62.3 vs 69.8).
    if (pl.path == IKL_PATH_MHA_FALLBACK && mfma_supported(a->dtype, a->head_dim, a->block_size, 1)) {
      const int64_t cap_tokens = a->table_width * (int64_t)a->block_size;
      const int64_t ctx = a->max_context_len > 0 ? std::min<int64_t>(a->max_context_len, cap_tokens) : cap_tokens;
      const double kv_bytes = (double)a->batch * a->num_kv_heads * ctx * a->head_dim * 2.0 * pl.eb;
      if (a->partition_size == -2 || kv_bytes <= 32.0 * (1 << 20)) pl.path = IKL_PATH_MFMA_GROUPED;
    }
  } else if (a->path == IKL_PATH_MHA_FALLBACK || a->path == IKL_PATH_SCALAR_GROUPED) {
    pl.path = pl.heads_per_kv == 1 ? IKL_PATH_MHA_FALLBACK : a->path;
  } else if (a->path == IKL_PATH_MFMA_GROUPED) {
    pl.path = IKL_PATH_MFMA_GROUPED;
  } else {
    return fail(IKL_EINVAL, "attention: unknown kernel path");
  }
  int gs = requested_gs == 0 || requested_gs > pl.heads_per_kv ? pl.heads_per_kv : requested_gs;
  if (pl.path == IKL_PATH_MHA_FALLBACK) gs = 1;
  const int cap_gs = pl.path == IKL_PATH_MFMA_GROUPED ? MFMA_MAX_GROUP : SCALAR_MAX_GROUP;
  if (gs > cap_gs) gs = cap_gs;
  if (pl.path == IKL_PATH_MFMA_GROUPED && !mfma_supported(a->dtype, a->head_dim, a->block_size, gs))
    return fail(IKL_EUNSUPPORTED, pl.kv_fp8 ? "the FP8 cache needs fp16/bf16 queries, head_dim 32/64/96/128 and "
                                              "a block size multiple of 16"
                                            : "MFMA path needs fp16/bf16, head_dim 32/64/96/128 and a block size "
                                              "multiple of 16");
  pl.group_size = gs;
  pl.gmax = next_pow2(gs);
  pl.groups_per_kv = (pl.heads_per_kv + gs - 1) / gs;

  // Split-context partitions.
  const int64_t cap = a->table_width * (int64_t)a->block_size;
  int64_t maxctx = a->max_context_len > 0 ? std::min<int64_t>(a->max_context_len, cap) : cap;
  pl.units = (int64_t)a->num_kv_heads * pl.groups_per_kv;
  const int64_t units = a->batch * pl.units;

  // Balanced split runs (workgroups of SKW waves): at least SK_MIN_TILES
  // tiles per wave at the longest context (a small batch runs fewer, longer
  // waves, not one tile each; e.g. MQA 32/1 hd64 B16 x 2048: 24.9 -> 16.5 us
  // going from 1 to 4), capped by the resident capacity.
  constexpr int64_t SK_MIN_TILES = 4;
  // The balanced split on the MFMA family (one run of ~T/W tiles per
  // resident wave): asked for with partition_size = -2, and picked
  // automatically above SK_MIN_BATCH_TILES tiles at the longest context.
  // Below that, fixed partitions (4-wave workgroups merging in LDS, one
  // partial per partition) measured faster on the whole operation (split
  // kernel + reduce, MALL flushed): MQA 32/1 hd128 B64 x U[1024, 4096]
  // 35.8 -> 31.5 us, GQA 32/8 hd128 B64 x 512 35.9 -> 30.2 us, B32 x 2048
  // 58.1 -> 56.3 us, the Llama decode shape (16/4, B16 x 544) 16.7 -> 15.0
  // us; above it the balanced split wins (B32 x U[4096, 8192] 145 vs 168
  // us, B16 x U[4096, 8192] 77 vs 87 us). Its in-kernel sums need a
  // 64-request chunk of tile counts to fit in 32 bits (cap < 2^29 tokens)
  // and (T + 1) * W to fit in 63 bits.
  constexpr int64_t SK_MIN_BATCH_TILES = 32768;
  constexpr int SK_SEG_COST_32 = 16, SK_SEG_COST_ONE = 4, SK_SEG_COST_UNITS = 1;
  if (a->partition_size == -2 && pl.path != IKL_PATH_MFMA_GROUPED)
    return fail(IKL_EUNSUPPORTED, "partition_size -2 (the balanced split) needs the MFMA kernel family");
  const int64_t t_max = units * ((maxctx + 15) / 16);
  // 32-head units also take the balanced split as soon as their 512-token
  // fixed partitions would not fit one round of the fixed kernel's resident
  // workgroups. MQA 32/1 hd128 bf16, whole operation: B80 x
  // U[1024, 4096] (640 workgroups for 512 resident) 46.6 -> 39.4 us, B48 x
  // U[4096, 8192] 53.2 -> 44.9, B128 54.6 -> 49.1; at or under one round
  // the fixed partitions stay faster (B64 x U[1024, 4096] 32.8 vs 35.3 us,
  // B96 x 2048 33.2 vs 39.5).
  bool past_one_round = false;
  if (a->partition_size == 0 && pl.path == IKL_PATH_MFMA_GROUPED && pl.group_size > 16)
    past_one_round = units * ((maxctx + 511) / 512) >
                     mfma_fixed_capacity(a->dtype, a->head_dim, pl.group_size, pl.kv_fp8);
  const bool want_balanced =
      a->partition_size == -2 ||
      (a->partition_size == 0 && pl.path == IKL_PATH_MFMA_GROUPED && (t_max > SK_MIN_BATCH_TILES || past_one_round));
  if (want_balanced && cap < (int64_t(1) << 29)) {
    // Units of up to 16 heads run unit-parallel (workgroups of UW waves, one
    // unit each, walking the same request tiles): the GQA decode workload's
    // kernel (32/8 hd128 bf16 B32 x U[4096, 8192]) streams faster that way
    // than as one-unit runs. Sequence entries: units / UW per request tile.
    const int uw = mfma_streamk_unitw(pl.units, pl.group_size);
    const int64_t t_seq = t_max / uw;
    const int64_t skw = uw > 1 ? 1 : mfma_launch_shape(true, pl.group_size).waves_per_workgroup;
    const int64_t w =
        std::min<int64_t>(mfma_streamk_capacity(a->dtype, a->head_dim, pl.group_size, pl.kv_fp8, uw),
                          std::max<int64_t>((t_seq + SK_MIN_TILES * skw - 1) / (SK_MIN_TILES * skw), 1));
    // A run that enters a segment of the sequence pays a restart (its
    // epilogue, then a pipeline fill from the new request's blocks): each
    // segment counts that many leading entries, so such runs take fewer
    // tiles. On MQA 32/1 hd128 bf16 (32-head units, two-wave runs) runs
    // crossing a request ended 3.7 us after the others at no cost; the
    // kernel, with costs 0 / 4 / 8 / 16 / 20: B64 x U[1024, 4096] 28.4 /
    // 26.8 / 25.4 / 24.9 / 25.3 us, B128 x U[1024, 4096] 40.4 (4) / 39.3 /
    // 38.4 us, B48 x U[4096, 8192] 36.7 (4) / 35.1 / 35.1 us. Unit-parallel
    // runs (one entry streams UW tiles) and 16-head one-unit runs move
    // within noise (GQA 32/8 B32 x U[4096, 8192] 126.0-126.5 us at 0, 125.3-
    // 125.9 at 1; GQA 48/3 B32 x U[4096, 8192] 60.0-60.2 us at 4 / 8 / 16).
    const int seg_cost = uw > 1 ? SK_SEG_COST_UNITS : (pl.group_size > 16 ? SK_SEG_COST_32 : SK_SEG_COST_ONE);
    const int64_t t_virt = t_seq + (int64_t)seg_cost * a->batch * (pl.units / uw);
    if ((double)(t_virt + 1) * (double)w < 4.0e18) {
      pl.sk_waves = (int)w;
      pl.sk_unitw = uw;
      pl.sk_seg_cost = seg_cost;
      pl.split = true;
      pl.num_parts = 1;
      pl.partition = (int)std::min<int64_t>(16 * ((t_seq + w - 1) / w), 0x7fffffffLL);
      const int64_t rows = (units / uw + w) * uw * pl.group_size;
      pl.ws_o_bytes = ((rows * a->head_dim * 4) + 255) / 256 * 256;
      pl.ws_bytes = pl.ws_o_bytes + rows * 4;
      return IKL_OK;
    }
  }
  int64_t P;
  if (a->partition_size == -1) {
    P = maxctx;
  } else if (a->partition_size > 0) {
    if (a->partition_size % 64 != 0)
      return fail(IKL_EINVAL, "partition_size must be a positive multiple of 64");
    P = a->partition_size;
  } else if (pl.path == IKL_PATH_MFMA_GROUPED) {
    // 512 tokens, halved (down to 128) while fewer than 160 workgroups. On
    // measured small batches this picked the best of 128/256/512 each time:
    // 256 for the Llama decode shape (192 workgroups), 128 for GQA hd64
    // B4 x 512 (11.9 -> 10.6 us) and MQA hd64 B16 x 2048 (16.4 -> 13.9 us)
    P = 512;
    while (P > 128 && units * ((maxctx + P - 1) / P) < 160) P /= 2;
    if (pl.group_size <= 16 && units >= mfma_cu_count()) {
      // A workgroup per CU without splitting (here at most 32768 tiles, so
      // contexts of at most 2048 tokens): each (request, unit) runs unsplit
      // on its workgroup's 4 waves, with no partials and no reduce. GQA
      // 32/8 hd128 bf16 step (MALL flushed): B32 x 1024 28.2-28.4 -> 25.5-25.7
      // us, B32 x 2048 49.2 -> 45.3, B32 x U[512, 1024] 24.8-25.3 ->
      // 22.3-22.8, hd64 fp16 B32 x 1024 18.7-19.3 -> 15.2-15.4; with fewer
      // units than CUs the split stays faster (B16 x 1024 17.2-17.7 against
      // 18.8-19.0), and 384 units came out even (B48 x 1024 38.7 / 39.2).
      P = maxctx;
    }
    if (pl.group_size > 16) {
      // 32-head units: the longest of 128 ... 1024 tokens that still
      // launches a workgroup per CU (two per CU over the FP8 cache, whose
      // tiles carry half the bytes), and no more workgroups than are
      // resident at once (past that at 512 tokens the balanced split runs
      // instead). Sweeping MQA 32/1 over 128-2048 tokens (whole step, MALL
      // flushed) this picked the fastest size, or one within 1 %, on all 8
      // shapes: hd128 bf16 B64 x U[1024, 4096] (1024), B32 x U[4096, 8192]
      // (1024), B16 x U[1024, 4096] (256), B64 x 2048 (512), B8 x 512 (128),
      // the FP8 cache B64 x U[1024, 4096] (512), hd96 B64 x U[1024, 4096]
      // (1024) and hd64 B16 x 2048 (128).
      const int64_t cap_wg = mfma_fixed_capacity(a->dtype, a->head_dim, pl.group_size, pl.kv_fp8);
      const int64_t target = (int64_t)mfma_cu_count() * (pl.kv_fp8 ? 2 : 1);
      P = 128;
      while (P < 1024 && (units * ((maxctx + 2 * P - 1) / (2 * P)) >= target || units * ((maxctx + P - 1) / P) > cap_wg))
        P *= 2;
      // Over the FP8 cache, 1024-token partitions that give a workgroup per
      // CU, all resident at once, run as 8-wave workgroups (two waves per
      // SIMD, 8 tiles each) in place of 512-token partitions at two 4-wave
      // workgroups per CU. MQA 32/1 hd128 over the FP8 cache, whole step,
      // MALL flushed: B64 x U[1024, 4096] 22.8-22.9 -> 21.5-21.6 us, B32 x
      // U[4096, 8192] 23.9-24.2 -> 21.2-21.8; 1024-token partitions on 4
      // waves took 25.3. The 16-bit cache stays on 4 waves: 8 came out
      // faster only on ragged U[1024, 4096] contexts (bf16 B64 26.2-26.6 ->
      // 25.8-25.9 us, hd96 22.9-23.1 -> 21.4-21.7) and slower on B64 x 4096
      // (31.1-31.8 -> 32.2-32.3), B128 x 2048 (32.5-32.7 -> 33.5-33.6), B64 x
      // U[2048, 4096] and B32 x U[4096, 8192] (26.2-26.5 -> 26.9-27.1).
      const int64_t wg1024 = units * ((maxctx + 1023) / 1024);
      if (pl.kv_fp8 && maxctx >= 1024 && wg1024 >= mfma_cu_count() &&
          wg1024 <= mfma_fixed8_capacity(a->dtype, a->head_dim)) {
        P = 1024;
        pl.fixed_waves = 8;
      }
    }
  } else {
    P = 512;
    // one wave per SIMD of the 256 CUs: on the MHA shapes measured, longer
    // runs beat a second wave per SIMD (fp16 B16 x 32 heads, 512 tokens:
    // 31.3 -> 29.1 us with 256-token partitions instead of 128)
    const int64_t target = 1024;
    while (P > 128 && units * ((maxctx + P - 1) / P) < target) P /= 2;
    // When a request needs at most 4 partitions, they become the waves of
    // one workgroup that merges them in LDS: same waves, no partials and no
    // reduce launch (MHA fp16 B16 x 512: two 256-token partitions + reduce
    // -> one 2-wave workgroup per head). With more partitions the split
    // stays one wave per workgroup: folding 8 into 2 x 4 waves measured
    // slower on ragged batches (MHA bf16 B32 x 1k-4k: 237 -> 258 us).
    const int64_t np = (maxctx + P - 1) / P;
    if (fold_waves && np <= 4) {
      pl.scalar_waves = np == 1 ? 1 : (np == 2 ? 2 : 4);  // 3 partitions: 4 waves of 3/4 partition each
      P = maxctx;
    }
  }
  if (P >= maxctx) {
    pl.split = false;
    pl.num_parts = 1;
    pl.partition = (int)std::min<int64_t>(std::max<int64_t>(cap, maxctx), 0x7fffffffLL);
  } else {
    pl.split = true;
    const int64_t np = (maxctx + P - 1) / P;
    if (np > 65535) return fail(IKL_EINVAL, "too many split partitions for one launch");
    pl.num_parts = (int)np;
    pl.partition = (int)P;
  }
  if (pl.split) {
    const int64_t rows = a->batch * (int64_t)a->num_heads * pl.num_parts;
    pl.ws_o_bytes = ((rows * a->head_dim * 4) + 255) / 256 * 256;
    pl.ws_bytes = pl.ws_o_bytes + rows * 4;
  }
  return IKL_OK;
}

void record(void *ev, hipStream_t s) {
  if (ev) (void)hipEventRecord((hipEvent_t)ev, s);
}

template <typename Tag, int D, int W>
void launch_scalar_waves(int gmax, const AttnParams &p, dim3 grid, hipStream_t s) {
  switch (gmax) {
    case 1: paged_decode_scalar_kernel<Tag, D, 1, W><<<grid, 64 * W, 0, s>>>(p); break;
    case 2: paged_decode_scalar_kernel<Tag, D, 2, W><<<grid, 64 * W, 0, s>>>(p); break;
    case 4: paged_decode_scalar_kernel<Tag, D, 4, W><<<grid, 64 * W, 0, s>>>(p); break;
    default: paged_decode_scalar_kernel<Tag, D, 8, W><<<grid, 64 * W, 0, s>>>(p); break;
  }
}

template <typename Tag, int D>
void launch_scalar(int gmax, int waves, const AttnParams &p, dim3 grid, hipStream_t s) {
  switch (waves) {
    case 2: launch_scalar_waves<Tag, D, 2>(gmax, p, grid, s); break;
    case 4: launch_scalar_waves<Tag, D, 4>(gmax, p, grid, s); break;
    default: launch_scalar_waves<Tag, D, 1>(gmax, p, grid, s); break;
  }
}

template <typename Tag, int D>
void launch_reduce(const AttnParams &p, dim3 grid, hipStream_t s) {
  dim3 rgrid((unsigned)p.num_heads, grid.z);
  paged_decode_reduce_kernel<Tag, D><<<rgrid, 64, 0, s>>>(p);
}

template <typename Tag>
void launch_family(int d, const Plan &pl, const AttnParams &p, dim3 grid, hipStream_t s, int dtype) {
  if (pl.path == IKL_PATH_MFMA_GROUPED) {
    (void)launch_mfma_attention(dtype, d, p, grid, s);
    return;
  }
  switch (d) {
    case 16: launch_scalar<Tag, 16>(pl.gmax, pl.scalar_waves, p, grid, s); break;
    case 32: launch_scalar<Tag, 32>(pl.gmax, pl.scalar_waves, p, grid, s); break;
    case 64: launch_scalar<Tag, 64>(pl.gmax, pl.scalar_waves, p, grid, s); break;
    case 96: launch_scalar<Tag, 96>(pl.gmax, pl.scalar_waves, p, grid, s); break;
    default: launch_scalar<Tag, 128>(pl.gmax, pl.scalar_waves, p, grid, s); break;
  }
}

template <typename Tag>
void launch_reduce_dim(int d, const AttnParams &p, dim3 grid, hipStream_t s) {
  switch (d) {
    case 16: launch_reduce<Tag, 16>(p, grid, s); break;
    case 32: launch_reduce<Tag, 32>(p, grid, s); break;
    case 64: launch_reduce<Tag, 64>(p, grid, s); break;
    case 96: launch_reduce<Tag, 96>(p, grid, s); break;
    default: launch_reduce<Tag, 128>(p, grid, s); break;
  }
}

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace
}  // namespace ikl

using namespace ikl;

extern "C" int64_t ikl_paged_attention_workspace_size(const ikl_paged_attention_args *a) {
  Plan pl;
  int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  return pl.ws_bytes;
}

extern "C" int32_t ikl_paged_attention_partition_size(const ikl_paged_attention_args *a) {
  Plan pl;
  int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  return pl.split ? pl.partition : 0;
}

namespace ikl {
namespace {
template <typename Tag, int D>
int scalar_tile_tokens(int gmax) {
  switch (gmax) {
    case 1: return ScalarCfg<Tag, D, 1>::TI;
    case 2: return ScalarCfg<Tag, D, 2>::TI;
    case 4: return ScalarCfg<Tag, D, 4>::TI;
    default: return ScalarCfg<Tag, D, 8>::TI;
  }
}
template <typename Tag>
int scalar_tile_tokens_dim(int d, int gmax) {
  switch (d) {
    case 16: return scalar_tile_tokens<Tag, 16>(gmax);
    case 32: return scalar_tile_tokens<Tag, 32>(gmax);
    case 64: return scalar_tile_tokens<Tag, 64>(gmax);
    case 96: return scalar_tile_tokens<Tag, 96>(gmax);
    default: return scalar_tile_tokens<Tag, 128>(gmax);
  }
}
}  // namespace
}  // namespace ikl

static_assert(offsetof(ikl_launch_config, group_size) == IKL_LAUNCH_CONFIG_MIN_BYTES,
              "IKL_LAUNCH_CONFIG_MIN_BYTES ends at the first field added after the first version");

extern "C" int ikl_paged_attention_launch_config(const ikl_paged_attention_args *a, ikl_launch_config *out) {
  if (!out) return fail(IKL_EINVAL, "launch config: null output struct");
  if (out->struct_size < IKL_LAUNCH_CONFIG_MIN_BYTES)
    return fail(IKL_EINVAL, "launch config: struct_size " + std::to_string(out->struct_size) +
                                " is below the " + std::to_string(IKL_LAUNCH_CONFIG_MIN_BYTES) +
                                " bytes of the smallest ikl_launch_config");
  Plan pl;
  int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  ikl_launch_config c{};
  c.path = pl.path;
  c.partition_size = pl.split ? pl.partition : 0;
  if (pl.path == IKL_PATH_MFMA_GROUPED) {
    const MfmaShape sh = mfma_launch_shape(pl.sk_waves > 0, pl.group_size, pl.sk_unitw, pl.fixed_waves);
    c.tile_tokens = sh.tile_tokens;
    c.waves_per_workgroup = sh.waves_per_workgroup;
    c.stages = sh.stages;
  } else {
    switch (a->dtype) {
      case IKL_F16: c.tile_tokens = scalar_tile_tokens_dim<f16_tag>(a->head_dim, pl.gmax); break;
      case IKL_BF16: c.tile_tokens = scalar_tile_tokens_dim<bf16_tag>(a->head_dim, pl.gmax); break;
      default: c.tile_tokens = scalar_tile_tokens_dim<f32_tag>(a->head_dim, pl.gmax); break;
    }
    c.waves_per_workgroup = pl.scalar_waves;
    c.stages = 2;
  }
  c.split = pl.sk_waves > 0 ? 2 : (pl.split ? 1 : 0);
  c.workgroups = pl.sk_waves > 0 ? (int64_t)pl.sk_waves
                                 : (int64_t)pl.num_parts * a->num_kv_heads * pl.groups_per_kv * a->batch;
  c.group_size = pl.group_size;
  // fill what the caller's struct holds (an older, shorter struct keeps its size)
  const size_t n = std::min<size_t>((size_t)out->struct_size, sizeof(c));
  c.struct_size = out->struct_size;
  std::memcpy(out, &c, n);
  return IKL_OK;
}

extern "C" int32_t ikl_paged_attention_path(int32_t dtype, int32_t head_dim, int32_t block_size,
                                            int64_t table_width, int32_t heads_per_kv,
                                            int32_t query_group_size) {
  (void)table_width;
  return select_path(dtype, head_dim, block_size, heads_per_kv, query_group_size);
}

namespace ikl {
namespace {
// Validates and enqueues one attention launch; `app` (optional) rides on the
// split reduce kernel, which the caller has checked runs (pl.split).
int run_attention(const ikl_paged_attention_args *a, const Plan &pl, const FusedAppend *app, void *stream) {
  if (!a->query || !a->k_cache || !a->v_cache || !a->block_tables || !a->context_lens || !a->out)
    return fail(IKL_EINVAL, "attention: null tensor pointer");
  const int vec = 16 / pl.eb;
  const int cvec = pl.kv_fp8 ? 16 : vec;  // cache elements per 16 bytes
  // 16-byte vector access needs every row start 16-byte aligned.
  if (!aligned16(a->query) || !aligned16(a->k_cache) || !aligned16(a->v_cache) || !aligned16(a->out) ||
      a->q_stride_b % vec || a->q_stride_h % vec || a->k_stride_block % cvec ||
      a->k_stride_token % cvec || a->k_stride_head % cvec || a->v_stride_block % cvec ||
      a->v_stride_token % cvec || a->v_stride_head % cvec || a->out_stride_b % vec ||
      a->out_stride_h % vec)
    return fail(IKL_EINVAL, "attention: query/cache/out rows must be 16-byte aligned");
  // the MFMA family addresses the rows of a 16-token tile through 32-bit byte offsets
  if (pl.path == IKL_PATH_MFMA_GROUPED &&
      (16 * a->k_stride_token * (pl.kv_fp8 ? 1 : pl.eb) >= (int64_t(1) << 31) ||
       16 * a->v_stride_token * (pl.kv_fp8 ? 1 : pl.eb) >= (int64_t(1) << 31) ||
       a->k_stride_token < a->head_dim || a->v_stride_token < a->head_dim))
    return fail(IKL_EINVAL, "attention: token strides must lie in [head_dim, 2^27 bytes / 16)");
  // ... and reaches a tile's block through a 32-bit block stride in bytes
  if (pl.path == IKL_PATH_MFMA_GROUPED &&
      (a->k_stride_block * (pl.kv_fp8 ? 1 : pl.eb) >= (int64_t(1) << 32) ||
       a->v_stride_block * (pl.kv_fp8 ? 1 : pl.eb) >= (int64_t(1) << 32) || a->k_stride_block < 0 ||
       a->v_stride_block < 0 || (pl.kv_fp8 && (a->scale_stride_block * 4 >= (int64_t(1) << 32) ||
                                                a->scale_stride_head * 4 >= (int64_t(1) << 31)))))
    return fail(IKL_EINVAL, "attention: block strides must lie below 4 GiB");
  if (pl.kv_fp8 && (!a->k_scale || !a->v_scale || !aligned16(a->k_scale) || !aligned16(a->v_scale) ||
                    a->scale_stride_block % 4 || a->scale_stride_head % 4))
    return fail(IKL_EINVAL, "attention: the FP8 cache needs 16-byte aligned k_scale / v_scale rows");
  if (pl.split && (!a->workspace || a->workspace_bytes < pl.ws_bytes || !aligned16(a->workspace)))
    return fail(IKL_EWORKSPACE, "attention: workspace missing or smaller than " +
                                    std::to_string(pl.ws_bytes) + " bytes");

  AttnParams p;
  p.q = (const char *)a->query;
  p.q_sb = a->q_stride_b;
  p.q_sh = a->q_stride_h;
  p.kc = (const char *)a->k_cache;
  p.vc = (const char *)a->v_cache;
  p.k_sb = a->k_stride_block;
  p.k_st = a->k_stride_token;
  p.k_sh = a->k_stride_head;
  p.v_sb = a->v_stride_block;
  p.v_st = a->v_stride_token;
  p.v_sh = a->v_stride_head;
  p.tables = a->block_tables;
  p.t_sb = a->table_stride_b;
  p.table_width = a->table_width;
  p.lens = a->context_lens;
  p.out = (char *)a->out;
  p.o_sb = a->out_stride_b;
  p.o_sh = a->out_stride_h;
  p.part_o = pl.split ? (float *)a->workspace : nullptr;
  p.part_lse = pl.split ? (float *)((char *)a->workspace + pl.ws_o_bytes) : nullptr;
  p.num_blocks = a->num_blocks;
  p.num_heads = a->num_heads;
  p.heads_per_kv = pl.heads_per_kv;
  p.group_size = pl.group_size;
  p.groups_per_kv = pl.groups_per_kv;
  p.block_size = a->block_size;
  p.bs_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1 << sh) == a->block_size) p.bs_shift = sh;
  p.partition_size = pl.partition;
  p.num_parts = pl.num_parts;
  p.split = pl.split ? 1 : 0;
  p.table_i64 = a->table_type == IKL_I64;
  p.lens_i64 = a->lens_type == IKL_I64;
  p.scale_log2 = a->scale * LOG2E;
  p.sk_waves = pl.sk_waves;
  p.sk_unitw = pl.sk_unitw;
  p.sk_seg_cost = pl.sk_seg_cost;
  p.fixed_waves = pl.sk_waves > 0 ? 0 : pl.fixed_waves;
  p.units = (int32_t)pl.units;
  p.grid_spread = pl.path == IKL_PATH_MFMA_GROUPED && pl.sk_waves == 0 && spread_grid(pl.units, pl.num_parts, a->batch);
  p.batch = a->batch;
  p.cap_tokens = a->table_width * (int64_t)a->block_size;
  p.kv_fp8 = pl.kv_fp8 ? 1 : 0;
  p.k_scale = (const float *)a->k_scale;
  p.v_scale = (const float *)a->v_scale;
  p.s_sb = a->scale_stride_block;
  p.s_sh = a->scale_stride_head;
  p.app = app ? *app : FusedAppend{};

  dim3 grid((unsigned)pl.num_parts, (unsigned)(a->num_kv_heads * pl.groups_per_kv), (unsigned)a->batch);
  hipStream_t s = (hipStream_t)stream;
  record(a->events[0], s);
  switch (a->dtype) {
    case IKL_F16: launch_family<f16_tag>(a->head_dim, pl, p, grid, s, a->dtype); break;
    case IKL_BF16: launch_family<bf16_tag>(a->head_dim, pl, p, grid, s, a->dtype); break;
    default: launch_family<f32_tag>(a->head_dim, pl, p, grid, s, a->dtype); break;
  }
  record(a->events[1], s);
  if (pl.split) {
    switch (a->dtype) {
      case IKL_F16: launch_reduce_dim<f16_tag>(a->head_dim, p, grid, s); break;
      case IKL_BF16: launch_reduce_dim<bf16_tag>(a->head_dim, p, grid, s); break;
      default: launch_reduce_dim<f32_tag>(a->head_dim, p, grid, s); break;
    }
  }
  record(a->events[2], s);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IKL_ELAUNCH, std::string("paged attention launch: ") + hipGetErrorString(e));
  return IKL_OK;
}

// Whether a decode step's append rides on the reduce kernel (1), runs as
// its own launch after the attention (0), or the arguments are invalid (<0).
// A split launch's reduce carries the append. An unsplit one (a VALU plan
// folded into multi-wave workgroups included) is followed by the append
// kernel: keeping such a plan split so that its reduce could carry the
// append measured slower per step (MHA fp16 hd128 B16 x 512 27.8-28.6 ->
// 26.8-27.3 us with the append kernel, B32 x 1024 88.4 -> 85.3, hd64 B16 x
// 512 18.7-19.2 -> 16.9-17.1; fp32 GQA 32/8 hd64 B4 x 512 equal).
int step_plan(const ikl_paged_attention_args *a, const ikl_append_args *app, Plan &pl, FusedAppend &f) {
  int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  rc = prepare_fused_append(app, f);
  if (rc < 0) return rc;
  // an FP8 append rides along when its rows are in the query dtype (the
  // reduce kernel's element type)
  const bool can_fuse = rc == IKL_OK && f.rows > 0 && (!f.fp8 || f.src_dtype == a->dtype);
  return can_fuse && pl.split ? 1 : 0;
}
}  // namespace
}  // namespace ikl

extern "C" int ikl_paged_attention(const ikl_paged_attention_args *a, void *stream) {
  Plan pl;
  const int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  return run_attention(a, pl, nullptr, stream);
}

// Split workspace of ikl_paged_attention_noalloc: one array per device for
// the whole process. Every call on a device shares it, so calls that
// overlap on one device race; nothing in it needs clearing (each launch
// writes every partial its reduce reads).
static __device__ __align__(256) unsigned char scratch[IKL_NOALLOC_SCRATCH_BYTES];

namespace ikl {
namespace {
constexpr int SCRATCH_MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[SCRATCH_MAX_DEVICES] = {};

// Device address of `scratch` on the current device, looked up once per
// device (the array's name is only a host-side stand-in).
int scratch_address(void **out) {
  int dev = -1;
  const hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) {
    (void)hipGetLastError();
    return fail(IKL_ELAUNCH, std::string("attention (no-alloc): no current device: ") + hipGetErrorString(de));
  }
  if (dev < 0 || dev >= SCRATCH_MAX_DEVICES)
    return fail(IKL_EUNSUPPORTED, "attention (no-alloc): device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return fail(IKL_ELAUNCH, std::string("attention (no-alloc): hipGetSymbolAddress(scratch) failed: ") +
                                   hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return IKL_OK;
}
}  // namespace
}  // namespace ikl

extern "C" int ikl_paged_attention_noalloc(const ikl_paged_attention_args *a, void *stream) {
  Plan pl;
  int rc = make_plan(a, pl);
  if (rc != IKL_OK) return rc;
  if (pl.ws_bytes > (int64_t)IKL_NOALLOC_SCRATCH_BYTES)
    return fail(IKL_EWORKSPACE, "attention (no-alloc): the launch needs " + std::to_string(pl.ws_bytes) +
                                    " bytes of split workspace, more than the " +
                                    std::to_string((int64_t)IKL_NOALLOC_SCRATCH_BYTES) +
                                    "-byte scratch; call ikl_paged_attention with a workspace instead");
  ikl_paged_attention_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (pl.split) {
    rc = scratch_address(&b.workspace);
    if (rc != IKL_OK) return rc;
    b.workspace_bytes = (int64_t)IKL_NOALLOC_SCRATCH_BYTES;
  }
  return run_attention(&b, pl, nullptr, stream);
}

extern "C" int64_t ikl_paged_decode_step_workspace_size(const ikl_paged_attention_args *a,
                                                        const ikl_append_args *app) {
  Plan pl;
  FusedAppend f;
  const int mode = step_plan(a, app, pl, f);
  if (mode < 0) return mode;
  return pl.ws_bytes;
}

extern "C" int32_t ikl_paged_decode_step_fused(const ikl_paged_attention_args *a, const ikl_append_args *app) {
  Plan pl;
  FusedAppend f;
  return step_plan(a, app, pl, f);
}

extern "C" int ikl_paged_decode_step(const ikl_paged_attention_args *a, const ikl_append_args *app,
                                     void *stream) {
  Plan pl;
  FusedAppend f;
  const int mode = step_plan(a, app, pl, f);
  if (mode < 0) return mode;
  const int rc = run_attention(a, pl, mode == 1 ? &f : nullptr, stream);
  if (rc != IKL_OK || mode == 1 || app->num_tokens == 0) return rc;
  return ikl_append_kv(app, stream);
}
