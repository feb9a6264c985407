// Paged decode attention on the gfx950 matrix cores (MFMA family).
//
// Same result as the scalar family (paged_reference, attention.py:134-175);
// used for fp16/bf16 caches with head_dim in {32, 64, 96, 128} and a block
// size that is a multiple of 16. One wave per (partition, kv head, query
// group of <= 16 heads, request) walks its partition in 16-token tiles (a
// tile never crosses a block, so it needs one block-table entry):
//
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T      D/32 v_mfma_f32_16x16x32
//   online softmax on S (lane = one head x 4 tokens; lazily rescaled)
//   O^T[D x 16 heads]     += V^T[D x 16] . P[16 x 16]   D/16 v_mfma_f32_16x16x16
//
// K rows feed the QK^T MFMA straight from HBM (lane l loads 16 bytes of
// token l%16), and the S accumulator of lane l — P[tokens 4(l/16)..+3][head
// l%16] — is already the B operand of the PV MFMA. V tiles are staged
// row-major in LDS (16-byte pieces rotated by row to spread banks) and read
// back transposed with ds_read_b64_tr_b16, which hands each lane four
// consecutive tokens of one head_dim column: the V^T operand.
//
// MFMA operand layouts (gfx950; 16x16x32 checked by a lane-layout probe):
//   16x16x32: lane l supplies A[l%16][8(l/16)+j], B[8(l/16)+j][l%16], j < 8;
//   16x16x16: lane l supplies A[l%16][4(l/16)+j], B[4(l/16)+j][l%16], j < 4;
//   both:     lane l receives D[4(l/16)+i][l%16], i < 4.
// ds_read_b64_tr_b16: in each 16-lane group, lane i receives element i%4 of
//   the 8-byte chunks supplied by lanes 4k + i/4, k < 4.
#include "ikl_common.h"
#include "paged_attn.h"

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

constexpr int TILE = 16;  // tokens per tile

// Tuning knobs: tiles prefetched ahead of the one computing (1 or 2), and an
// optional minimum-occupancy request to the register allocator.
#ifndef IKL_MFMA_PREFETCH
#define IKL_MFMA_PREFETCH 1
#endif
#ifndef IKL_MFMA_MIN_WAVES
#define IKL_MFMA_WAVES_ATTR
#else
#define IKL_MFMA_WAVES_ATTR __attribute__((amdgpu_waves_per_eu(IKL_MFMA_MIN_WAVES, 8)))
#endif

template <typename Tag>
struct mfma_ops;

template <>
struct mfma_ops<bf16_tag> {
  // S^T tile: K[16 x 32] . Q^T[32 x 16]
  __device__ static inline f32x4_t mma_k32(v4u32 a, v4u32 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // O^T tile: V^T[16 x 16] . P[16 x 16]
  __device__ static inline f32x4_t mma_k16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two probabilities (v_cvt_pk_bf16_f32).
  __device__ static inline uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x, y}, bf16x2_t));
  }
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
};

__device__ inline v4u32 zero4() { return v4u32{0u, 0u, 0u, 0u}; }

template <typename Tag, int D>
__global__ __launch_bounds__(64) IKL_MFMA_WAVES_ATTR void paged_decode_mfma_kernel(const AttnParams p) {
  static_assert(D % 32 == 0 && D <= 128, "MFMA path needs head_dim = 32k <= 128");
  constexpr int EB = 2;
  constexpr int KSTEPS = D / 32;              // QK^T k-steps
  constexpr int MTILES = D / 16;              // PV output tiles of 16 dims
  constexpr int PIECES = D * EB / 16;         // 16-byte pieces per row
  constexpr int ROWB = D * EB;                // bytes per K/V row
  constexpr int VLOADS = (TILE * PIECES + 63) / 64;  // 16-byte V loads per lane per tile
  // V tile staging during the loop; the wave's [16 heads x D] fp32 results
  // at the end (coalesced stores), hence the larger of the two sizes.
  __shared__ __attribute__((aligned(16))) char vtile[16 * D * 4 > TILE * ROWB ? 16 * D * 4 : TILE * ROWB];
  using ops = mfma_ops<Tag>;

  const int lane = threadIdx.x;
  const int hl = lane & 15;   // MFMA row/column index inside a 16-lane group
  const int grp = lane >> 4;  // 16-lane group
  const int part = blockIdx.x;
  const int kvh = blockIdx.y / p.groups_per_kv;
  const int qg = blockIdx.y % p.groups_per_kv;
  const int64_t b = blockIdx.z;

  const int64_t ctx = p.lens_i64 ? load_index<int64_t>(p.lens, b) : load_index<int32_t>(p.lens, b);
  const int64_t part_start = (int64_t)part * p.partition_size;
  if (part > 0 && part_start >= ctx) return;
  const int64_t part_end = ctx < part_start + p.partition_size ? ctx : part_start + p.partition_size;
  const int n_tiles = part_end > part_start ? (int)((part_end - part_start + TILE - 1) / TILE) : 0;

  // ---- Q^T operand: lane l holds q[head0 + l%16][32s + 8(l/16) .. +7]
  const int head0 = qg * p.group_size;
  const bool head_ok = (hl < p.group_size) && (head0 + hl < p.heads_per_kv);
  const int64_t hq = (int64_t)kvh * p.heads_per_kv + head0 + hl;
  v4u32 qb[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    qb[s] = zero4();
    if (head_ok) qb[s] = load16v_global(p.q + (b * p.q_sb + hq * p.q_sh + 32 * s + 8 * grp) * EB);
  }

  // ---- per-lane constant offsets (bytes)
  const int k_lane = (hl * (int)p.k_st + 8 * grp) * EB;  // token hl, dims 8g.. of each k-step
  int v_lds[VLOADS], v_lane[VLOADS];
#pragma unroll
  for (int u = 0; u < VLOADS; ++u) {
    const int pi = u * 64 + lane;  // V piece: row pi / PIECES, piece pi % PIECES
    const int row = pi / PIECES < TILE ? pi / PIECES : TILE - 1, c = pi % PIECES;
    v_lds[u] = row * ROWB + ((c + row) % PIECES) * 16;
    v_lane[u] = row * (int)p.v_st * EB + c * 16;
  }
  int tr_lds[MTILES];  // V^T reads: token 4g + (l%16)/4, dims 16mt + 4((l%16)%4)
#pragma unroll
  for (int mt = 0; mt < MTILES; ++mt) {
    const int row = 4 * grp + (hl >> 2);
    const int c = 2 * mt + ((hl & 3) >> 1);
    tr_lds[mt] = row * ROWB + ((c + row) % PIECES) * 16 + (hl & 1) * 8;
  }

  const char *kbase = p.kc + (int64_t)kvh * p.k_sh * EB;
  const char *vbase = p.vc + (int64_t)kvh * p.v_sh * EB;
  const char *zero_row = reinterpret_cast<const char *>(g_zero_row);
  const int bs = p.block_size;
  int64_t win_base = p.bs_shift >= 0 ? (part_start >> p.bs_shift) : part_start / bs;
  int win = load_table_window(p, b, win_base, lane);

  f32x4_t acc[MTILES];
#pragma unroll
  for (int mt = 0; mt < MTILES; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = NEG_SENTINEL, lsum = 0.f;

  struct Tile {
    v4u32 k[KSTEPS];
    v4u32 v[VLOADS];
    int n_valid;  // tokens of the tile inside the partition with a valid block (0..16)
  };

  // Resolves tile t's block and issues its K/V loads (straight-line:
  // masked rows read the zero row).
  auto issue = [&](int t, Tile &T) {
    const int64_t base = part_start + (int64_t)t * TILE;
    const int64_t lb = p.bs_shift >= 0 ? (base >> p.bs_shift) : base / bs;
    if (lb >= win_base + 64) {
      win_base = lb;
      win = load_table_window(p, b, win_base, lane);
    }
    const int64_t off = base - lb * bs;
    const int phys = __builtin_amdgcn_readlane(win, (int)(lb - win_base));
    int64_t left = part_end - base;
    T.n_valid = phys < 0 || left <= 0 ? 0 : (left >= TILE ? TILE : (int)left);
    const int64_t kro = ((int64_t)phys * p.k_sb + off * p.k_st) * EB;
    const int64_t vro = ((int64_t)phys * p.v_sb + off * p.v_st) * EB;
    const bool k_ok = hl < T.n_valid;
    const char *kr = k_ok ? kbase + kro + k_lane : zero_row;
    const int kstep = k_ok ? 64 : 0;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) T.k[s] = load16v_stream(kr + s * kstep);
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      const int row = (u * 64 + lane) / PIECES;
      const bool v_ok = row < T.n_valid;
      T.v[u] = load16v_stream(v_ok ? vbase + vro + v_lane[u] : zero_row);
    }
  };

  auto compute = [&](Tile &T) {
    // stage V row-major in LDS (rows past the tile are never read)
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      if (TILE * PIECES % 64 == 0 || u * 64 + lane < TILE * PIECES)
        *reinterpret_cast<v4u32 *>(vtile + v_lds[u]) = T.v[u];
    }
    // S^T for tokens 4g + i and head hl
    f32x4_t sa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) sa = ops::mma_k32(T.k[s], qb[s], sa);
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = sa[i] * p.scale_log2;
      if (T.n_valid < TILE) sc[i] = 4 * grp + i < T.n_valid ? sc[i] : -INFINITY;
    }
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
    const bool need = tmax > m + RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(need) != 0ull) {
      const float alpha = need ? fast_exp2(m - tmax) : 1.f;
      m = need ? tmax : m;
      lsum *= alpha;
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt) acc[mt] *= alpha;
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = fast_exp2(sc[i] - m);
      lsum += pr[i];
    }
    const u32x2_t pb = {ops::pack(pr[0], pr[1]), ops::pack(pr[2], pr[3])};
    // O^T += V^T P
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) {
      typedef __attribute__((address_space(3))) s16x4_t *lds_s4_ptr;
      const s16x4_t va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_ptr)(vtile + tr_lds[mt]));
      acc[mt] = ops::mma_k16(__builtin_bit_cast(u32x2_t, va), pb, acc[mt]);
    }
  };

  // ---- software pipeline: the loads of the next IKL_MFMA_PREFETCH tiles
  // fly while a tile computes
#if IKL_MFMA_PREFETCH == 2
  Tile ta, tb, tc;
  issue(0, ta);
  issue(1, tb);
  for (int t = 0; t < n_tiles; t += 3) {
    issue(t + 2, tc);
    compute(ta);
    issue(t + 3, ta);
    if (t + 1 < n_tiles) compute(tb);
    issue(t + 4, tb);
    if (t + 2 < n_tiles) compute(tc);
  }
#else
  Tile ta, tb;
  issue(0, ta);
  for (int t = 0; t < n_tiles; t += 2) {
    issue(t + 1, tb);
    compute(ta);
    issue(t + 2, ta);
    if (t + 1 < n_tiles) compute(tb);
  }
#endif

  // ---- combine the four groups' partial sums (m is already common)
  lsum += shfl_xor_f(lsum, 16);
  lsum += shfl_xor_f(lsum, 32);
  // Stage the normalised [heads x D] block in LDS so all 64 lanes store
  // whole 16-byte pieces: the wave's heads are contiguous in the output
  // and in the [B, NP, H, D] partials.
  const int nh = p.group_size < p.heads_per_kv - head0 ? p.group_size : p.heads_per_kv - head0;
  const float inv = p.split ? (lsum > 0.f ? 1.f / lsum : 0.f) : 1.f / lsum;  // 0/0 -> NaN like the reference
  float *stage = reinterpret_cast<float *>(vtile);
  if (head_ok) {
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) {
      const f32x4_t o = acc[mt] * inv;
      *reinterpret_cast<f32x4_t *>(stage + hl * D + 16 * mt + 4 * grp) = o;
    }
  }
  const int64_t hq0 = (int64_t)kvh * p.heads_per_kv + head0;
  if (p.split) {
    const int64_t prow = (b * p.num_parts + part) * p.num_heads + hq0;
    float *dst = p.part_o + prow * D;
    for (int i = lane; i < nh * D / 4; i += 64)
      *reinterpret_cast<f32x4_t *>(dst + 4 * i) = *reinterpret_cast<const f32x4_t *>(stage + 4 * i);
    if (head_ok && grp == 0) p.part_lse[prow + hl] = lsum > 0.f ? m + log2f(lsum) : -INFINITY;
  } else {
    constexpr int CPR = D / 8;  // 16-byte output pieces per head row
    for (int i = lane; i < nh * CPR; i += 64) {
      const int h = i / CPR, c = i % CPR;
      const float *src = stage + h * D + 8 * c;
      u32x4 w;
      if constexpr (__is_same(Tag, bf16_tag)) {
        w.x = elem<bf16_tag>::pack2(src[0], src[1]);
        w.y = elem<bf16_tag>::pack2(src[2], src[3]);
        w.z = elem<bf16_tag>::pack2(src[4], src[5]);
        w.w = elem<bf16_tag>::pack2(src[6], src[7]);
      } else {
        w.x = elem<f16_tag>::pack2(src[0], src[1]);
        w.y = elem<f16_tag>::pack2(src[2], src[3]);
        w.z = elem<f16_tag>::pack2(src[4], src[5]);
        w.w = elem<f16_tag>::pack2(src[6], src[7]);
      }
      store16(p.out + (b * p.o_sb + (hq0 + h) * p.o_sh + 8 * c) * EB, w);
    }
  }
}

template <typename Tag>
hipError_t launch_dim(int d, const AttnParams &p, dim3 grid, hipStream_t s) {
  switch (d) {
    case 32: paged_decode_mfma_kernel<Tag, 32><<<grid, 64, 0, s>>>(p); break;
    case 64: paged_decode_mfma_kernel<Tag, 64><<<grid, 64, 0, s>>>(p); break;
    case 96: paged_decode_mfma_kernel<Tag, 96><<<grid, 64, 0, s>>>(p); break;
    default: paged_decode_mfma_kernel<Tag, 128><<<grid, 64, 0, s>>>(p); break;
  }
  return hipGetLastError();
}

}  // namespace

bool mfma_supported(int dtype, int head_dim, int block_size, int group_size) {
  return (dtype == IKL_F16 || dtype == IKL_BF16) &&
         (head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128) &&
         block_size > 0 && block_size % 16 == 0 && group_size >= 1 && group_size <= 16;
}

hipError_t launch_mfma_attention(int dtype, int head_dim, const AttnParams &p, dim3 grid, hipStream_t s) {
  if (dtype == IKL_BF16) return launch_dim<bf16_tag>(head_dim, p, grid, s);
  return launch_dim<f16_tag>(head_dim, p, grid, s);
}

}  // namespace ikl
