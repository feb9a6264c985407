// Paged prefill attention: causal attention of a ragged batch of prompt
// chunks over the block-table addressed cache. Same result as the gather +
// masked SDPA of paged_prefill_attention_sdpa (attention.py:230-321):
//
//   row t of request b sits at position start_b + t; rows t < len_b - start_b
//   attend the keys at positions <= start_b + t (all < len_b); the remaining
//   (padding) rows of the query width receive the value at position 0, which
//   is what the reference's mask leaves them (attention.py:305).
//
// Two kernel families:
//
//  * MFMA (fp16 / bf16, head_dim 32k <= 128, block_size % 16 == 0):
//    paged_prefill_mfma_kernel. A workgroup of 4 waves takes 64 * NG query
//    rows of one (request, kv head) — a row is one (token, query head) pair,
//    token-major, so the heads sharing a KV head sit in consecutive rows —
//    and streams the request's keys in 32-token tiles that the workgroup
//    stages once in LDS for all its waves (double-buffered, one barrier per
//    tile). Each wave owns 16 * NG rows and runs, per tile and 16-row group:
//
//      S^T[32 keys x 16 rows] = K . Q^T     2 * D/32 v_mfma_f32_16x16x32
//      online softmax (lane = one row x 8 keys, causal mask on the diagonal)
//      O^T[D x 16 rows]     += V^T . P      D/16 v_mfma_f32_16x16x32
//
//    Both products use the full-rate gfx950 16x16x32 shape: the K rows of the
//    two S^T halves are permuted (MFMA row 4g + i of half h holds key
//    8g + 4h + i) so that lane l ends with the scores of keys 8(l/16)..+7,
//    exactly the P operand of a 32-deep PV MFMA; its V^T operand is two
//    ds_read_b64_tr_b16 of the staged tile.
//
//  * VALU (every other dtype / head_dim <= 256 / block size):
//    paged_prefill_scalar_kernel, one wave per (request, head, row), keys in
//    sequence, fp32 online softmax.
//
// Blocks whose table entry lies outside [0, num_blocks) are masked as in the
// decode kernels; no load ever leaves the cache.
#include "ikl_common.h"
#include "mfma_ops.h"
#include "paged_attn.h"

namespace ikl {

struct PrefillParams {
  const char *q;
  int64_t q_sb, q_sh, q_st;  // elements
  const char *kc;
  const char *vc;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  const void *tables;
  int64_t t_sb;
  int64_t table_width;
  const void *starts;
  const void *lens;
  char *out;
  int64_t o_sb, o_sh, o_st;
  int64_t batch;
  int64_t width;       // query rows per request (T)
  int64_t num_blocks;
  int64_t cap_tokens;  // table_width * block_size
  int64_t row_blocks;  // workgroups per (request, kv head) of the MFMA kernel
  int64_t bh_pad;      // batch * num_kv_heads rounded up to a multiple of 8
  int32_t stream_major;  // each XCD takes its (request, kv head) prefixes one after another
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t heads_per_kv;
  int32_t head_dim;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) or -1
  int32_t table_i64;
  int32_t idx_i64;   // starts / lens element type
  float scale_log2;  // scale * log2(e)
  // FP8 KV cache: E4M3 codes, one fp32 scale per (token, head) row in
  // k_scale / v_scale [blocks, kv heads, block_size]
  int32_t kv_fp8;
  const float *k_scale;
  const float *v_scale;
  int64_t s_sb, s_sh;  // elements
};

namespace {

__device__ inline int64_t pf_index(const void *base, int64_t i, int i64) {
  return i64 ? load_index<int64_t>(base, i) : load_index<int32_t>(base, i);
}

// Block-table entry (b, lb), or -1 when it is outside the table or names a
// block outside the cache.
__device__ inline int pf_block(const PrefillParams &p, int64_t b, int64_t lb) {
  if (lb < 0 || lb >= p.table_width) return -1;
  const int64_t e = pf_index(p.tables, b * p.t_sb + lb, p.table_i64);
  return e >= 0 && e < p.num_blocks ? (int)e : -1;
}

// Prefill range of request b: start (clamped to [0, end]), end (clamped to
// [0, cap_tokens]) and the number of attending rows (<= width).
__device__ inline void pf_range(const PrefillParams &p, int64_t b, int64_t *start, int64_t *end, int64_t *rows) {
  int64_t e = pf_index(p.lens, b, p.idx_i64);
  e = e < 0 ? 0 : (e < p.cap_tokens ? e : p.cap_tokens);
  int64_t s = pf_index(p.starts, b, p.idx_i64);
  s = s < 0 ? 0 : (s < e ? s : e);
  *start = s;
  *end = e;
  *rows = e - s < p.width ? e - s : p.width;
}

__device__ inline int64_t pf_logical(const PrefillParams &p, int64_t pos) {
  return p.bs_shift >= 0 ? (pos >> p.bs_shift) : pos / p.block_size;
}

constexpr int PT = 32;     // keys per tile
constexpr int PWAVES = 4;  // waves per workgroup

// 16-row MFMA groups per wave and register budget, measured on 8 x
// 4096-token GQA-32/8 prompts: two groups at 2 waves/SIMD beat four at 1
// wave/SIMD (1.49 vs 2.14 ms); fetching two tiles ahead gains ~3 % over
// one; bf16 P is not split into a second MFMA (that cost ~13 % for
// accuracy the bf16 bound does not need).
constexpr int PREFILL_NG = 2;
constexpr int PF = 2;  // tiles held in registers ahead of the one being staged
#define IKL_PREFILL_WAVES_ATTR __attribute__((amdgpu_waves_per_eu(2, 8)))

// Two E4M3 codes times one fp32 scale -> two 16-bit values (one rounding).
template <typename Tag>
__device__ inline uint32_t fp8x2_scaled(uint32_t w, float scale, bool hi);
template <>
__device__ inline uint32_t fp8x2_scaled<bf16_tag>(uint32_t w, float scale, bool hi) {
  return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, true)
                                        : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, false));
}
template <>
__device__ inline uint32_t fp8x2_scaled<f16_tag>(uint32_t w, float scale, bool hi) {
  return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, scale, true)
                                        : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, scale, false));
}

// KV8: the cache holds E4M3 codes with per-row scales. The copy waves load
// the codes (half the bytes) and each row's scale, and stage
// round(code * scale) in the same 16-bit tile layout, so the tile loop is
// unchanged.
template <typename Tag, int D, int NG, bool KV8>
__global__ __launch_bounds__(64 * PWAVES) IKL_PREFILL_WAVES_ATTR void paged_prefill_mfma_kernel(const PrefillParams p) {
  static_assert(D % 32 == 0 && D <= 128, "MFMA prefill needs head_dim = 32k <= 128");
  using ops = mfma_ops<Tag>;
  constexpr int EB = 2;
  constexpr int ROWB = D * EB;               // bytes per K/V row
  constexpr int PIECES = ROWB / 16;          // 16-byte pieces per row
  constexpr int KSTEPS = D / 32;             // QK^T k-steps
  constexpr int MTILES = D / 16;             // PV output tiles of 16 dims
  constexpr int RW = 16 * NG;                // query rows per wave
  constexpr int RWG = RW * PWAVES;           // query rows per workgroup
  constexpr int TILE_BYTES = PT * ROWB;      // one staged K or V tile
  constexpr int CEB = KV8 ? 1 : EB;          // bytes per cache element
  constexpr int CPIECES = D * CEB / 16;      // 16-byte pieces per cache row
  constexpr int PPL = (16 * CPIECES + 63) / 64;  // copy pieces per lane (a wave moves a half tile)
  static_assert(PWAVES == 4 && (KV8 || (16 * PIECES) % 64 == 0), "four waves copy K / V halves");
  // Per-row offsets of the staged K and V tiles' 16-byte pieces (bijective
  // per row). V pieces are rotated by vswz. K pieces are rotated by kswz,
  // or, for rows of 16 pieces, XORed with it: gfx950 serves a 16-byte LDS
  // read conflict-free when each 16 consecutive lanes hit 16 distinct
  // pieces of a 256-byte window and lanes l and l + 16 stay in the same
  // 64-byte quarter of it. The K read's lane l + 16 takes the next k-step
  // piece of lane l's row, which the XOR keeps in its quarter and the
  // rotation does not (a probe of this read pattern: 89-90 against 71 TB/s
  // of LDS reads across the GPU).
  auto kswz = [](int row) { return (row & 3) + 4 * (row >> 3); };
  auto vswz = [](int row) { return 2 * (row & 3) + 8 * ((row >> 3) & 1); };
  auto kpiece = [](int c, int sw) { return PIECES == 16 ? (c ^ sw) & 15 : (c + sw) % PIECES; };
  __shared__ __attribute__((aligned(16))) char lds[2][2][TILE_BYTES];  // [stage][K, V]

  const int tid = threadIdx.x;
  const int lane = tid & 63, hl = lane & 15, grp = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Workgroup -> (row block, request, kv head). All row blocks of one
  // (request, kv head) share blockIdx.x mod 8, hence one XCD and its L2; the
  // row blocks nearest the end of the prompts (most keys) start first.
  // stream_major: XCD x (workgroups x, x + 8, ...) runs all row blocks of
  // its prefixes x, x + 8, ... one prefix after another, so the workgroups
  // resident on it at any time read one prefix's K/V and share its L2 lines;
  // otherwise the row blocks of all its prefixes interleave.
  const int64_t idx = blockIdx.x;
  int64_t bh, rb;
  if (p.stream_major) {
    const int64_t j = idx / 8, k = j / p.row_blocks;
    bh = idx % 8 + 8 * k;
    rb = p.row_blocks - 1 - (j - k * p.row_blocks);
  } else {
    bh = idx % p.bh_pad;
    rb = p.row_blocks - 1 - idx / p.bh_pad;
  }
  if (bh >= p.batch * p.num_kv_heads) return;
  const int64_t b = bh / p.num_kv_heads;
  const int kvh = (int)(bh % p.num_kv_heads);
  const int G = p.heads_per_kv;

  int64_t start64, end64, nrows;
  pf_range(p, b, &start64, &end64, &nrows);
  // positions fit in 31 bits (the host bounds table_width * block_size)
  const int start = (int)start64, end = (int)end64;
  const int64_t rows_valid = nrows * G, rows_all = p.width * G;
  const int64_t row0 = rb * RWG;
  const int64_t wr0 = row0 + (int64_t)wave * RW;

  // keys the workgroup needs, and the wave's own causal window
  const int64_t wg_last = (row0 + RWG < rows_valid ? row0 + RWG : rows_valid) - 1;
  const int kv_hi = wg_last >= row0 ? start + (int)(wg_last / G) + 1 : 0;
  const int n_tiles = (kv_hi + PT - 1) / PT;
  const int64_t w_last = (wr0 + RW < rows_valid ? wr0 + RW : rows_valid) - 1;
  const int w_hi = w_last >= wr0 ? start + (int)(w_last / G) + 1 : 0;  // keys [0, w_hi) reach some row
  const int w_lo = start + (int)(wr0 / G);                             // every row sees keys <= w_lo

  // Q^T operands and the position of each lane's row (-1: not attending)
  v4u32 qb[NG][KSTEPS];
  int qpos[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int64_t r = wr0 + 16 * g + hl;
    const bool ok = r < rows_valid;
    const int64_t t = ok ? r / G : 0;
    const int h = ok ? (int)(r % G) : 0;
    qpos[g] = ok ? start + (int)t : -1;
    const char *qrow = p.q + (b * p.q_sb + ((int64_t)kvh * G + h) * p.q_sh + t * p.q_st + 8 * grp) * EB;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qb[g][s] = ok ? load16v_global(qrow + 64 * s) : zero4();
  }
  // Wait for Q here: otherwise the loop's first MFMA would wait for every
  // load in flight, the next tiles' prefetch included.
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) asm volatile("" ::"v"(qb[g][s]));

  f32x4_t acc[NG][MTILES];
  float m[NG];    // running max of each lane's row, log2 domain (scaled)
  float thr[NG];  // (m + RESCALE_LOG2) in raw score units (scale > 0)
  const float inv_scale_log2 = 1.f / p.scale_log2;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) acc[g][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m[g] = NEG_SENTINEL;
    thr[g] = NEG_SENTINEL;
  }

  // LDS offsets. The 16-byte pieces of a staged row are placed by a
  // row-dependent offset (kpiece / vswz) so that the lanes of one LDS read
  // hit distinct banks: the K reads take rows 8(l/4) + l%4 (+4) of a 32-row
  // tile, the transposing V reads rows 8g + 4h + l/4.
  const int kappa = 8 * (hl >> 2) + (hl & 3);  // key of MFMA row hl in half 0 (+4 in half 1)
  int k_off[2][KSTEPS], tr_off[2][MTILES];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = kappa + 4 * h;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) k_off[h][s] = row * ROWB + kpiece(4 * s + grp, kswz(row)) * 16;
    const int vrow = 8 * grp + 4 * h + (hl >> 2);
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) {
      const int c = 2 * mt + ((hl & 3) >> 1);
      tr_off[h][mt] = vrow * ROWB + ((c + vswz(vrow)) % PIECES) * 16 + (hl & 1) * 8;
    }
  }
  // Cooperative copy: wave w moves half (w & 1) of each tile of K (w < 2)
  // or V (w >= 2), PPL 16-byte pieces per lane, so each wave resolves one
  // block and builds one buffer resource per tile.
  const int cp_v = wave >> 1, cp_h = wave & 1;
  const int row_bytes = (int)((cp_v ? p.v_st : p.k_st) * CEB);
  const char *cp_base = (cp_v ? p.vc + (int64_t)kvh * p.v_sh * CEB : p.kc + (int64_t)kvh * p.k_sh * CEB);
  const int64_t cp_sb = cp_v ? p.v_sb : p.k_sb, cp_st = cp_v ? p.v_st : p.k_st;
  const char *cp_scale = KV8 ? (const char *)(cp_v ? p.v_scale : p.k_scale) + (int64_t)kvh * p.s_sh * 4 : nullptr;
  // piece u of this lane: cache piece c of half-row r; staged (16-bit)
  // pieces sp .. sp + (KV8 ? 1 : 0) of tile row 16 cp_h + r
  int cp_off[PPL], cp_lds[PPL], cp_lds2[PPL], cp_row[PPL];
  bool cp_ok[PPL];
#pragma unroll
  for (int u = 0; u < PPL; ++u) {
    const int pi = u * 64 + lane, r = pi / CPIECES, c = pi % CPIECES;
    const int row = 16 * cp_h + (r < 16 ? r : 15);
    const int sw = cp_v ? vswz(row) : kswz(row);
    const int sp = KV8 ? 2 * c : c;
    cp_ok[u] = pi < 16 * CPIECES;
    cp_row[u] = r < 16 ? r : 15;
    cp_off[u] = cp_row[u] * row_bytes + c * 16;
    cp_lds[u] = row * ROWB + (cp_v ? (sp + sw) % PIECES : kpiece(sp, sw)) * 16;
    cp_lds2[u] = row * ROWB + (cp_v ? (sp + 1 + sw) % PIECES : kpiece(sp + 1, sw)) * 16;
  }
  const char *vbase = p.vc + (int64_t)kvh * p.v_sh * CEB;

  // The block table as a window of 64 consecutive 16-key halves, one per
  // lane: the byte offset of the half's first row from the wave's cache base
  // (and, for FP8, of its first row scale), plus a bit of `holes` for each
  // half whose block lies outside the cache. A tile reads its offsets with
  // v_readlane and its hole bits with a scalar shift, so the per-tile block
  // lookup is a handful of scalar instructions; the window moves every 32
  // tiles (block_size % 16 == 0: a half never straddles two blocks).
  const int64_t cp_blk_bytes = cp_sb * CEB, cp_row_bytes = cp_st * CEB;
  int hbase = 0;
  uint32_t woff_lo, woff_hi, wsc_lo = 0, wsc_hi = 0;
  uint64_t holes_w;
  auto load_window = [&](int h0) {
    const uint32_t pos = 16u * (uint32_t)(h0 + lane);
    const uint32_t lb = pos / (uint32_t)p.block_size;
    const int ph = pf_block(p, b, lb);
    const int64_t in_blk = pos - (int64_t)lb * p.block_size;
    const int64_t off = ph >= 0 ? ph * cp_blk_bytes + in_blk * cp_row_bytes : 0;
    woff_lo = (uint32_t)off;
    woff_hi = (uint32_t)((uint64_t)off >> 32);
    if constexpr (KV8) {
      const int64_t so = ph >= 0 ? (ph * p.s_sb + in_blk) * 4 : 0;
      wsc_lo = (uint32_t)so;
      wsc_hi = (uint32_t)((uint64_t)so >> 32);
    }
    holes_w = __builtin_amdgcn_ballot_w64(ph < 0);
    asm volatile("" ::"v"(woff_lo), "v"(woff_hi));  // in registers before the tiles that read them
  };
  load_window(0);

  // Register staging of the copy (PF tiles in flight), with the tile's hole
  // bits (bit h: half h lies in a block outside the cache).
  struct Staged {
    v4u32 d[PPL];
    float sc[PPL];  // KV8: the scale of each piece's row
    uint32_t holes;
  };

  // Global -> registers for tile j into T. The half is one block window
  // addressed by a buffer resource whose record count ends at the half's
  // last valid row: rows past it (and a whole half whose block is masked)
  // read as zero without a branch. Keys past the end need no other mask:
  // they lie past every row's causal limit.
  auto fetch = [&](int j, Staged &T) {
    const int h0 = 2 * j;
    if (h0 + 1 - hbase >= 64) {
      hbase = h0;
      load_window(hbase);
    }
    const int i0 = h0 - hbase, i = i0 + cp_h;
    T.holes = (uint32_t)(holes_w >> i0) & 3u;
    const uint64_t off = ((uint64_t)__builtin_amdgcn_readlane(woff_hi, i) << 32) | __builtin_amdgcn_readlane(woff_lo, i);
    const int left = end - 16 * (h0 + cp_h);
    const int nv = (T.holes >> cp_h) & 1u ? 0 : (left <= 0 ? 0 : (left < 16 ? left : 16));
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(cp_base + off), (short)0, nv * row_bytes, 0x00020000);
#pragma unroll
    for (int u = 0; u < PPL; ++u)
      if (cp_ok[u]) T.d[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, cp_off[u], 0, 0);
    if constexpr (KV8) {
      // the half's 16 row scales (rows past nv read as 0)
      const uint64_t so = ((uint64_t)__builtin_amdgcn_readlane(wsc_hi, i) << 32) | __builtin_amdgcn_readlane(wsc_lo, i);
      const __amdgpu_buffer_rsrc_t ss =
          __builtin_amdgcn_make_buffer_rsrc((void *)(cp_scale + so), (short)0, nv * 4, 0x00020000);
#pragma unroll
      for (int u = 0; u < PPL; ++u)
        if (cp_ok[u]) T.sc[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ss, cp_row[u] * 4, 0, 0));
    }
  };

  // Row sums of P on the matrix cores: ones[16 x 32] . P gives every row
  // of the result the column sums, i.e. the softmax denominators of the
  // rounded probabilities the PV product uses.
  f32x4_t lacc[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) lacc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const v4u32 ones = v4u32{ops::ONE2, ops::ONE2, ops::ONE2, ops::ONE2};

  auto compute = [&](const char *kt, const char *vt, int base, uint32_t holes_t) {
    if (base >= w_hi) return;                  // no row of this wave reaches the tile
    const bool causal = base + PT - 1 > w_lo;  // diagonal tile: per-key causal test
    const bool holes = holes_t != 0u;          // keys in blocks outside the cache
    v4u32 ka[2][KSTEPS];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) ka[h][s] = *reinterpret_cast<const v4u32 *>(kt + k_off[h][s]);
    // every group's S^T first, so one group's softmax overlaps the next
    // group's MFMAs
    f32x4_t s0[NG], s1[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      s0[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      s1[g] = s0[g];
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        s0[g] = ops::mma_k32(ka[0][s], qb[g][s], s0[g]);
        s1[g] = ops::mma_k32(ka[1][s], qb[g][s], s1[g]);
      }
    }
    v4u32 pb[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // lane: row hl of group g, keys 8 grp + j (j < 4 from s0, 4.. from s1);
      // raw (unscaled) scores: the scale is folded into the exponent
      float sc[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sc[i] = s0[g][i];
        sc[4 + i] = s1[g][i];
      }
      if (causal) {
        const int lim = qpos[g] - base - 8 * grp;  // keys j <= lim are visible
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = j <= lim ? sc[j] : -INFINITY;
      }
      if (holes) {
        // the lane's 8 keys lie in half grp / 2
        const bool dead = (holes_t >> (grp >> 1)) & 1u;
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = dead ? -INFINITY : sc[j];
      }
      // Lazy rescale: the row maximum is only needed when a score passes
      // m + RESCALE_LOG2 (scaled), and each lane can test its own 8 scores
      // against that bound in raw units, so the cross-lane reduction runs
      // on those tiles only (the first one and rare growth).
      const float lmax = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                               fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
      if (__builtin_amdgcn_ballot_w64(lmax > thr[g]) != 0ull) {
        const float tmax = max_xor32(max_xor16(lmax)) * p.scale_log2;
        const bool need = tmax > m[g] + RESCALE_LOG2;
        const float alpha = need ? fast_exp2(m[g] - tmax) : 1.f;
        m[g] = need ? tmax : m[g];
        thr[g] = (m[g] + RESCALE_LOG2) * inv_scale_log2;
        lacc[g] *= alpha;
#pragma unroll
        for (int mt = 0; mt < MTILES; ++mt) acc[g][mt] *= alpha;
      }
      const float neg_m = -m[g];
      float pr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(fmaf(sc[j], p.scale_log2, neg_m));
      pb[g] = v4u32{ops::pack(pr[0], pr[1]), ops::pack(pr[2], pr[3]), ops::pack(pr[4], pr[5]),
                    ops::pack(pr[6], pr[7])};
      lacc[g] = ops::mma_k32(ones, pb[g], lacc[g]);
    }
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) {
      const u32x2_t v0 = lds_read_tr(vt + tr_off[0][mt]), v1 = lds_read_tr(vt + tr_off[1][mt]);
      const v4u32 va = v4u32{v0.x, v0.y, v1.x, v1.y};  // V^T[16mt + hl][keys 8 grp .. +7]
#pragma unroll
      for (int g = 0; g < NG; ++g) acc[g][mt] = ops::mma_k32(va, pb[g], acc[g][mt]);
    }
  };

  // registers -> LDS (16-bit values; FP8 codes widened with their row scale)
  auto store_tile = [&](const Staged &T, char *kt, char *vt) {
    char *mine = cp_v ? vt : kt;
#pragma unroll
    for (int u = 0; u < PPL; ++u) {
      if (!cp_ok[u]) continue;
      if constexpr (KV8) {
        const v4u32 w = T.d[u];
        const float sc = T.sc[u];
        *reinterpret_cast<v4u32 *>(mine + cp_lds[u]) =
            v4u32{fp8x2_scaled<Tag>(w.x, sc, false), fp8x2_scaled<Tag>(w.x, sc, true),
                  fp8x2_scaled<Tag>(w.y, sc, false), fp8x2_scaled<Tag>(w.y, sc, true)};
        *reinterpret_cast<v4u32 *>(mine + cp_lds2[u]) =
            v4u32{fp8x2_scaled<Tag>(w.z, sc, false), fp8x2_scaled<Tag>(w.z, sc, true),
                  fp8x2_scaled<Tag>(w.w, sc, false), fp8x2_scaled<Tag>(w.w, sc, true)};
      } else {
        *reinterpret_cast<v4u32 *>(mine + cp_lds[u]) = T.d[u];
      }
    }
  };

  // Tile j: store tile j + 1 (held in registers) into LDS stage (j + 1) % 2
  // and refill those registers with tile j + 1 + PF, compute tile j from
  // stage j % 2, then one barrier. Stage (j + 1) % 2 last held tile j - 1,
  // which every wave finished before the barrier ending step j - 1; tile j
  // was stored in step j - 1 and is visible after that barrier. The stores'
  // latency thus overlaps the compute instead of preceding the barrier
  // (8 x 4096 GQA-32/8: 1202-1218 -> 1181-1203 us; the 3k + 1k chunk
  // 512-558 -> 500-545 us). Even tiles stage through `ta`, odd ones
  // through `tb`; hol[s] keeps the hole bits of the tile in stage s.
  static_assert(PF == 2, "a tile and the one it is refilled with share a register set");
  auto step = [&](int j, Staged &Tn, uint32_t (&hol)[2]) {
    if (j + 1 < n_tiles) {
      store_tile(Tn, lds[(j + 1) & 1][0], lds[(j + 1) & 1][1]);
      hol[(j + 1) & 1] = Tn.holes;
      if (j + 1 + PF < n_tiles) fetch(j + 1 + PF, Tn);
    }
    compute(lds[j & 1][0], lds[j & 1][1], j * PT, hol[j & 1]);
    __syncthreads();
  };
  Staged ta, tb;
  uint32_t hol[2] = {0u, 0u};
  if (n_tiles > 0) {
    fetch(0, ta);
    if (n_tiles > 1) fetch(1, tb);
    store_tile(ta, lds[0][0], lds[0][1]);
    hol[0] = ta.holes;
    if (PF < n_tiles) fetch(PF, ta);
    __syncthreads();
  }
  for (int j = 0; j < n_tiles; j += 2) {
    step(j, tb, hol);
    if (j + 1 < n_tiles) step(j + 1, ta, hol);
  }

  // Normalise and store. Lane (hl, grp) holds O^T[16 mt + 4 grp + i][row hl].
  float lsum[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) lsum[g] = lacc[g][0];
  const int ph_first = pf_block(p, b, 0);
  const char *v0row = ph_first >= 0 && end > 0 ? vbase + (int64_t)ph_first * p.v_sb * CEB : nullptr;
  const float v0scale = KV8 && v0row ? p.v_scale[(int64_t)ph_first * p.s_sb + (int64_t)kvh * p.s_sh] : 0.f;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int64_t r = wr0 + 16 * g + hl;
    if (r >= rows_all) continue;
    const int64_t t = r / G;
    const int h = (int)(r % G);
    char *dst = p.out + (b * p.o_sb + ((int64_t)kvh * G + h) * p.o_sh + t * p.o_st + 4 * grp) * EB;
    if (r < rows_valid) {
      const float inv = 1.f / lsum[g];  // no attended key: 0/0 -> NaN
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt) {
        const f32x4_t o = acc[g][mt] * inv;
        const u32x2_t w = u32x2_t{ops::pack(o[0], o[1]), ops::pack(o[2], o[3])};
        *reinterpret_cast<u32x2_t *>(dst + 32 * mt) = w;
      }
    } else {
      // padding row: the value at position 0 (zero when its block is masked)
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt) {
        u32x2_t w = u32x2_t{0u, 0u};
        if (v0row) {
          if constexpr (KV8) {
            const uint32_t c = *reinterpret_cast<const uint32_t *>(v0row + 16 * mt + 4 * grp);
            w = u32x2_t{fp8x2_scaled<Tag>(c, v0scale, false), fp8x2_scaled<Tag>(c, v0scale, true)};
          } else {
            w = *reinterpret_cast<const u32x2_t *>(v0row + (16 * mt + 4 * grp) * EB);
          }
        }
        *reinterpret_cast<u32x2_t *>(dst + 32 * mt) = w;
      }
    }
  }
}

// ------------------------------------------------------------------ VALU
// One wave per (request, head, row). The lanes split the row's head_dim in
// 4-byte granules (one fp32 or two 16-bit elements; up to 4 per lane), walk
// the keys in order and keep an fp32 online softmax in the log2 domain.
template <typename Tag>
struct granule;
template <>
struct granule<f32_tag> {
  static constexpr int EB = 4, PER = 1;
  __device__ static inline void unpack(uint32_t w, float *x) { x[0] = __uint_as_float(w); }
  __device__ static inline uint32_t pack(const float *x) { return __float_as_uint(x[0]); }
};
template <>
struct granule<bf16_tag> {
  static constexpr int EB = 2, PER = 2;
  __device__ static inline void unpack(uint32_t w, float *x) {
    x[0] = elem<bf16_tag>::lo(w);
    x[1] = elem<bf16_tag>::hi(w);
  }
  __device__ static inline uint32_t pack(const float *x) { return elem<bf16_tag>::pack2(x[0], x[1]); }
};
template <>
struct granule<f16_tag> {
  static constexpr int EB = 2, PER = 2;
  __device__ static inline void unpack(uint32_t w, float *x) {
    x[0] = elem<f16_tag>::lo(w);
    x[1] = elem<f16_tag>::hi(w);
  }
  __device__ static inline uint32_t pack(const float *x) { return elem<f16_tag>::pack2(x[0], x[1]); }
};

__device__ inline float wave_sum(float v) { return sum_xor32(sum_xor16(group_sum<16>(v))); }

template <typename Tag>
__global__ __launch_bounds__(64) void paged_prefill_scalar_kernel(const PrefillParams p) {
  using GR = granule<Tag>;
  constexpr int EB = GR::EB, PER = GR::PER, MAXG = 4;
  const int lane = threadIdx.x;
  const int64_t idx = blockIdx.x;
  const int64_t t = idx % p.width;
  const int h = (int)((idx / p.width) % p.num_heads);
  const int64_t b = idx / (p.width * p.num_heads);
  const int kvh = h / p.heads_per_kv;
  const int ngr = p.head_dim * EB / 4;  // granules per row (<= 256)

  int64_t start, end, nrows;
  pf_range(p, b, &start, &end, &nrows);
  uint32_t *dst = reinterpret_cast<uint32_t *>(p.out + (b * p.o_sb + (int64_t)h * p.o_sh + t * p.o_st) * EB);
  const char *kbase = p.kc + (int64_t)kvh * p.k_sh * EB;
  const char *vbase = p.vc + (int64_t)kvh * p.v_sh * EB;

  if (t >= nrows) {  // padding row: the value at position 0
    const int ph = end > 0 ? pf_block(p, b, 0) : -1;
    const uint32_t *src = ph >= 0 ? reinterpret_cast<const uint32_t *>(vbase + (int64_t)ph * p.v_sb * EB) : nullptr;
    for (int gi = lane; gi < ngr; gi += 64) dst[gi] = src ? src[gi] : 0u;
    return;
  }

  float q[MAXG][PER], acc[MAXG][PER];
  const uint32_t *qrow = reinterpret_cast<const uint32_t *>(p.q + (b * p.q_sb + (int64_t)h * p.q_sh + t * p.q_st) * EB);
#pragma unroll
  for (int k = 0; k < MAXG; ++k) {
    const int gi = lane + 64 * k;
    GR::unpack(gi < ngr ? qrow[gi] : 0u, q[k]);
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[k][e] = 0.f;
  }
  float m = NEG_SENTINEL, l = 0.f;
  const int64_t kend = start + t + 1;
  int64_t cur_lb = -1;
  int ph = -1;
  for (int64_t kp = 0; kp < kend; ++kp) {
    const int64_t lb = pf_logical(p, kp);
    if (lb != cur_lb) {
      cur_lb = lb;
      ph = pf_block(p, b, lb);
    }
    if (ph < 0) continue;
    const int64_t off = kp - lb * p.block_size;
    const uint32_t *krow = reinterpret_cast<const uint32_t *>(kbase + ((int64_t)ph * p.k_sb + off * p.k_st) * EB);
    const uint32_t *vrow = reinterpret_cast<const uint32_t *>(vbase + ((int64_t)ph * p.v_sb + off * p.v_st) * EB);
    float s = 0.f;
    float vv[MAXG][PER];
#pragma unroll
    for (int k = 0; k < MAXG; ++k) {
      const int gi = lane + 64 * k;
      float kx[PER];
      GR::unpack(gi < ngr ? krow[gi] : 0u, kx);
      GR::unpack(gi < ngr ? vrow[gi] : 0u, vv[k]);
#pragma unroll
      for (int e = 0; e < PER; ++e) s = fmaf(q[k][e], kx[e], s);
    }
    s = wave_sum(s) * p.scale_log2;
    const float mn = fmaxf(m, s);
    const float alpha = fast_exp2(m - mn), pr = fast_exp2(s - mn);
    l = l * alpha + pr;
#pragma unroll
    for (int k = 0; k < MAXG; ++k)
#pragma unroll
      for (int e = 0; e < PER; ++e) acc[k][e] = acc[k][e] * alpha + pr * vv[k][e];
    m = mn;
  }
  const float inv = 1.f / l;  // no attended key: 0/0 -> NaN
#pragma unroll
  for (int k = 0; k < MAXG; ++k) {
    const int gi = lane + 64 * k;
    if (gi >= ngr) continue;
    float o[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] = acc[k][e] * inv;
    dst[gi] = GR::pack(o);
  }
}

template <typename Tag, int NG, bool KV8>
hipError_t launch_mfma_dim(int d, const PrefillParams &p, dim3 grid, hipStream_t s) {
  switch (d) {
    case 32: paged_prefill_mfma_kernel<Tag, 32, NG, KV8><<<grid, 64 * PWAVES, 0, s>>>(p); break;
    case 64: paged_prefill_mfma_kernel<Tag, 64, NG, KV8><<<grid, 64 * PWAVES, 0, s>>>(p); break;
    case 96: paged_prefill_mfma_kernel<Tag, 96, NG, KV8><<<grid, 64 * PWAVES, 0, s>>>(p); break;
    default: paged_prefill_mfma_kernel<Tag, 128, NG, KV8><<<grid, 64 * PWAVES, 0, s>>>(p); break;
  }
  return hipGetLastError();
}

bool prefill_mfma_supported(int dtype, int head_dim, int block_size) {
  return (dtype == IKL_F16 || dtype == IKL_BF16) &&
         (head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128) && block_size > 0 &&
         block_size % 16 == 0;
}

bool aligned(const void *ptr, int64_t bytes) { return ((uintptr_t)ptr) % bytes == 0; }

}  // namespace
}  // namespace ikl

using namespace ikl;

extern "C" int32_t ikl_paged_prefill_path(int32_t dtype, int32_t head_dim, int32_t block_size) {
  return prefill_mfma_supported(dtype, head_dim, block_size) ? IKL_PATH_MFMA_GROUPED : IKL_PATH_SCALAR_GROUPED;
}

extern "C" int ikl_paged_prefill_attention(const ikl_paged_prefill_args *a, void *stream) {
  if (!a) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: args is NULL");
  if (a->batch <= 0 || a->query_width <= 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 ||
      a->block_size <= 0 || a->num_blocks <= 0 || a->table_width <= 0)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: sizes must be positive");
  if (a->num_heads % a->num_kv_heads != 0)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: num_heads must be divisible by num_kv_heads");
  if (a->dtype != IKL_F16 && a->dtype != IKL_BF16 && a->dtype != IKL_F32)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: unknown dtype");
  if ((a->table_type != IKL_I32 && a->table_type != IKL_I64) || (a->lens_type != IKL_I32 && a->lens_type != IKL_I64))
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: unknown index type");
  if (!a->query || !a->k_cache || !a->v_cache || !a->block_tables || !a->query_starts || !a->context_lens || !a->out)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: NULL tensor pointer");
  const int eb = a->dtype == IKL_F32 ? 4 : 2;
  if (a->head_dim * eb % 4 != 0 || a->head_dim * eb > 1024)
    return fail(IKL_EUNSUPPORTED, "ikl_paged_prefill_attention: head_dim must give rows of 4k <= 1024 bytes");
  if (a->table_width > (int64_t(1) << 40) / a->block_size)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: table_width * block_size is too large");

  if (a->cache_dtype != 0 && a->cache_dtype != a->dtype && a->cache_dtype != IKL_FP8_E4M3)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: cache_dtype must be 0, the query dtype or IKL_FP8_E4M3");
  const bool kv8 = a->cache_dtype == IKL_FP8_E4M3;
  const int auto_path = ikl_paged_prefill_path(a->dtype, a->head_dim, a->block_size);
  const int path = a->path < 0 ? auto_path : a->path;
  if (kv8 && path != IKL_PATH_MFMA_GROUPED)
    return fail(IKL_EUNSUPPORTED, "ikl_paged_prefill_attention: the FP8 cache is read by the MFMA kernel only "
                                  "(fp16/bf16 queries, head_dim 32/64/96/128, block size a multiple of 16)");
  if (kv8 && (!a->k_scale || !a->v_scale || ((uintptr_t)a->k_scale & 3u) || ((uintptr_t)a->v_scale & 3u)))
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: the FP8 cache needs aligned k_scale / v_scale");
  const int ceb = kv8 ? 1 : eb;  // cache bytes per element
  if (path != IKL_PATH_MFMA_GROUPED && path != IKL_PATH_SCALAR_GROUPED)
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: path must be -1, IKL_PATH_SCALAR_GROUPED or IKL_PATH_MFMA_GROUPED");
  if (path == IKL_PATH_MFMA_GROUPED && auto_path != IKL_PATH_MFMA_GROUPED)
    return fail(IKL_EUNSUPPORTED, "ikl_paged_prefill_attention: no MFMA kernel for this dtype / head_dim / block_size");
  if (path == IKL_PATH_MFMA_GROUPED) {
    // 32-bit positions and 32-bit byte offsets inside a 16-row half tile
    if (a->table_width * a->block_size >= (int64_t(1) << 31) - 64)
      return fail(IKL_EINVAL, "ikl_paged_prefill_attention: table_width * block_size must stay below 2^31");
    if (16 * a->k_stride_token * ceb >= (int64_t(1) << 31) || 16 * a->v_stride_token * ceb >= (int64_t(1) << 31) ||
        a->k_stride_token < a->head_dim || a->v_stride_token < a->head_dim)
      return fail(IKL_EINVAL, "ikl_paged_prefill_attention: token strides must lie in [head_dim, 2^27)");
  }

  // every row the kernels touch must be aligned to its access width
  const int64_t align = path == IKL_PATH_MFMA_GROUPED ? 16 : 4;
  const int64_t out_align = path == IKL_PATH_MFMA_GROUPED ? 8 : 4;
  const int64_t q_strides[] = {a->q_stride_b, a->q_stride_h, a->q_stride_t};
  for (int64_t st : q_strides)
    if ((st * eb) % align != 0) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: misaligned input stride");
  const int64_t c_strides[] = {a->k_stride_block, a->k_stride_token, a->k_stride_head,
                               a->v_stride_block, a->v_stride_token, a->v_stride_head};
  for (int64_t st : c_strides)
    if ((st * ceb) % align != 0) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: misaligned input stride");
  const int64_t out_strides[] = {a->out_stride_b, a->out_stride_h, a->out_stride_t};
  for (int64_t st : out_strides)
    if ((st * eb) % out_align != 0) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: misaligned output stride");
  if (!aligned(a->query, align) || !aligned(a->k_cache, align) || !aligned(a->v_cache, align) ||
      !aligned(a->out, out_align))
    return fail(IKL_EINVAL, "ikl_paged_prefill_attention: misaligned tensor pointer");

  PrefillParams p{};
  p.q = static_cast<const char *>(a->query);
  p.q_sb = a->q_stride_b;
  p.q_sh = a->q_stride_h;
  p.q_st = a->q_stride_t;
  p.kc = static_cast<const char *>(a->k_cache);
  p.vc = static_cast<const char *>(a->v_cache);
  p.k_sb = a->k_stride_block;
  p.k_st = a->k_stride_token;
  p.k_sh = a->k_stride_head;
  p.v_sb = a->v_stride_block;
  p.v_st = a->v_stride_token;
  p.v_sh = a->v_stride_head;
  p.tables = a->block_tables;
  p.t_sb = a->table_stride_b;
  p.table_width = a->table_width;
  p.starts = a->query_starts;
  p.lens = a->context_lens;
  p.out = static_cast<char *>(a->out);
  p.o_sb = a->out_stride_b;
  p.o_sh = a->out_stride_h;
  p.o_st = a->out_stride_t;
  p.batch = a->batch;
  p.width = a->query_width;
  p.num_blocks = a->num_blocks;
  p.cap_tokens = a->table_width * a->block_size;
  p.num_heads = a->num_heads;
  p.num_kv_heads = a->num_kv_heads;
  p.heads_per_kv = a->num_heads / a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.block_size = a->block_size;
  p.bs_shift = (a->block_size & (a->block_size - 1)) == 0 ? __builtin_ctz((unsigned)a->block_size) : -1;
  p.table_i64 = a->table_type == IKL_I64;
  p.idx_i64 = a->lens_type == IKL_I64;
  const float scale = a->scale > 0.f ? a->scale : 1.f / sqrtf((float)a->head_dim);
  p.scale_log2 = scale * LOG2E;
  p.kv_fp8 = kv8 ? 1 : 0;
  p.k_scale = (const float *)a->k_scale;
  p.v_scale = (const float *)a->v_scale;
  p.s_sb = a->scale_stride_block;
  p.s_sh = a->scale_stride_head;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t ev0 = static_cast<hipEvent_t>(a->events[0]), ev1 = static_cast<hipEvent_t>(a->events[1]);
  if (ev0 && hipEventRecord(ev0, s) != hipSuccess) return check_launch("ikl_paged_prefill_attention: event record");
  hipError_t err;
  if (path == IKL_PATH_MFMA_GROUPED) {
    constexpr int NG = PREFILL_NG;
    const int64_t rows = a->query_width * p.heads_per_kv;
    constexpr int64_t rows_per_wg = 16 * NG * PWAVES;  // RWG of the kernel
    p.row_blocks = (rows + rows_per_wg - 1) / rows_per_wg;
    p.bh_pad = (a->batch * a->num_kv_heads + 7) / 8 * 8;
    // stream-major once a prefix has enough row blocks to fill an XCD's
    // resident workgroups (32 CUs x 2). GQA 32/8 hd128 bf16, 8 x 4096
    // prompts: FETCH_SIZE 3.50 -> 0.67 x the algorithmic bytes, kernel
    // 1252 -> 1238 us. Over the FP8 cache (half the K/V bytes per tile) it
    // measured 1.5 % slower (1270 -> 1289 us) and stays off.
    p.stream_major = p.row_blocks >= 64 && !p.kv_fp8;
    const int64_t blocks = p.row_blocks * p.bh_pad;
    if (blocks > 0x7fffffffLL) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: launch too large");
    const dim3 grid((unsigned)blocks);
    if (a->dtype == IKL_BF16)
      err = p.kv_fp8 ? launch_mfma_dim<bf16_tag, NG, true>(a->head_dim, p, grid, s)
                     : launch_mfma_dim<bf16_tag, NG, false>(a->head_dim, p, grid, s);
    else
      err = p.kv_fp8 ? launch_mfma_dim<f16_tag, NG, true>(a->head_dim, p, grid, s)
                     : launch_mfma_dim<f16_tag, NG, false>(a->head_dim, p, grid, s);
  } else {
    const int64_t blocks = a->batch * a->num_heads * a->query_width;
    if (blocks > 0x7fffffffLL) return fail(IKL_EINVAL, "ikl_paged_prefill_attention: launch too large");
    const dim3 grid((unsigned)blocks);
    if (a->dtype == IKL_BF16) paged_prefill_scalar_kernel<bf16_tag><<<grid, 64, 0, s>>>(p);
    else if (a->dtype == IKL_F16) paged_prefill_scalar_kernel<f16_tag><<<grid, 64, 0, s>>>(p);
    else paged_prefill_scalar_kernel<f32_tag><<<grid, 64, 0, s>>>(p);
    err = hipGetLastError();
  }
  if (err != hipSuccess) return fail(IKL_ELAUNCH, std::string("ikl_paged_prefill_attention: ") + hipGetErrorString(err));
  if (ev1 && hipEventRecord(ev1, s) != hipSuccess) return check_launch("ikl_paged_prefill_attention: event record");
  return IKL_OK;
}
