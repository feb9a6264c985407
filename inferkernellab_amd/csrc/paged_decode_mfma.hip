// Paged decode attention on the gfx950 matrix cores (MFMA family).
//
// Same result as the scalar family (paged_reference, attention.py:134-175);
// used for fp16/bf16 caches with head_dim in {32, 64, 96, 128} and a block
// size that is a multiple of 16. A wave attends one (request, kv head,
// query group of <= 16 heads) over a run of 16-token tiles (a tile never
// crosses a block, so it needs one block-table entry):
//
//   S^T[16 tok x 16 heads] = K[16 x D] . Q^T      D/32 v_mfma_f32_16x16x32
//   online softmax on S (lane = one head x 4 tokens; lazily rescaled)
//   O^T[D x 16 heads]     += V^T[D x 16] . P[16 x 16]   D/16 v_mfma_f32_16x16x16
//
// K and V tiles are loaded as whole rows (each load instruction covers
// 64 / (D * elem / 16) complete rows) and staged row-major in LDS (16-byte
// pieces rotated by row to spread banks). K comes back in the QK^T operand
// layout (lane l: 16 bytes of token l%16); V comes back transposed with
// ds_read_b64_tr_b16, which hands each lane four consecutive tokens of one
// head_dim column: the V^T operand. The S accumulator of lane l —
// P[tokens 4(l/16)..+3][head l%16] — is already the B operand of the PV
// MFMA.
//
// Two schedules share that tile loop:
//  * fixed partitions (paged_decode_mfma_kernel): a workgroup of WAVES
//    waves per (partition, unit, request); its waves split the partition's
//    tiles and merge their softmax states in LDS before one store;
//  * balanced split (paged_decode_mfma_streamk_kernel): exactly as many
//    workgroups as the GPU holds at once, each taking an equal run of the
//    batch's global tile sequence (see AttnParams::sk_waves) and splitting
//    each piece of it among its waves, so every wave starts once, streams
//    ~T/W tiles and all finish together.
//
// MFMA operand layouts and the transposing LDS read: see mfma_ops.h.
#include <atomic>
#include <type_traits>

#include "ikl_common.h"
#include "mfma_ops.h"
#include "paged_attn.h"

namespace ikl {
namespace {

constexpr int TILE = 16;  // tokens per tile
constexpr int CPOL_NT = 2;  // buffer-load cache policy: non-temporal (K/V rows are read once)

// Register budget: kernels with 16-head units ask for at least 2 waves per
// SIMD (VGPRs + AGPRs <= 256); the allocator then keeps their accumulators
// in VGPRs, without the accumulator-register copies it otherwise places in
// every tile (81 -> 78 us on the FP8 GQA decode workload). The 32-head
// kernels run one wave per SIMD (at two they would spill; two waves per SIMD
// at 217 VGPRs without the split masking path measured slower on MQA, 31.0
// against 28.4 us); the build keeps their accumulators in VGPRs as well
// (-amdgpu-mfma-vgpr-form for this file).
#define IKL_MFMA_WAVES_ATTR __attribute__((amdgpu_waves_per_eu(NG == 1 ? 2 : 1, 8)))

// bf16 P enters the PV product with its rounding residual in a second MFMA
// (fp16 P, <= 2^8, already keeps 11 bits and is not split). The FP8 cache
// skips it: its values carry 4 significant bits, far below what the
// residual would add.
template <typename Tag, bool KV8 = false>
constexpr bool split_p() {
  return !KV8 && mfma_ops<Tag>::NARROW_P;
}

// Two E4M3 codes -> two bf16 / fp16 values (exact: every E4M3 value is a
// bf16 and an fp16 value), as one packed dword. `hi` selects the upper
// code pair of `w`.
template <typename Tag>
__device__ inline uint32_t fp8x2_to(uint32_t w, bool hi);
template <>
__device__ inline uint32_t fp8x2_to<bf16_tag>(uint32_t w, bool hi) {
  return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                                        : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <>
__device__ inline uint32_t fp8x2_to<f16_tag>(uint32_t w, bool hi) {
  return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true)
                                        : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
// Eight codes (two dwords) -> one 16-byte MFMA operand of 8 elements.
template <typename Tag>
__device__ inline v4u32 fp8x8_to(uint32_t lo, uint32_t hi) {
  return v4u32{fp8x2_to<Tag>(lo, false), fp8x2_to<Tag>(lo, true), fp8x2_to<Tag>(hi, false),
               fp8x2_to<Tag>(hi, true)};
}

// Per-wave state of the tile loop: lane constants, the Q^T operands and the
// running softmax states (acc, m, lsum) of one (request, unit) run. A unit
// has up to NG * 16 query heads: NG 16-head MFMA groups share every K/V tile
// the wave loads (NG = 2 serves 32-head groups such as MQA-32 without
// reading K/V twice).
//
// KV8: the cache holds E4M3 codes with one fp32 scale per (token, head)
// row. K codes are widened in registers (the k order inside the QK^T
// product is free as long as Q uses the same one, so lane group g takes
// the contiguous elements [8 KSTEPS g, 8 KSTEPS (g + 1))), each score is
// multiplied by its token's K scale, the probabilities that enter the PV
// product by the token's V scale (the softmax sum keeps the unscaled
// ones), and V codes are widened on their way into the same LDS tile the
// 16-bit path stages.
template <typename Tag, int D, int NG, bool KV8>
struct WaveTiles {
  static_assert(D % 32 == 0 && D <= 128, "MFMA path needs head_dim = 32k <= 128");
  static_assert(NG == 1 || NG == 2, "one or two 16-head groups per wave");
  static constexpr int EB = 2;
  static constexpr int CEB = KV8 ? 1 : 2;                   // bytes per cache element
  static constexpr int NH = 16 * NG;                        // query heads per wave
  static constexpr int KSTEPS = D / 32;                     // QK^T k-steps
  static constexpr int MTILES = D / 16;                     // PV output tiles of 16 dims
  static constexpr int PIECES = D * EB / 16;                // 16-byte pieces per staged (16-bit) row
  static constexpr int ROWB = D * EB;                       // bytes per staged row
  static constexpr int CPIECES = D * CEB / 16;              // 16-byte pieces per cache row
  static constexpr int VLOADS = (TILE * CPIECES + 63) / 64; // 16-byte V loads per lane per tile
  static constexpr int VT_BYTES = TILE * ROWB;              // one staged V tile
  static constexpr int KROWB = D * CEB;                     // bytes per staged K row (codes for KV8)
  static constexpr int KT_BYTES = TILE * KROWB;             // one staged K tile
  static constexpr int TILE_BYTES = VT_BYTES + KT_BYTES;    // a wave's LDS during the tile loop
  // LDS reads of the QK^T operands per tile: one per k-step (16-bit; KV8
  // with odd KSTEPS, 8 bytes each), or one 16-byte read per two k-steps
  static constexpr int KREADS = KV8 && KSTEPS % 2 == 0 ? KSTEPS / 2 : KSTEPS;
  static constexpr int SROW = D + 4;                        // staged fp32 row (padded vs bank conflicts)
  static constexpr int ST_BYTES = NH * SROW * 4;            // one staged [NH heads x D] block
  using ops = mfma_ops<Tag>;
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

  struct Tile {
    v4u32 k[VLOADS];       // whole K rows, as V (KV8: codes)
    v4u32 v[VLOADS];
    f32x4_t ks, vs;        // KV8: scales of tokens 4 grp .. +3
    int n_valid;  // tokens of the tile inside the run with a valid block (0..16)
  };

  int lane, hl, grp;
  int k_lane[VLOADS], k_lds[VLOADS], k_rd[KREADS];
  int v_lds[VLOADS], v_lane[VLOADS], tr_lds[MTILES];
  v4u32 qb[NG][KSTEPS];
  f32x4_t acc[NG][MTILES];
  float m[NG], lsum[NG];

  // element offset of k-step s inside a row for this lane
  __device__ __forceinline__ int k_elem(int s) const { return KV8 ? 8 * KSTEPS * grp + 8 * s : 32 * s + 8 * grp; }

  __device__ __forceinline__ explicit WaveTiles(const AttnParams &p) {
    lane = threadIdx.x & 63;
    hl = lane & 15;   // MFMA row/column index inside a 16-lane group
    grp = lane >> 4;  // 16-lane group
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      // K and V cache piece: row pi / CPIECES, piece pi % CPIECES, so each
      // load instruction covers whole rows (a row is one contiguous
      // D * CEB-byte run; loads that cover 16 rows x 64 bytes each, the
      // MFMA operand's own shape, stream about 12 % slower on the GQA
      // decode workload's tiles). For KV8 the V piece widens into staged
      // pieces 2c, 2c + 1; K stays in codes.
      const int pi = u * 64 + lane;
      const int row = pi / CPIECES < TILE ? pi / CPIECES : TILE - 1, c = pi % CPIECES;
      const int sc = KV8 ? 2 * c : c;
      v_lds[u] = row * ROWB + ((sc + row) % PIECES) * 16;
      v_lane[u] = row * (int)p.v_st * CEB + c * 16;
      k_lds[u] = row * KROWB + ((c + row) % CPIECES) * 16;
      k_lane[u] = row * (int)p.k_st * CEB + c * 16;
    }
    // QK^T operand reads: k-step s of lane (hl, grp) is bytes [k_elem(s) CEB,
    // +8 CEB) of staged row hl (16-byte pieces rotated by row, as stored)
#pragma unroll
    for (int r = 0; r < KREADS; ++r) {
      const int byte = KV8 && KSTEPS % 2 == 0 ? k_elem(2 * r) : k_elem(r) * CEB;
      k_rd[r] = hl * KROWB + (((byte >> 4) + hl) % CPIECES) * 16 + (byte & 15);
    }
#pragma unroll
    for (int mt = 0; mt < MTILES; ++mt) {  // V^T reads: token 4g + (l%16)/4, dims 16mt + 4((l%16)%4)
      const int row = 4 * grp + (hl >> 2);
      const int c = 2 * mt + ((hl & 3) >> 1);
      tr_lds[mt] = row * ROWB + ((c + row) % PIECES) * 16 + (hl & 1) * 8;
    }
  }

  // Q^T operands: in group g, lane l holds q[hq0 + 16g + l%16][k_elem(s) .. +7]
  // (zero for heads >= nh).
  __device__ __forceinline__ void load_q(const AttnParams &p, int64_t b, int64_t hq0, int nh) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int h = 16 * g + hl;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        qb[g][s] = zero4();
        if (h < nh) qb[g][s] = load16v_global(p.q + (b * p.q_sb + (hq0 + h) * p.q_sh + k_elem(s)) * EB);
      }
    }
  }

  // Attends positions [t0, t1) of request b against kv head kvh (t0 is a
  // multiple of TILE) into fresh acc / m / lsum; lsum ends summed over the
  // four lane groups. vtile: this wave's TILE_BYTES of LDS (the staged V
  // tile, then the staged K tile).
  //
  // LOCKSTEP: the wave meets a workgroup barrier (no memory fence) every
  // two tiles, so the waves of a workgroup that walk the same blocks stay
  // together (every wave must call with the same tile count). has_pre_win:
  // pre_win is the table window starting at t0's block, already loaded by
  // the caller.
  // q_nh > 0: load the Q^T operands of heads [q_hq0, q_hq0 + q_nh) here,
  // after the first tile's loads are issued, so their latency overlaps.
  template <bool LOCKSTEP = false>
  __device__ __forceinline__ void attend(const AttnParams &p, int64_t b, int kvh, int64_t t0, int64_t t1,
                                         char *vtile, bool has_pre_win = false, int pre_win = 0,
                                         int64_t q_hq0 = 0, int q_nh = 0) {
    char *const ktile = vtile + VT_BYTES;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt) acc[g][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m[g] = NEG_SENTINEL;
      lsum[g] = 0.f;
    }
    const int n_tiles = t1 > t0 ? (int)((t1 - t0 + TILE - 1) / TILE) : 0;
    const char *kbase = p.kc + (int64_t)kvh * p.k_sh * CEB;
    const char *vbase = p.vc + (int64_t)kvh * p.v_sh * CEB;
    // KV8: the head's scale rows, in 64 bits (kvh * head stride may pass 4 GiB)
    const int64_t shead = KV8 ? (int64_t)kvh * p.s_sh * 4 : 0;
    const char *ksbase = KV8 ? (const char *)p.k_scale + shead : nullptr;
    const char *vsbase = KV8 ? (const char *)p.v_scale + shead : nullptr;
    // byte strides: blocks (< 2^32, checked by the host) and token rows
    const uint32_t kblk = (uint32_t)(p.k_sb * CEB), vblk = (uint32_t)(p.v_sb * CEB);
    const uint32_t kst = (uint32_t)(p.k_st * CEB), vst = (uint32_t)(p.v_st * CEB);
    const int bs = p.block_size;
    int64_t win_base = p.bs_shift >= 0 ? (t0 >> p.bs_shift) : t0 / bs;
    int win = has_pre_win ? pre_win : load_table_window(p, b, win_base, lane);

    // Resolves tile t's block and issues its K/V loads through buffer
    // resources whose record count ends at the tile's last valid row: rows
    // past it (all 16 for a masked block) read as zero, with no per-lane
    // address select and no branch around the loads.
    auto issue = [&](int t, Tile &T) {
      const int64_t base = t0 + (int64_t)t * TILE;
      const int64_t lb = p.bs_shift >= 0 ? (base >> p.bs_shift) : base / bs;
      if (lb >= win_base + 64) {
        win_base = lb;
        win = load_table_window(p, b, win_base, lane);
      }
      const uint32_t off = (uint32_t)(base - lb * bs);
      const int phys = __builtin_amdgcn_readlane(win, (int)(lb - win_base));
      const int64_t left = t1 - base;
      const int nv = phys < 0 || left <= 0 ? 0 : (left >= TILE ? TILE : (int)left);
      T.n_valid = nv;
      const uint32_t pu = phys < 0 ? 0u : (uint32_t)phys;
      const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(kbase + (uint64_t)pu * kblk + off * kst), (short)0, (int)(nv * kst), 0x00020000);
      const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(vbase + (uint64_t)pu * vblk + off * vst), (short)0, (int)(nv * vst), 0x00020000);
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) T.k[u] = __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane[u], 0, CPOL_NT);
      if constexpr (KV8) {
        // scales of tokens 4 grp .. +3 of the tile's block (16 bytes; a
        // masked block reads zero)
        const uint64_t so = (uint64_t)pu * (uint32_t)(p.s_sb * 4) + off * 4;
        const int sn = nv > 0 ? 64 : 0;
        const __amdgpu_buffer_rsrc_t ksr =
            __builtin_amdgcn_make_buffer_rsrc((void *)(ksbase + so), (short)0, sn, 0x00020000);
        const __amdgpu_buffer_rsrc_t vsr =
            __builtin_amdgcn_make_buffer_rsrc((void *)(vsbase + so), (short)0, sn, 0x00020000);
        T.ks = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ksr, 16 * grp, 0, CPOL_NT));
        T.vs = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(vsr, 16 * grp, 0, CPOL_NT));
      }
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) T.v[u] = __builtin_amdgcn_raw_buffer_load_b128(vr, v_lane[u], 0, CPOL_NT);
    };

    // partial: the tile has fewer than 16 valid rows (the run's last tile,
    // or a masked block). Full and partial tiles share this one body, the
    // masks behind a wave-uniform branch: a body compiled per case (masks
    // compiled out of full tiles) held the accumulators in two register
    // sets, copied between them where the cases met (32-head units: 256
    // VGPRs + 85 AGPRs of spills against 213 VGPRs; the GQA 32/8 decode
    // kernel over the FP8 cache 73.9-76.5 -> 72.8-74.7 us).
    auto compute = [&](Tile &T) {
      const bool partial = T.n_valid < TILE;
      wave_lds_sync();  // the previous tile's LDS reads come before these stores
      // stage V row-major in LDS (rows past the tile are never read)
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) {
        if (TILE * CPIECES % 64 == 0 || u * 64 + lane < TILE * CPIECES) {
          if constexpr (KV8) {
            const int row = (u * 64 + lane) / CPIECES;
            const int c2 = (((v_lds[u] - row * ROWB) / 16) + 1) % PIECES;  // rotated slot of piece 2c + 1
            *reinterpret_cast<v4u32 *>(vtile + v_lds[u]) = fp8x8_to<Tag>(T.v[u].x, T.v[u].y);
            *reinterpret_cast<v4u32 *>(vtile + row * ROWB + c2 * 16) = fp8x8_to<Tag>(T.v[u].z, T.v[u].w);
          } else {
            *reinterpret_cast<v4u32 *>(vtile + v_lds[u]) = T.v[u];
          }
        }
      }
      // stage K rows (codes for KV8) the same way, then read the QK^T
      // operands back in the MFMA layout: lane (hl, grp) takes row hl
#pragma unroll
      for (int u = 0; u < VLOADS; ++u) {
        if (TILE * CPIECES % 64 == 0 || u * 64 + lane < TILE * CPIECES)
          *reinterpret_cast<v4u32 *>(ktile + k_lds[u]) = T.k[u];
      }
      wave_lds_sync();  // every lane's stores come before any lane's reads
      // S^T of each group for tokens 4g' + i and head hl
      v4u32 ka[KSTEPS];
      if constexpr (!KV8) {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) ka[s] = *reinterpret_cast<const v4u32 *>(ktile + k_rd[s]);
      } else if constexpr (KSTEPS % 2 == 0) {
#pragma unroll
        for (int r = 0; r < KREADS; ++r) {
          const v4u32 w = *reinterpret_cast<const v4u32 *>(ktile + k_rd[r]);
          ka[2 * r] = fp8x8_to<Tag>(w.x, w.y);
          ka[2 * r + 1] = fp8x8_to<Tag>(w.z, w.w);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const u32x2v w = *reinterpret_cast<const u32x2v *>(ktile + k_rd[s]);
          ka[s] = fp8x8_to<Tag>(w.x, w.y);
        }
      }
      f32x4_t sa[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        sa[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) sa[g] = ops::mma_k32(ka[s], qb[g][s], sa[g]);
      }
      f32x4_t kscale = f32x4_t{p.scale_log2, p.scale_log2, p.scale_log2, p.scale_log2};
      f32x4_t vscale = f32x4_t{1.f, 1.f, 1.f, 1.f};
      if constexpr (KV8) {
        kscale = T.ks * p.scale_log2;
        vscale = T.vs;
        if (partial) {
#pragma unroll
          for (int i = 0; i < 4; ++i) vscale[i] = 4 * grp + i < T.n_valid ? vscale[i] : 0.f;
        }
      }
      u32x2_t pb[NG], pl[NG];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = sa[g][i] * kscale[i];
        if (partial) {
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[i] = 4 * grp + i < T.n_valid ? sc[i] : -INFINITY;
        }
        float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        tmax = max_xor32(max_xor16(tmax));
        const bool need = tmax > m[g] + RESCALE_LOG2;
        if (__builtin_amdgcn_ballot_w64(need) != 0ull) {
          const float alpha = need ? fast_exp2(m[g] - tmax) : 1.f;
          m[g] = need ? tmax : m[g];
          lsum[g] *= alpha;
#pragma unroll
          for (int mt = 0; mt < MTILES; ++mt) acc[g][mt] *= alpha;
        }
        float pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[i] = fast_exp2(sc[i] - m[g]);
          lsum[g] += pr[i];
          if constexpr (KV8) pr[i] *= vscale[i];  // the PV product takes p * v_scale
        }
        pb[g] = u32x2_t{ops::pack(pr[0], pr[1]), ops::pack(pr[2], pr[3])};
        // A bf16 P keeps 8 significant bits; with SPLIT_P its rounding
        // residual P - bf16(P) goes through a second MFMA, so P enters with
        // ~16 bits (as the fp32 P of the reference's kernels).
        if constexpr (split_p<Tag, KV8>())
          pl[g] = u32x2_t{ops::pack(pr[0] - ops::lo(pb[g].x), pr[1] - ops::hi(pb[g].x)),
                          ops::pack(pr[2] - ops::lo(pb[g].y), pr[3] - ops::hi(pb[g].y))};
      }
      // O^T += V^T P, every group on the same V^T operand
      s16x4_t va[MTILES];
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt) {
        va[mt] = __builtin_bit_cast(s16x4_t, lds_read_tr(vtile + tr_lds[mt]));
#pragma unroll
        for (int g = 0; g < NG; ++g)
          acc[g][mt] = ops::mma_k16(__builtin_bit_cast(u32x2_t, va[mt]), pb[g], acc[g][mt]);
      }
      if constexpr (split_p<Tag, KV8>()) {
#pragma unroll
        for (int mt = 0; mt < MTILES; ++mt)
#pragma unroll
          for (int g = 0; g < NG; ++g)
            acc[g][mt] = ops::mma_k16(__builtin_bit_cast(u32x2_t, va[mt]), pl[g], acc[g][mt]);
      }
    };

    auto run = [&](Tile &T) { compute(T); };
    // software pipeline: the next tile's loads fly while a tile computes (a
    // tile's registers taking the load two ahead right after it is staged
    // in LDS measured slower: GQA 32/8 hd128 bf16 B32 x U[4096, 8192]
    // 124.5 -> 126-128 us, its FP8-cache form 73 -> 80 us)
    Tile ta, tb;
    issue(0, ta);
    if (q_nh > 0) load_q(p, b, q_hq0, q_nh);
    for (int t = 0; t < n_tiles; t += 2) {
      if constexpr (LOCKSTEP) __builtin_amdgcn_s_barrier();
      issue(t + 1, tb);
      run(ta);
      issue(t + 2, ta);
      if (t + 1 < n_tiles) run(tb);
    }
    // combine the four lane groups' sums (m is already common to them)
#pragma unroll
    for (int g = 0; g < NG; ++g) lsum[g] = sum_xor32(sum_xor16(lsum[g]));
  }

  // Writes acc[g] * f[g] as rows [head 16g + hl][dims] of an [NH][SROW]
  // fp32 block, for heads < nh.
  __device__ __forceinline__ void stage(float *blk, const float *f, int nh) const {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int h = 16 * g + hl;
      if (h >= nh) continue;
#pragma unroll
      for (int mt = 0; mt < MTILES; ++mt)
        *reinterpret_cast<f32x4_t *>(blk + h * SROW + 16 * mt + 4 * grp) = acc[g][mt] * f[g];
    }
  }
};

// Sum of NSUM staged [NH][D + 4] blocks (consecutive) at head h, dims d .. d + 3.
template <int D, int NH, int NSUM>
__device__ __forceinline__ f32x4_t gather4(const float *st, int h, int d) {
  constexpr int SROW = D + 4;
  f32x4_t v = *reinterpret_cast<const f32x4_t *>(st + h * SROW + d);
#pragma unroll
  for (int w = 1; w < NSUM; ++w) v += *reinterpret_cast<const f32x4_t *>(st + w * NH * SROW + h * SROW + d);
  return v;
}

// nh rows of D fp32 (contiguous) from the staged blocks, 16 bytes a thread.
template <int D, int NH, int NSUM>
__device__ __forceinline__ void store_rows_f32(float *dst, const float *st, int nh, int tid, int nthreads) {
  for (int i = tid; i < nh * D / 4; i += nthreads)
    *reinterpret_cast<f32x4_t *>(dst + 4 * i) = gather4<D, NH, NSUM>(st, 4 * i / D, 4 * i % D);
}

// nh output rows (heads hq0.., stride o_sh elements) of request b, rounded
// to the output dtype, 16 bytes a thread.
template <typename Tag, int D, int NH, int NSUM>
__device__ __forceinline__ void store_rows_out(const AttnParams &p, int64_t b, int64_t hq0, const float *st,
                                               int nh, int tid, int nthreads) {
  constexpr int CPR = D / 8;  // 16-byte output pieces per head row
  for (int i = tid; i < nh * CPR; i += nthreads) {
    const int h = i / CPR, c = i % CPR;
    const f32x4_t lo = gather4<D, NH, NSUM>(st, h, 8 * c), hi = gather4<D, NH, NSUM>(st, h, 8 * c + 4);
    const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    store_out_chunk<Tag>(p.out + (b * p.o_sb + (hq0 + h) * p.o_sh + 8 * c) * 2, v);
  }
}

template <typename Tag, int D, int NG, int WAVES, bool KV8>
__global__ __launch_bounds__(64 * WAVES) IKL_MFMA_WAVES_ATTR void paged_decode_mfma_kernel(const AttnParams p) {
  static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4 || WAVES == 8, "1, 2, 4 or 8 waves per workgroup");
  using WT = WaveTiles<Tag, D, NG, KV8>;
  constexpr int NH = WT::NH;
  // LDS: each wave's V and K tiles during the loop; at the end each wave's
  // staged [NH heads x D] block, which the workgroup sums. The uses never
  // overlap.
  constexpr int SLOT = WT::ST_BYTES > WT::TILE_BYTES ? WT::ST_BYTES : WT::TILE_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[WAVES * SLOT];
  __shared__ float lds_m[WAVES][NH], lds_l[WAVES][NH];

  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Grid order (spread_grid): unit-fastest (unit, partition, request), or
  // request-fastest (request, unit, partition) with the request rotated by
  // partition % 8, which deals each request's partitions over the 8 XCDs
  // (MQA 32/1 hd128 B64 x U[1024, 4096]: 27.0 -> 26.4 us; GQA 32/4 B32 x
  // U[1024, 4096]: 48.7 -> 41.8 us; MQA B128 x U[1024, 4096]: 49.4 -> 47.1 us).
  const bool spread = p.grid_spread != 0;
  const int part = spread ? (int)blockIdx.z : (int)blockIdx.y;
  const int unit = spread ? (int)blockIdx.y : (int)blockIdx.x;
  const int kvh = unit / p.groups_per_kv;
  const int qg = unit % p.groups_per_kv;
  int64_t b = spread ? (int64_t)blockIdx.x + (blockIdx.z & 7u) : (int64_t)blockIdx.z;
  while (b >= p.batch) b -= p.batch;  // at most once for 8 or more requests

  const int64_t ctx = p.lens_i64 ? load_index<int64_t>(p.lens, b) : load_index<int32_t>(p.lens, b);
  const int64_t part_start = (int64_t)part * p.partition_size;
  if (part > 0 && part_start >= ctx) return;
  const int64_t part_end = ctx < part_start + p.partition_size ? ctx : part_start + p.partition_size;
  // The workgroup's waves take contiguous, equal (+-1) runs of the
  // partition's tiles: [w_start, w_end) for this wave.
  const int wg_tiles = part_end > part_start ? (int)((part_end - part_start + TILE - 1) / TILE) : 0;
  const int t_lo = wave * wg_tiles / WAVES, t_hi = (wave + 1) * wg_tiles / WAVES;
  const int64_t w_start = part_start + (int64_t)t_lo * TILE;
  const int64_t w_end = part_end < part_start + (int64_t)t_hi * TILE ? part_end : part_start + (int64_t)t_hi * TILE;

  WT wt(p);
  const int head0 = qg * p.group_size;
  const int nh = p.group_size < p.heads_per_kv - head0 ? p.group_size : p.heads_per_kv - head0;
  const int64_t hq0 = (int64_t)kvh * p.heads_per_kv + head0;
  wt.load_q(p, b, hq0, nh);
  wt.attend(p, b, kvh, w_start, w_end, lds + wave * WT::TILE_BYTES);

  // combine the workgroup's waves: common max M per head, rescaled sums
  float M[NG], L[NG], f[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    M[g] = wt.m[g];
    L[g] = wt.lsum[g];
  }
  if constexpr (WAVES > 1) {
    if (wt.grp == 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        lds_m[wave][16 * g + wt.hl] = wt.m[g];
        lds_l[wave][16 * g + wt.hl] = wt.lsum[g];
      }
    }
    __syncthreads();  // also ends every wave's use of its V tile
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const int h = 16 * g + wt.hl;
      M[g] = lds_m[0][h];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) M[g] = fmaxf(M[g], lds_m[w][h]);
      L[g] = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) L[g] += lds_l[w][h] * fast_exp2(lds_m[w][h] - M[g]);
    }
  }
  // Each wave stages its rescaled, normalised block; the workgroup sums the
  // blocks and stores whole 16-byte pieces (the heads are contiguous in the
  // output and in the [B, NP, H, D] partials).
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float inv = p.split ? (L[g] > 0.f ? 1.f / L[g] : 0.f) : 1.f / L[g];  // 0/0 -> NaN like the reference
    f[g] = (WAVES > 1 ? fast_exp2(wt.m[g] - M[g]) : 1.f) * inv;
  }
  float *const stage = reinterpret_cast<float *>(lds);
  wt.stage(stage + wave * NH * WT::SROW, f, nh);
  if constexpr (WAVES > 1) __syncthreads();
  else wave_lds_sync();
  if (p.split) {
    const int64_t prow = (b * p.num_parts + part) * p.num_heads + hq0;
    store_rows_f32<D, NH, WAVES>(p.part_o + prow * D, stage, nh, threadIdx.x, 64 * WAVES);
    if (wave == 0 && wt.grp == 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g)
        if (16 * g + wt.hl < nh) p.part_lse[prow + 16 * g + wt.hl] = L[g] > 0.f ? M[g] + log2f(L[g]) : -INFINITY;
    }
  } else {
    store_rows_out<Tag, D, NH, WAVES>(p, b, hq0, stage, nh, threadIdx.x, 64 * WAVES);
  }
}

// Start of balanced-split run w: the batch's total tiles T (units x
// request tiles), the run [g0, g1) = [w T / W, (w + 1) T / W) with W =
// min(sk_waves, T), and the request b holding tile g0 with its clamped
// length ctx, its tile count nb and the tiles pb of the requests before it
// (all from one scan of the lengths). Every lane of the calling
// wave gets the same values; `active` is false for runs past W.
struct SkRun {
  int64_t g0, g1, b, pb, ctx;
  int64_t lane_ctx;  // batches of up to 64 requests: lane q holds request q's clamped length
  int nb;
  bool active;
};

// The value of lane 0 (every lane of the wave holds the same one), in
// scalar registers: the split's bookkeeping comes out of cross-lane ops
// the compiler cannot prove uniform, and without this every buffer
// resource built from it (one per tile) would be wrapped in a loop over
// distinct lane values around each K/V load.
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ SkRun sk_run(const AttnParams &p, int64_t w, int lane) {
  SkRun r{0, 0, -1, 0, 0, 0, 0, false};
  const int64_t U = p.units / p.sk_unitw;  // sequence entries per request tile
  // total sequence entries, then the request holding the run's first entry
  // (a batch of up to 64 requests takes one scan for both); pb counts the
  // entries of the requests before b
  int64_t total, c1 = 0;
  int n1 = 0, incl1 = 0;
  if (p.batch <= 64) {
    c1 = lane < p.batch ? clamped_ctx(p, lane) : 0;
    n1 = (int)((c1 + 15) >> 4);
    incl1 = wave_incl_scan(seg_len(p, n1), lane);
    total = __builtin_amdgcn_readlane(incl1, 63);
  } else {
    int64_t before0;
    int own0;
    total = request_tiles(p, 0, lane, &before0, &own0);
  }
  const int64_t T = U * total;
  const int64_t W = (int64_t)p.sk_waves < T ? (int64_t)p.sk_waves : T;
  if (w >= W) return r;
  r.active = true;
  r.g0 = w * T / W;
  r.g1 = (w + 1) * T / W;

  if (p.batch <= 64) {
    const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < p.batch && U * incl1 > r.g0);
    const int l = __builtin_ctzll(hit);  // g0 < T: some request's tiles end past it
    r.b = l;
    r.nb = __shfl(n1, l, 64);
    r.pb = __shfl(incl1, l, 64) - seg_len(p, r.nb);
    r.ctx = ((int64_t)__shfl((int)(c1 >> 32), l, 64) << 32) | (uint32_t)__shfl((int)c1, l, 64);
    r.lane_ctx = c1;
  }
  int64_t base = 0;
  for (int64_t c0 = 0; c0 < p.batch && r.b < 0; c0 += 64) {
    const int64_t q = c0 + lane;
    const int64_t c = q < p.batch ? clamped_ctx(p, q) : 0;
    const int n = (int)((c + 15) >> 4);
    const int incl = wave_incl_scan(seg_len(p, n), lane);
    const uint64_t hit = __builtin_amdgcn_ballot_w64(q < p.batch && U * (base + incl) > r.g0);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      r.b = c0 + l;
      r.nb = __shfl(n, l, 64);
      r.pb = base + __shfl(incl, l, 64) - seg_len(p, r.nb);
      r.ctx = ((int64_t)__shfl((int)(c >> 32), l, 64) << 32) | (uint32_t)__shfl((int)c, l, 64);
    }
    base += __shfl(incl, 63, 64);
  }
  r.g0 = uniform64(r.g0);
  r.g1 = uniform64(r.g1);
  r.b = uniform64(r.b);
  r.pb = uniform64(r.pb);
  r.ctx = uniform64(r.ctx);
  r.nb = __builtin_amdgcn_readfirstlane(r.nb);
  return r;
}

// Moves a run to the next request with tiles after finishing request b's
// last unit (one exists while the run has tiles left), handing back the new
// request's clamped length.
// lane_ctx: the run's per-lane lengths from its scan (batches of up to 64
// requests), read across lanes instead of loaded again.
__device__ __forceinline__ void sk_next_request_ctx(const AttnParams &p, int64_t &b, int &nb, int64_t &pb,
                                                    int64_t &ctx, int64_t lane_ctx) {
  do {
    pb += seg_len(p, nb);
    ++b;
    if (p.batch <= 64)
      ctx = uniform64(((int64_t)__shfl((int)(lane_ctx >> 32), (int)b, 64) << 32) |
                      (uint32_t)__shfl((int)lane_ctx, (int)b, 64));
    else
      ctx = uniform64(clamped_ctx(p, b));
    nb = (int)((ctx + 15) >> 4);
  } while (nb == 0);
}

// Balanced split: p.sk_waves runs, one workgroup of WAVES waves each
// (grid.x). Workgroup w takes entries [w T / W, (w + 1) T / W) of the
// batch's sequence (T entries: per request and unit a segment of
// p.sk_seg_cost leading entries and then its tiles; W = min(sk_waves, T))
// piece by piece — a piece is the part of one (request, unit) segment
// inside the run, and a run that ends among a segment's leading entries
// has no piece there. Its waves take equal (+-1) shares of each piece's
// tiles and merge them in LDS, as the fixed partitions' workgroups do, and
// the piece's normalised output and log2-sum-exp go to partial slot unit +
// w. As in the unit-parallel kernel below, the next piece's length and
// table window load while a piece runs, and its Q loads behind its first
// tile.
template <typename Tag, int D, int NG, int WAVES, bool KV8>
__global__ __launch_bounds__(64 * WAVES) IKL_MFMA_WAVES_ATTR void paged_decode_mfma_streamk_kernel(const AttnParams p) {
  static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4, "1, 2 or 4 waves per workgroup");
  using WT = WaveTiles<Tag, D, NG, KV8>;
  constexpr int NH = WT::NH;
  // LDS: each wave's V and K tiles during a piece; at its end each wave's
  // staged [NH heads x D] block, which the workgroup sums (separated by
  // barriers).
  constexpr int SLOT = WT::ST_BYTES > WT::TILE_BYTES ? WT::ST_BYTES : WT::TILE_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[WAVES * SLOT];
  __shared__ float lds_m[WAVES][NH], lds_l[WAVES][NH];
  const int lane = (int)(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t U = p.units;
  const int64_t w = blockIdx.x;
  // every wave computes the same run: the loop below is uniform over the
  // workgroup, so its barriers are met by all waves
  const SkRun run = sk_run(p, w, lane);
  if (!run.active) return;
  const int64_t g0 = run.g0, g1 = run.g1;
  int64_t b = run.b, pb = run.pb;
  int nb = run.nb;

  WT wt(p);
  float *const stage = reinterpret_cast<float *>(lds);
  int64_t g = g0;
  int64_t ctx = run.ctx;
  int win = 0;
  bool have_win = false;
  const int64_t c = p.sk_seg_cost;
  while (true) {
    // piece: unit u of request b, segment entries [v_in, v_hi), request
    // tiles [t_in, t_hi)
    const int64_t sl = seg_len(p, nb);
    const int64_t rel = g - U * pb;
    const int u = (int)(rel / sl);
    const int64_t v_in = rel - (int64_t)u * sl;
    const int64_t v_hi = sl < v_in + (g1 - g) ? sl : v_in + (g1 - g);
    const int64_t t_in = v_in > c ? v_in - c : 0, t_hi = v_hi > c ? v_hi - c : 0;
    const int kvh = u / p.groups_per_kv, qg = u % p.groups_per_kv;
    const int head0 = qg * p.group_size;
    const int nh = p.group_size < p.heads_per_kv - head0 ? p.group_size : p.heads_per_kv - head0;
    const int64_t hq0 = (int64_t)kvh * p.heads_per_kv + head0;
    // this wave's share of the piece: tiles [a0, a1), positions [a0 * 16, e)
    const int64_t n = t_hi - t_in;
    const int64_t a0 = t_in + wave * n / WAVES, a1 = t_in + (wave + 1) * n / WAVES;
    const int64_t e = a1 * TILE < ctx ? a1 * TILE : ctx;
    // the run's next piece starts at tile 0 of unit u + 1, or of the next
    // request with tiles: its length and this wave's first table window
    // load now, and its Q loads behind its first tile (as in the
    // unit-parallel kernel; each piece start otherwise waited out three
    // dependent loads: MQA 32/1 hd128 bf16 B64 x U[1024, 4096], balanced
    // split, runs crossing a request ended 4-6 us after the others)
    const int64_t gn = g + (v_hi - v_in);
    int64_t bn = b, pbn = pb, ctxn = ctx;
    int nbn = nb, win_n = 0;
    if (gn < g1) {
      if (v_hi == sl && u == U - 1) sk_next_request_ctx(p, bn, nbn, pbn, ctxn, run.lane_ctx);  // one exists: gn < T
      const int64_t ve = seg_len(p, nbn) < g1 - gn ? seg_len(p, nbn) : g1 - gn;
      const int64_t nn = ve > c ? ve - c : 0;  // the next piece's tiles
      const int64_t blk = (int64_t)(wave * nn / WAVES) * TILE;
      win_n = load_table_window(p, bn, p.bs_shift >= 0 ? (blk >> p.bs_shift) : blk / p.block_size, lane);
    }
    if (n == 0) {  // the run ends inside the segment's leading entries: no tiles, no partial
      g = gn;
      if (g >= g1) break;
      b = bn;
      pb = pbn;
      nb = nbn;
      ctx = ctxn;
      win = win_n;
      have_win = true;
      continue;
    }
    wt.attend(p, b, kvh, a0 * TILE, a1 > a0 ? e : a0 * TILE, lds + wave * WT::TILE_BYTES, have_win, win, hq0, nh);

    // combine the waves: common max M per head, rescaled sums
    float M[NG], L[NG], f[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      M[gi] = wt.m[gi];
      L[gi] = wt.lsum[gi];
    }
    if constexpr (WAVES > 1) {
      if (wt.grp == 0) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          lds_m[wave][16 * gi + wt.hl] = wt.m[gi];
          lds_l[wave][16 * gi + wt.hl] = wt.lsum[gi];
        }
      }
      __syncthreads();  // also ends every wave's use of its V tile
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const int h = 16 * gi + wt.hl;
        M[gi] = lds_m[0][h];
#pragma unroll
        for (int k = 1; k < WAVES; ++k) M[gi] = fmaxf(M[gi], lds_m[k][h]);
        L[gi] = 0.f;
#pragma unroll
        for (int k = 0; k < WAVES; ++k) L[gi] += lds_l[k][h] * fast_exp2(lds_m[k][h] - M[gi]);
      }
    } else {
      wave_lds_sync();
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
      f[gi] = (WAVES > 1 ? fast_exp2(wt.m[gi] - M[gi]) : 1.f) * (L[gi] > 0.f ? 1.f / L[gi] : 0.f);
    wt.stage(stage + wave * NH * WT::SROW, f, nh);
    if constexpr (WAVES > 1) __syncthreads();
    else wave_lds_sync();
    const int64_t slot = b * U + u + w;
    store_rows_f32<D, NH, WAVES>(p.part_o + slot * p.group_size * D, stage, nh, (int)threadIdx.x, 64 * WAVES);
    if (wave == 0 && wt.grp == 0) {
#pragma unroll
      for (int gi = 0; gi < NG; ++gi)
        if (16 * gi + wt.hl < nh)
          p.part_lse[slot * p.group_size + 16 * gi + wt.hl] = L[gi] > 0.f ? M[gi] + log2f(L[gi]) : -INFINITY;
    }
    // the staged blocks are read before the next piece's V tiles overwrite them
    if constexpr (WAVES > 1) __syncthreads();
    else wave_lds_sync();

    g = gn;
    if (g >= g1) break;
    b = bn;
    pb = pbn;
    nb = nbn;
    ctx = ctxn;
    win = win_n;
    have_win = true;
  }
}

// Unit-parallel balanced split: p.sk_waves workgroups of UW waves, for
// units of up to 16 heads. The sequence is request-major, then unit group
// (UW consecutive units: a segment of p.sk_seg_cost leading entries, then
// its tiles); workgroup w takes the run [w T / W, (w + 1) T / W) of it and
// its wave i attends unit ug * UW + i over each
// piece — so the UW waves read their heads' rows of the same cache blocks
// at about the same time (in the token-major cache those rows interleave
// inside each block). A load-only probe of the GQA 32/8 hd128 bf16 B32 x
// U[4096, 8192] pattern streams it in 115 us this way against 126 us as
// one-unit runs. The waves meet a barrier every two tiles, which keeps them
// on the same blocks (that shape's kernel 131 -> 127 us; every wave of the
// workgroup walks the same tile counts); they share no LDS. Each writes its
// own unit's normalised partial and log2-sum-exp per piece, to slot
// ((b * NUG + ug) + w) * UW + i (NUG = units / UW groups per request).
// While a piece runs, the next piece's context length and first table
// window are already loaded, and each piece's Q rows load behind its first
// tile's K/V, so a piece boundary exposes one memory round trip instead of
// three.
template <typename Tag, int D, int UW, bool KV8>
__global__ __launch_bounds__(64 * UW) __attribute__((amdgpu_waves_per_eu(2, 8))) void paged_decode_mfma_unitk_kernel(
    const AttnParams p) {
  using WT = WaveTiles<Tag, D, 1, KV8>;
  constexpr int NH = WT::NH;
  // LDS: per wave, its V and K tiles during a piece, then its staged
  // [NH heads x D] block (the wave's own region; waves do not share LDS)
  constexpr int SLOT = WT::ST_BYTES > WT::TILE_BYTES ? WT::ST_BYTES : WT::TILE_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[UW * SLOT];
  const int lane = (int)(threadIdx.x & 63u);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t NUG = p.units / UW;
  const int64_t w = blockIdx.x;
  const SkRun run = sk_run(p, w, lane);
  if (!run.active) return;
  const int64_t g1 = run.g1;
  int64_t g = run.g0, b = run.b, pb = run.pb;
  int nb = run.nb;
  char *const mine = lds + wave * SLOT;
  float *const stage = reinterpret_cast<float *>(mine);

  WT wt(p);
  int64_t ctx = run.ctx;
  int win = 0;
  bool have_win = false;
  const int64_t c = p.sk_seg_cost;
  while (true) {
    // piece: unit group ug of request b, segment entries [v_in, v_hi),
    // request tiles [t_in, t_hi)
    const int64_t sl = seg_len(p, nb);
    const int64_t rel = g - NUG * pb;
    const int64_t ug = rel / sl;
    const int64_t v_in = rel - ug * sl;
    const int64_t v_hi = sl < v_in + (g1 - g) ? sl : v_in + (g1 - g);
    const int64_t t_in = v_in > c ? v_in - c : 0, t_hi = v_hi > c ? v_hi - c : 0;
    const int u = (int)ug * UW + wave;
    const int kvh = u / p.groups_per_kv, qg = u % p.groups_per_kv;
    const int head0 = qg * p.group_size;
    const int nh = p.group_size < p.heads_per_kv - head0 ? p.group_size : p.heads_per_kv - head0;
    const int64_t hq0 = (int64_t)kvh * p.heads_per_kv + head0;
    const int64_t e = t_hi * TILE < ctx ? t_hi * TILE : ctx;
    // the run's next piece starts at tile 0 of group ug + 1, or of the next
    // request with tiles: its length and first window load now
    const int64_t gn = g + (v_hi - v_in);
    int64_t bn = b, pbn = pb, ctxn = ctx;
    int nbn = nb, win_n = 0;
    if (gn < g1) {
      if (v_hi == sl && ug == NUG - 1) sk_next_request_ctx(p, bn, nbn, pbn, ctxn, run.lane_ctx);  // one exists: gn < T
      win_n = load_table_window(p, bn, 0, lane);
    }
    if (t_hi == t_in) {  // the run ends inside the segment's leading entries: no tiles, no partial
      g = gn;
      if (g >= g1) break;
      b = bn;
      pb = pbn;
      nb = nbn;
      ctx = ctxn;
      win = win_n;
      have_win = true;
      continue;
    }
    wt.template attend<true>(p, b, kvh, t_in * TILE, e, mine, have_win, win, hq0, nh);
    const float L = wt.lsum[0], M = wt.m[0];
    const float f[1] = {L > 0.f ? 1.f / L : 0.f};
    wave_lds_sync();  // the tile loop's LDS reads come before the staged block
    wt.stage(stage, f, nh);
    wave_lds_sync();
    const int64_t slot = ((b * NUG + ug) + w) * UW + wave;
    store_rows_f32<D, NH, 1>(p.part_o + slot * p.group_size * D, stage, nh, lane, 64);
    if (wt.grp == 0 && wt.hl < nh) p.part_lse[slot * p.group_size + wt.hl] = L > 0.f ? M + log2f(L) : -INFINITY;
    wave_lds_sync();  // the staged block is read before the next piece's tiles overwrite it

    g = gn;
    if (g >= g1) break;
    b = bn;
    pb = pbn;
    nb = nbn;
    ctx = ctxn;
    win = win_n;
    have_win = true;
  }
}

// Waves sharing one fixed partition: 4. For 32-head units that is 68 KB
// of LDS at 128 dims (their staged [32 x D] blocks), two workgroups and
// two waves per SIMD on a CU; with 2 waves per workgroup, one per SIMD,
// each wave walked twice the tiles (MQA 32/1 hd128 bf16 step, planned as
// below: B64 x U[1024, 4096] 27.4 -> 26.3 us, B16 x U[1024, 4096] 16.5 ->
// 14.6, B64 x 2048 23.9 -> 21.3, over the FP8 cache B64 x U[1024, 4096]
// 26.9 -> 22.7). Over the FP8 cache the planner can give 32-head units
// 8-wave workgroups (p.fixed_waves) for 1024-token partitions: 135 KB of LDS
// at 128 dims, one workgroup and two waves per SIMD on a CU, each wave
// walking 8 tiles.
template <int NG>
constexpr int wg_waves() {
  return 4;
}

// Waves per balanced-split workgroup. 32-head units take 4: their pieces'
// partials are 16 KB each, and merging the waves' shares in LDS divides
// them (MQA 32/1 hd128 bf16, kernel: B64 x U[1024, 4096] 28.8 -> 27.5 us
// from 1 to 2 waves, B128 41.8 -> 40.3, B32 x U[4096, 8192] 31.0 -> 29.6;
// whole step from 2 to 4 waves: B128 x U[1024, 4096] 43.9-44.6 -> 42.1-42.2
// us, B48 x U[4096, 8192] 38.1-38.2 -> 36.3-36.7, over the FP8 cache
// unchanged). 16-head units keep one wave per run: with 4 waves sharing
// each piece a wave meets more piece starts and barriers, and the GQA 32/8
// bf16 B32 x U[4096, 8192] kernel went from 137.7 to 144.1 us.
template <int NG>
constexpr int sk_wg_waves() {
  return NG == 1 ? 1 : 4;
}

template <typename Tag, int D, int NG, bool KV8>
void launch_shape(const AttnParams &p, dim3 grid, hipStream_t s) {
  if constexpr (NG == 1) {
    if (p.sk_waves > 0 && p.sk_unitw > 1) {
      const dim3 g((unsigned)p.sk_waves);
      switch (p.sk_unitw) {
        case 2: paged_decode_mfma_unitk_kernel<Tag, D, 2, KV8><<<g, dim3(128), 0, s>>>(p); break;
        case 4: paged_decode_mfma_unitk_kernel<Tag, D, 4, KV8><<<g, dim3(256), 0, s>>>(p); break;
        default: paged_decode_mfma_unitk_kernel<Tag, D, 8, KV8><<<g, dim3(512), 0, s>>>(p); break;
      }
      return;
    }
  }
  if (p.sk_waves > 0) {
    constexpr int SKW = sk_wg_waves<NG>();
    paged_decode_mfma_streamk_kernel<Tag, D, NG, SKW, KV8><<<dim3((unsigned)p.sk_waves), dim3(64 * SKW), 0, s>>>(p);
    return;
  }
  // grid arrives as (partition, unit, request)
  grid = p.grid_spread ? dim3(grid.z, grid.y, grid.x) : dim3(grid.y, grid.x, grid.z);
  if constexpr (NG == 2 && KV8) {
    if (p.fixed_waves == 8) {
      paged_decode_mfma_kernel<Tag, D, NG, 8, KV8><<<grid, dim3(512), 0, s>>>(p);
      return;
    }
  }
  constexpr int WAVES = wg_waves<NG>();
  paged_decode_mfma_kernel<Tag, D, NG, WAVES, KV8><<<grid, dim3(64 * WAVES), 0, s>>>(p);
}

template <typename Tag, int NG, bool KV8>
void launch_dim(int d, const AttnParams &p, dim3 grid, hipStream_t s) {
  switch (d) {
    case 32: launch_shape<Tag, 32, NG, KV8>(p, grid, s); break;
    case 64: launch_shape<Tag, 64, NG, KV8>(p, grid, s); break;
    case 96: launch_shape<Tag, 96, NG, KV8>(p, grid, s); break;
    default: launch_shape<Tag, 128, NG, KV8>(p, grid, s); break;
  }
}

template <typename Tag, int NG>
void launch_kv(int d, const AttnParams &p, dim3 grid, hipStream_t s) {
  if (p.kv_fp8) launch_dim<Tag, NG, true>(d, p, grid, s);
  else launch_dim<Tag, NG, false>(d, p, grid, s);
}

// Resident workgroups of a kernel on the current device (CUs x workgroups
// per CU, its registers and LDS included), cached per device; 256 CUs x
// the kernel's waves per CU (8 for 16-head units, 4 for 32-head) / its
// waves per workgroup when no device answers (planning on a host without a
// GPU).
template <typename K>
int resident_capacity(K kernel, int threads, int waves_per_cu, std::atomic<int> *cache) {
  constexpr int MAX_DEV = 64;
  const int fallback = 256 * waves_per_cu / (threads / 64);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
    (void)hipGetLastError();
    return fallback;
  }
  // Written once per device by whichever thread gets there first; every
  // writer stores the same value, and readers see 0 (query again) or it.
  const int known = cache[dev].load(std::memory_order_acquire);
  if (known > 0) return known;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || cus <= 0 ||
      per_cu <= 0) {
    (void)hipGetLastError();
    return fallback;
  }
  cache[dev].store(cus * per_cu, std::memory_order_release);
  return cus * per_cu;
}

template <typename Tag, int D, int NG, bool KV8>
int streamk_capacity_for(int unitw) {
  constexpr int SKW = sk_wg_waves<NG>();
  if constexpr (NG == 1) {
    static std::atomic<int> c2[64] = {}, c4[64] = {}, c8[64] = {};
    switch (unitw) {
      case 2: return resident_capacity(paged_decode_mfma_unitk_kernel<Tag, D, 2, KV8>, 128, 8, c2);
      case 4: return resident_capacity(paged_decode_mfma_unitk_kernel<Tag, D, 4, KV8>, 256, 8, c4);
      case 8: return resident_capacity(paged_decode_mfma_unitk_kernel<Tag, D, 8, KV8>, 512, 8, c8);
      default: break;
    }
  }
  static std::atomic<int> c1[64] = {};
  return resident_capacity(paged_decode_mfma_streamk_kernel<Tag, D, NG, SKW, KV8>, 64 * SKW, NG == 1 ? 8 : 4, c1);
}

// Resident workgroups of the fixed-partition kernel (its LDS included;
// without a device, two waves per SIMD).
template <typename Tag, int D, int NG, bool KV8>
int fixed_capacity_for() {
  constexpr int WAVES = wg_waves<NG>();
  static std::atomic<int> c[64] = {};
  return resident_capacity(paged_decode_mfma_kernel<Tag, D, NG, WAVES, KV8>, 64 * WAVES, 8, c);
}

// The same for the 8-wave form of 32-head units over the FP8 cache.
template <typename Tag, int D>
int fixed8_capacity_for() {
  static std::atomic<int> c[64] = {};
  return resident_capacity(paged_decode_mfma_kernel<Tag, D, 2, 8, true>, 512, 8, c);
}

template <typename Tag>
int fixed8_capacity_dim(int d) {
  switch (d) {
    case 32: return fixed8_capacity_for<Tag, 32>();
    case 64: return fixed8_capacity_for<Tag, 64>();
    case 96: return fixed8_capacity_for<Tag, 96>();
    default: return fixed8_capacity_for<Tag, 128>();
  }
}

template <typename Tag, int NG, bool KV8>
int fixed_capacity_dim(int d) {
  switch (d) {
    case 32: return fixed_capacity_for<Tag, 32, NG, KV8>();
    case 64: return fixed_capacity_for<Tag, 64, NG, KV8>();
    case 96: return fixed_capacity_for<Tag, 96, NG, KV8>();
    default: return fixed_capacity_for<Tag, 128, NG, KV8>();
  }
}

template <typename Tag, int NG, bool KV8>
int capacity_dim(int d, int unitw) {
  switch (d) {
    case 32: return streamk_capacity_for<Tag, 32, NG, KV8>(unitw);
    case 64: return streamk_capacity_for<Tag, 64, NG, KV8>(unitw);
    case 96: return streamk_capacity_for<Tag, 96, NG, KV8>(unitw);
    default: return streamk_capacity_for<Tag, 128, NG, KV8>(unitw);
  }
}

template <typename Tag, int NG>
int capacity_kv(int d, bool kv8, int unitw) {
  return kv8 ? capacity_dim<Tag, NG, true>(d, unitw) : capacity_dim<Tag, NG, false>(d, unitw);
}

}  // namespace

bool mfma_supported(int dtype, int head_dim, int block_size, int group_size) {
  return (dtype == IKL_F16 || dtype == IKL_BF16) &&
         (head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128) &&
         block_size > 0 && block_size % 16 == 0 && group_size >= 1 && group_size <= 32;
}

hipError_t launch_mfma_attention(int dtype, int head_dim, const AttnParams &p, dim3 grid, hipStream_t s) {
  const bool two = p.group_size > 16;
  if (dtype == IKL_BF16) {
    if (two) launch_kv<bf16_tag, 2>(head_dim, p, grid, s);
    else launch_kv<bf16_tag, 1>(head_dim, p, grid, s);
  } else {
    if (two) launch_kv<f16_tag, 2>(head_dim, p, grid, s);
    else launch_kv<f16_tag, 1>(head_dim, p, grid, s);
  }
  return hipGetLastError();
}

MfmaShape mfma_launch_shape(bool balanced, int group_size, int unitw, int fixed_waves) {
  if (balanced && group_size <= 16 && unitw > 1) return MfmaShape{TILE, unitw, 2};
  if (!balanced && group_size > 16 && fixed_waves == 8) return MfmaShape{TILE, 8, 2};
  const int waves = group_size > 16 ? (balanced ? sk_wg_waves<2>() : wg_waves<2>())
                                    : (balanced ? sk_wg_waves<1>() : wg_waves<1>());
  return MfmaShape{TILE, waves, 2};
}

int mfma_streamk_capacity(int dtype, int head_dim, int group_size, bool kv_fp8, int unitw) {
  const bool bf = dtype == IKL_BF16, two = group_size > 16;
  if (bf)
    return two ? capacity_kv<bf16_tag, 2>(head_dim, kv_fp8, 1) : capacity_kv<bf16_tag, 1>(head_dim, kv_fp8, unitw);
  return two ? capacity_kv<f16_tag, 2>(head_dim, kv_fp8, 1) : capacity_kv<f16_tag, 1>(head_dim, kv_fp8, unitw);
}

int mfma_fixed_capacity(int dtype, int head_dim, int group_size, bool kv_fp8) {
  const bool two = group_size > 16;
  if (dtype == IKL_BF16) {
    if (two) return kv_fp8 ? fixed_capacity_dim<bf16_tag, 2, true>(head_dim) : fixed_capacity_dim<bf16_tag, 2, false>(head_dim);
    return kv_fp8 ? fixed_capacity_dim<bf16_tag, 1, true>(head_dim) : fixed_capacity_dim<bf16_tag, 1, false>(head_dim);
  }
  if (two) return kv_fp8 ? fixed_capacity_dim<f16_tag, 2, true>(head_dim) : fixed_capacity_dim<f16_tag, 2, false>(head_dim);
  return kv_fp8 ? fixed_capacity_dim<f16_tag, 1, true>(head_dim) : fixed_capacity_dim<f16_tag, 1, false>(head_dim);
}

int mfma_fixed8_capacity(int dtype, int head_dim) {
  return dtype == IKL_BF16 ? fixed8_capacity_dim<bf16_tag>(head_dim) : fixed8_capacity_dim<f16_tag>(head_dim);
}

int mfma_cu_count() {
  constexpr int MAX_DEV = 64;
  static std::atomic<int> cache[MAX_DEV] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
    (void)hipGetLastError();
    return 256;
  }
  const int known = cache[dev].load(std::memory_order_acquire);
  if (known > 0) return known;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cache[dev].store(cus, std::memory_order_release);
  return cus;
}

int mfma_streamk_unitw(int64_t units, int group_size) {
  if (group_size > 16) return 1;
  for (int c : {8, 4, 2})
    if (units % c == 0) return c;
  return 1;
}

}  // namespace ikl
