// Fused rotary embedding + KV append: one launch per layer and step for
// the step before paged decode attention (hf_benchmark.py:419-436): rotate
// q and k with rotate-half RoPE (hf_benchmark.py:69-85), write the rotated
// k and the raw v into the paged cache at their slots (as append.py:19-66 /
// cache.py:156-189 would after a separate rotation), and write the rotated
// q for the attention that follows.
//
// Bit-exact with the reference's torch sequence: with cos / sin rows in the
// tensors' dtype, torch computes t1 = round(x * cos), t2 =
// round(rotate_half(x) * sin) and round(t1 + t2), each elementwise op
// evaluated in fp32 and rounded once. A product of two fp16 / bf16 values
// is exact in fp32, so doing the same three roundings here reproduces it;
// fp32 tensors round each product before the add for the same reason.
//
// Layout: one workgroup per token; each thread takes 16-byte chunk c of the
// first half of a q or k row together with chunk c of the second half
// (rotate-half pairs element i with element i +- D/2), and v rows are
// copied in 16-byte chunks. Slots outside the cache are skipped.
#include "ikl_common.h"

namespace ikl {
namespace {

// A rounded product must reach the add as a value, not as a multiply the
// compiler may fuse into it (fp16: shrunk to half ops and v_fma_mix /
// v_fma_f16; fp32: v_fma_f32, also through __fmul_rn, whose header is
// compiled with contraction on). An empty asm with a VGPR operand makes the
// value opaque to every later pass.
__device__ inline float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

struct RopeParams {
  const char *q_in;
  char *q_out;
  int64_t qi_st, qi_sh, qo_st, qo_sh;  // bytes
  const char *key;
  const char *value;
  int64_t k_st, k_sh, v_st, v_sh;      // bytes
  const char *cos;
  const char *sin;
  int64_t cos_st, sin_st;              // bytes
  const void *slots;
  char *kc;
  char *vc;
  int64_t kc_sb, kc_st, kc_sh;         // bytes
  int64_t vc_sb, vc_st, vc_sh;         // bytes
  int64_t num_slots;
  int32_t block_size;
  int32_t num_heads;                   // 0 when q is not rotated
  int32_t num_kv_heads;
  int32_t half_chunks;                 // 16-byte chunks in half a row
};

template <typename Tag>
struct rope_math;

// Round-to-nearest-even fp32 -> 16-bit storage and back (exact widening).
template <>
struct rope_math<bf16_tag> {
  static constexpr int VEC = 8;
  __device__ static inline float get(const u32x4 &w, int i) {
    const uint32_t x = u32x4_at(w, i >> 1);
    return (i & 1) ? elem<bf16_tag>::hi(x) : elem<bf16_tag>::lo(x);
  }
  __device__ static inline float round(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }
  __device__ static inline uint32_t pack(float a, float b) { return elem<bf16_tag>::pack2(a, b); }
  __device__ static inline float mul(float a, float b) { return opaque(round(a * b)); }
  __device__ static inline float add(float a, float b) { return round(a + b); }
};

template <>
struct rope_math<f16_tag> {
  static constexpr int VEC = 8;
  __device__ static inline float get(const u32x4 &w, int i) {
    const uint32_t x = u32x4_at(w, i >> 1);
    return (i & 1) ? elem<f16_tag>::hi(x) : elem<f16_tag>::lo(x);
  }
  __device__ static inline float round(float x) { return (float)(_Float16)x; }
  __device__ static inline uint32_t pack(float a, float b) { return elem<f16_tag>::pack2(a, b); }
  // the exact fp32 product, then one RNE conversion (a v_fma_mix with a +0
  // addend would turn a -0 product into +0)
  __device__ static inline float mul(float a, float b) { return opaque(round(opaque(a * b))); }
  __device__ static inline float add(float a, float b) { return round(a + b); }
};

template <>
struct rope_math<f32_tag> {
  static constexpr int VEC = 4;
  __device__ static inline float get(const u32x4 &w, int i) { return __uint_as_float(u32x4_at(w, i)); }
  __device__ static inline float mul(float a, float b) { return opaque(a * b); }
  __device__ static inline float add(float a, float b) { return a + b; }
};

// Rotates the chunk pair (lo = elements c*VEC.., hi = the same + D/2).
template <typename Tag>
__device__ inline void rotate_pair(const u32x4 &xl, const u32x4 &xh, const u32x4 &cl, const u32x4 &ch,
                                   const u32x4 &sl, const u32x4 &sh, u32x4 &ol, u32x4 &oh) {
  using M = rope_math<Tag>;
  float lo[M::VEC], hi[M::VEC];
#pragma unroll
  for (int i = 0; i < M::VEC; ++i) {
    const float a = M::get(xl, i), b = M::get(xh, i);
    lo[i] = M::add(M::mul(a, M::get(cl, i)), M::mul(-b, M::get(sl, i)));  // x1 cos - x2 sin
    hi[i] = M::add(M::mul(b, M::get(ch, i)), M::mul(a, M::get(sh, i)));   // x2 cos + x1 sin
  }
  if constexpr (M::VEC == 8) {
    ol = u32x4{M::pack(lo[0], lo[1]), M::pack(lo[2], lo[3]), M::pack(lo[4], lo[5]), M::pack(lo[6], lo[7])};
    oh = u32x4{M::pack(hi[0], hi[1]), M::pack(hi[2], hi[3]), M::pack(hi[4], hi[5]), M::pack(hi[6], hi[7])};
  } else {
    ol = u32x4{__float_as_uint(lo[0]), __float_as_uint(lo[1]), __float_as_uint(lo[2]), __float_as_uint(lo[3])};
    oh = u32x4{__float_as_uint(hi[0]), __float_as_uint(hi[1]), __float_as_uint(hi[2]), __float_as_uint(hi[3])};
  }
}

template <typename Tag, typename IdxT>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeParams p) {
  const int64_t t = blockIdx.x;
  const int hc = p.half_chunks;
  const char *crow = p.cos + t * p.cos_st;
  const char *srow = p.sin + t * p.sin_st;
  const int64_t slot = (int64_t)reinterpret_cast<const IdxT *>(p.slots)[t];
  const bool slot_ok = slot >= 0 && slot < p.num_slots;
  const int64_t blk = slot_ok ? slot / p.block_size : 0;
  const int64_t off = slot_ok ? slot - blk * p.block_size : 0;
  // rows: num_heads q rows, then num_kv_heads k rows (rotated); then v rows (copied)
  const int rot_items = (p.num_heads + p.num_kv_heads) * hc;
  const int copy_items = p.num_kv_heads * 2 * hc;
  for (int i = threadIdx.x; i < rot_items + copy_items; i += blockDim.x) {
    if (i < rot_items) {
      const int row = i / hc, c = i - row * hc;
      const u32x4 cl = load16(crow + c * 16), ch = load16(crow + (c + hc) * 16);
      const u32x4 sl = load16(srow + c * 16), sh = load16(srow + (c + hc) * 16);
      u32x4 ol, oh;
      if (row < p.num_heads) {
        const char *src = p.q_in + t * p.qi_st + row * p.qi_sh;
        rotate_pair<Tag>(load16(src + c * 16), load16(src + (c + hc) * 16), cl, ch, sl, sh, ol, oh);
        char *dst = p.q_out + t * p.qo_st + row * p.qo_sh;
        store16(dst + c * 16, ol);
        store16(dst + (c + hc) * 16, oh);
      } else if (slot_ok) {
        const int h = row - p.num_heads;
        const char *src = p.key + t * p.k_st + h * p.k_sh;
        rotate_pair<Tag>(load16(src + c * 16), load16(src + (c + hc) * 16), cl, ch, sl, sh, ol, oh);
        char *dst = p.kc + blk * p.kc_sb + off * p.kc_st + h * p.kc_sh;
        store16(dst + c * 16, ol);
        store16(dst + (c + hc) * 16, oh);
      }
    } else if (slot_ok) {
      const int j = i - rot_items;
      const int h = j / (2 * hc), c = j - h * 2 * hc;
      store16(p.vc + blk * p.vc_sb + off * p.vc_st + h * p.vc_sh + c * 16,
              load16(p.value + t * p.v_st + h * p.v_sh + c * 16));
    }
  }
}

// ------------------------------------------------------ into an FP8 cache
// One wave per row of a token: q rows (rotated), k rows (rotated, then
// quantised) and v rows (quantised). Lane l takes elements 4l .. 4l+3 of
// the first half and their rotate-half partners 4l + D/2 ..; the k / v row
// maximum gives the power-of-two scale e4m3_row_scale(amax) and codes
// e4m3(x / scale), as ikl_append_kv does for rows that arrive already
// rotated.
struct RopeFp8Params {
  RopeParams r;  // kc / vc strides in bytes (= elements)
  float *k_scale;
  float *v_scale;
  int64_t s_sb, s_sh;  // elements
  int32_t head_dim;
};

template <typename Tag>
struct four;
template <>
struct four<bf16_tag> {
  static constexpr int BYTES = 8;
  __device__ static inline void load(const char *p, float *x) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    x[0] = elem<bf16_tag>::lo(w.x);
    x[1] = elem<bf16_tag>::hi(w.x);
    x[2] = elem<bf16_tag>::lo(w.y);
    x[3] = elem<bf16_tag>::hi(w.y);
  }
  __device__ static inline void store(char *p, const float *x) {
    *reinterpret_cast<uint2 *>(p) = uint2{elem<bf16_tag>::pack2(x[0], x[1]), elem<bf16_tag>::pack2(x[2], x[3])};
  }
};
template <>
struct four<f16_tag> {
  static constexpr int BYTES = 8;
  __device__ static inline void load(const char *p, float *x) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    x[0] = elem<f16_tag>::lo(w.x);
    x[1] = elem<f16_tag>::hi(w.x);
    x[2] = elem<f16_tag>::lo(w.y);
    x[3] = elem<f16_tag>::hi(w.y);
  }
  __device__ static inline void store(char *p, const float *x) {
    *reinterpret_cast<uint2 *>(p) = uint2{elem<f16_tag>::pack2(x[0], x[1]), elem<f16_tag>::pack2(x[2], x[3])};
  }
};
template <>
struct four<f32_tag> {
  static constexpr int BYTES = 16;
  __device__ static inline void load(const char *p, float *x) {
    const float4 w = *reinterpret_cast<const float4 *>(p);
    x[0] = w.x;
    x[1] = w.y;
    x[2] = w.z;
    x[3] = w.w;
  }
  __device__ static inline void store(char *p, const float *x) {
    *reinterpret_cast<float4 *>(p) = float4{x[0], x[1], x[2], x[3]};
  }
};

__device__ inline float wave_max_abs(float v) {
  v = fmaxf(v, dpp_mov<DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_mov<DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_mov<DPP_ROW_MIRROR>(v));
  return max_xor32(max_xor16(v));
}

// Quantises 8 values (lo[4] at element 4l, hi[4] at 4l + D/2) of a row whose
// wave-wide maximum magnitude is amax; writes codes and (lane 0) the scale.
__device__ inline void store_fp8_row(char *dst, float *scale_dst, int lane, int half, bool on, const float *lo,
                                     const float *hi, float amax) {
  const float scale = e4m3_row_scale(amax);
  float y[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = fminf(fmaxf(lo[i] / scale, -448.0f), 448.0f);
    y[4 + i] = fminf(fmaxf(hi[i] / scale, -448.0f), 448.0f);
  }
  int wl = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
  wl = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], wl, true);
  int wh = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
  wh = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], wh, true);
  if (on) {
    *reinterpret_cast<int *>(dst + 4 * lane) = wl;
    *reinterpret_cast<int *>(dst + half + 4 * lane) = wh;
  }
  if (lane == 0) *scale_dst = scale;
}

template <typename Tag, typename IdxT>
__global__ __launch_bounds__(64) void rope_append_fp8_kernel(RopeFp8Params f) {
  using M = rope_math<Tag>;
  using F = four<Tag>;
  constexpr int EB = F::BYTES / 4;
  const RopeParams &p = f.r;
  const int lane = threadIdx.x;
  const int row = blockIdx.x;  // q rows, then k rows, then v rows
  const int64_t t = blockIdx.y;
  const int half = f.head_dim / 2;
  const bool on = 4 * lane < half;
  const int64_t slot = (int64_t)reinterpret_cast<const IdxT *>(p.slots)[t];
  const bool slot_ok = slot >= 0 && slot < p.num_slots;
  const int64_t blk = slot_ok ? slot / p.block_size : 0;
  const int64_t off = slot_ok ? slot - blk * p.block_size : 0;
  if (row >= p.num_heads && !slot_ok) return;
  const int kv_row = row - p.num_heads;
  float a[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
  if (kv_row >= p.num_kv_heads) {  // v row: quantise as is
    const int h = kv_row - p.num_kv_heads;
    const char *src = p.value + t * p.v_st + h * p.v_sh;
    if (on) {
      F::load(src + 4 * lane * EB, a);
      F::load(src + (half + 4 * lane) * EB, b);
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(a[i]), fabsf(b[i])));
    store_fp8_row(p.vc + blk * p.vc_sb + off * p.vc_st + h * p.vc_sh, f.v_scale + blk * f.s_sb + h * f.s_sh + off,
                  lane, half, on, a, b, wave_max_abs(m));
    return;
  }
  // rotate a q or k row
  const char *src = row < p.num_heads ? p.q_in + t * p.qi_st + row * p.qi_sh : p.key + t * p.k_st + kv_row * p.k_sh;
  float x1[4] = {0.f, 0.f, 0.f, 0.f}, x2[4] = {0.f, 0.f, 0.f, 0.f}, c1[4], c2[4], s1[4], s2[4];
  if (on) {
    F::load(src + 4 * lane * EB, x1);
    F::load(src + (half + 4 * lane) * EB, x2);
    F::load(p.cos + t * p.cos_st + 4 * lane * EB, c1);
    F::load(p.cos + t * p.cos_st + (half + 4 * lane) * EB, c2);
    F::load(p.sin + t * p.sin_st + 4 * lane * EB, s1);
    F::load(p.sin + t * p.sin_st + (half + 4 * lane) * EB, s2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = M::add(M::mul(x1[i], c1[i]), M::mul(-x2[i], s1[i]));  // x1 cos - x2 sin
      b[i] = M::add(M::mul(x2[i], c2[i]), M::mul(x1[i], s2[i]));   // x2 cos + x1 sin
    }
  }
  if (row < p.num_heads) {
    if (on) {
      char *dst = p.q_out + t * p.qo_st + row * p.qo_sh;
      F::store(dst + 4 * lane * EB, a);
      F::store(dst + (half + 4 * lane) * EB, b);
    }
    return;
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(a[i]), fabsf(b[i])));
  store_fp8_row(p.kc + blk * p.kc_sb + off * p.kc_st + kv_row * p.kc_sh,
                f.k_scale + blk * f.s_sb + kv_row * f.s_sh + off, lane, half, on, a, b, wave_max_abs(m));
}

template <typename Tag>
void launch_rope(const RopeParams &p, int64_t tokens, bool i64, hipStream_t s) {
  if (i64) rope_append_kernel<Tag, int64_t><<<dim3((unsigned)tokens), 256, 0, s>>>(p);
  else rope_append_kernel<Tag, int32_t><<<dim3((unsigned)tokens), 256, 0, s>>>(p);
}

bool al16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace
}  // namespace ikl

using namespace ikl;

extern "C" int ikl_rope_append_kv(const ikl_rope_append_args *a, void *stream) {
  if (!a) return fail(IKL_EINVAL, "rope append: null argument struct");
  if (a->num_tokens < 0) return fail(IKL_EINVAL, "rope append: num_tokens must be non-negative");
  if (a->num_tokens == 0) return IKL_OK;
  if (a->num_tokens > 0x7fffffffLL) return fail(IKL_EINVAL, "rope append: too many tokens for one launch");
  if (a->block_size <= 0 || a->num_blocks <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 || a->num_heads < 0)
    return fail(IKL_EINVAL, "rope append: dimensions must be positive");
  if (!a->key || !a->value || !a->cos || !a->sin || !a->slots || !a->k_cache || !a->v_cache)
    return fail(IKL_EINVAL, "rope append: null tensor pointer");
  if (a->num_heads > 0 && (!a->query || !a->query_out))
    return fail(IKL_EINVAL, "rope append: query rotation needs query and query_out");
  if (a->slot_type != IKL_I32 && a->slot_type != IKL_I64)
    return fail(IKL_EINVAL, "rope append: slots must use int32 or int64");
  int eb;
  switch (a->dtype) {
    case IKL_F16:
    case IKL_BF16: eb = 2; break;
    case IKL_F32: eb = 4; break;
    default: return fail(IKL_EINVAL, "rope append: unsupported dtype");
  }
  const bool fp8 = a->cache_dtype == IKL_FP8_E4M3;
  if (a->cache_dtype != 0 && a->cache_dtype != a->dtype && !fp8)
    return fail(IKL_EINVAL, "rope append: cache_dtype must be 0, the tensor dtype or IKL_FP8_E4M3");
  const int64_t row = (int64_t)a->head_dim * eb;
  if (row % 32 != 0)
    return fail(IKL_EUNSUPPORTED, "rope append: head_dim * element size must be a multiple of 32 bytes");
  if (fp8 && (a->head_dim % 8 != 0 || a->head_dim > 512))
    return fail(IKL_EUNSUPPORTED, "rope append: the FP8 cache needs head_dim a multiple of 8, at most 512");
  if (fp8 && (!a->k_scale || !a->v_scale)) return fail(IKL_EINVAL, "rope append: the FP8 cache needs k_scale and v_scale");
  const int ceb = fp8 ? 1 : eb;  // cache bytes per element
  RopeParams p;
  p.q_in = (const char *)a->query;
  p.q_out = (char *)a->query_out;
  p.qi_st = a->q_stride_t * eb;
  p.qi_sh = a->q_stride_h * eb;
  p.qo_st = a->q_out_stride_t * eb;
  p.qo_sh = a->q_out_stride_h * eb;
  p.key = (const char *)a->key;
  p.value = (const char *)a->value;
  p.k_st = a->key_stride_t * eb;
  p.k_sh = a->key_stride_h * eb;
  p.v_st = a->value_stride_t * eb;
  p.v_sh = a->value_stride_h * eb;
  p.cos = (const char *)a->cos;
  p.sin = (const char *)a->sin;
  p.cos_st = a->cos_stride_t * eb;
  p.sin_st = a->sin_stride_t * eb;
  p.slots = a->slots;
  p.kc = (char *)a->k_cache;
  p.vc = (char *)a->v_cache;
  p.kc_sb = a->k_stride_block * ceb;
  p.kc_st = a->k_stride_token * ceb;
  p.kc_sh = a->k_stride_head * ceb;
  p.vc_sb = a->v_stride_block * ceb;
  p.vc_st = a->v_stride_token * ceb;
  p.vc_sh = a->v_stride_head * ceb;
  p.num_slots = a->num_blocks * (int64_t)a->block_size;
  p.block_size = a->block_size;
  p.num_heads = a->num_heads;
  p.num_kv_heads = a->num_kv_heads;
  p.half_chunks = (int32_t)(row / 32);
  const bool ok = al16(a->key) && al16(a->value) && al16(a->cos) && al16(a->sin) && al16(a->k_cache) &&
                  al16(a->v_cache) && (a->num_heads == 0 || (al16(a->query) && al16(a->query_out))) &&
                  p.qi_st % 16 == 0 && p.qi_sh % 16 == 0 && p.qo_st % 16 == 0 && p.qo_sh % 16 == 0 &&
                  p.k_st % 16 == 0 && p.k_sh % 16 == 0 && p.v_st % 16 == 0 && p.v_sh % 16 == 0 &&
                  p.cos_st % 16 == 0 && p.sin_st % 16 == 0 && p.kc_sb % 16 == 0 && p.kc_st % 16 == 0 &&
                  p.kc_sh % 16 == 0 && p.vc_sb % 16 == 0 && p.vc_st % 16 == 0 && p.vc_sh % 16 == 0;
  if (!ok) return fail(IKL_EINVAL, "rope append: rows must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const bool i64 = a->slot_type == IKL_I64;
  if (fp8) {
    if (((uintptr_t)a->k_scale & 3u) || ((uintptr_t)a->v_scale & 3u))
      return fail(IKL_EINVAL, "rope append: misaligned scale tensor");
    if ((int64_t)a->num_heads + 2 * (int64_t)a->num_kv_heads > 0x7fffffffLL)
      return fail(IKL_EINVAL, "rope append: too many heads");
    RopeFp8Params f;
    f.r = p;
    f.k_scale = (float *)a->k_scale;
    f.v_scale = (float *)a->v_scale;
    f.s_sb = a->scale_stride_block;
    f.s_sh = a->scale_stride_head;
    f.head_dim = a->head_dim;
    const dim3 grid((unsigned)(a->num_heads + 2 * a->num_kv_heads), (unsigned)a->num_tokens);
#define IKL_ROPE8(TAG)                                                                  \
  do {                                                                                  \
    if (i64) rope_append_fp8_kernel<TAG, int64_t><<<grid, 64, 0, s>>>(f);               \
    else rope_append_fp8_kernel<TAG, int32_t><<<grid, 64, 0, s>>>(f);                   \
  } while (0)
    switch (a->dtype) {
      case IKL_F16: IKL_ROPE8(f16_tag); break;
      case IKL_BF16: IKL_ROPE8(bf16_tag); break;
      default: IKL_ROPE8(f32_tag); break;
    }
#undef IKL_ROPE8
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(IKL_ELAUNCH, std::string("rope append launch: ") + hipGetErrorString(e));
    return IKL_OK;
  }
  switch (a->dtype) {
    case IKL_F16: launch_rope<f16_tag>(p, a->num_tokens, i64, s); break;
    case IKL_BF16: launch_rope<bf16_tag>(p, a->num_tokens, i64, s); break;
    default: launch_rope<f32_tag>(p, a->num_tokens, i64, s); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IKL_ELAUNCH, std::string("rope append launch: ") + hipGetErrorString(e));
  return IKL_OK;
}
