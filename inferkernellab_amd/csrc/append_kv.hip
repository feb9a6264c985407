// KV append: scatter [T, Hkv, D] key/value rows into the paged cache
// [num_blocks, block_size, Hkv, D] at physical slots (copy), or quantise
// them into an FP8 (E4M3) cache with per-row scales.
//
// Same result as cache.py:156-189 (write_slots: k[layer, slot//bs, slot%bs]
// = key) and append.py:19-66 (_append_kv_kernel), re-laid out for gfx950:
// one workgroup per token moves the token's whole Hkv*D row (2 KiB for
// 8x128 bf16) with 16-byte vector loads/stores, so a wave touches 1 KiB of
// contiguous cache memory per instruction instead of one head_dim row per
// program. Slots outside the cache are skipped (the reference's Triton
// kernel has no bound check, append.py:44-66).
#include "fp8_row.h"
#include "ikl_common.h"
#include "paged_attn.h"

namespace ikl {
namespace {

struct AppendParams {
  const char *key;
  const char *value;
  int64_t key_st, key_sh;      // bytes
  int64_t value_st, value_sh;  // bytes
  const void *slots;
  char *kc;
  char *vc;
  int64_t kc_sb, kc_st, kc_sh;  // bytes
  int64_t vc_sb, vc_st, vc_sh;  // bytes
  int64_t num_slots;            // num_blocks * block_size
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t chunks_per_head;      // head_dim * elem_bytes / CHUNK
};

template <int CHUNK>
struct chunk_t;
template <>
struct chunk_t<16> {
  using type = v4u32;  // a vector type: loads and stores stay in registers
};
template <>
struct chunk_t<4> {
  using type = uint32_t;
};
template <>
struct chunk_t<2> {
  using type = uint16_t;
};

template <typename IdxT, int CHUNK>
__global__ __launch_bounds__(256) void append_kv_kernel(AppendParams p) {
  using C = typename chunk_t<CHUNK>::type;
  const int64_t t = blockIdx.x;
  const int total = p.num_kv_heads * p.chunks_per_head;
  const char *ksrc = p.key + t * p.key_st;
  const char *vsrc = p.value + t * p.value_st;
  // The first chunk's K/V loads do not depend on the slot: they go out with
  // the slot load, so the copy costs one memory round trip before its stores.
  const bool has0 = (int)threadIdx.x < total;
  const int i0 = has0 ? (int)threadIdx.x : total - 1;  // in bounds either way; unused when !has0
  const int h0 = i0 / p.chunks_per_head, c0 = i0 - h0 * p.chunks_per_head;
  const int64_t slot = (int64_t)reinterpret_cast<const IdxT *>(p.slots)[t];
  const C kv0 = *reinterpret_cast<const C *>(ksrc + h0 * p.key_sh + c0 * CHUNK);
  const C vv0 = *reinterpret_cast<const C *>(vsrc + h0 * p.value_sh + c0 * CHUNK);
  asm volatile("" ::"v"(kv0), "v"(vv0));  // all three loads issued before the slot test
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size;
  const int64_t off = slot - blk * p.block_size;
  char *kdst = p.kc + blk * p.kc_sb + off * p.kc_st;
  char *vdst = p.vc + blk * p.vc_sb + off * p.vc_st;
  if (has0) {
    *reinterpret_cast<C *>(kdst + h0 * p.kc_sh + c0 * CHUNK) = kv0;
    *reinterpret_cast<C *>(vdst + h0 * p.vc_sh + c0 * CHUNK) = vv0;
  }
  for (int i = (int)threadIdx.x + (int)blockDim.x; i < total; i += blockDim.x) {
    const int h = i / p.chunks_per_head;
    const int c = i - h * p.chunks_per_head;
    const C kv = *reinterpret_cast<const C *>(ksrc + h * p.key_sh + c * CHUNK);
    const C vv = *reinterpret_cast<const C *>(vsrc + h * p.value_sh + c * CHUNK);
    *reinterpret_cast<C *>(kdst + h * p.kc_sh + c * CHUNK) = kv;
    *reinterpret_cast<C *>(vdst + h * p.vc_sh + c * CHUNK) = vv;
  }
}

// ------------------------------------------------------------ FP8 append
// One wave per (token, head, K or V) row: lane l converts elements
// 4l .. 4l+3 (head_dim <= 256). The row maximum gives the power-of-two
// scale e4m3_row_scale(amax); the codes are e4m3(x / scale) clamped to
// +-448, rounded to nearest even by v_cvt_pk_fp8_f32 (OCP E4M3 on gfx950).
struct Fp8AppendParams {
  const char *src[2];         // key, value rows
  int64_t src_st[2], src_sh[2];  // bytes
  const void *slots;
  char *dst[2];               // fp8 caches
  int64_t dst_sb[2], dst_st[2], dst_sh[2];  // bytes (= elements)
  float *scale[2];
  int64_t scale_sb, scale_sh;  // elements
  int64_t num_slots;
  int32_t block_size;
  int32_t head_dim;
};

template <typename Tag, typename IdxT>
__global__ __launch_bounds__(64) void append_kv_fp8_kernel(Fp8AppendParams p) {
  constexpr int EB = elem<Tag>::bytes;
  const int lane = threadIdx.x;
  const int which = blockIdx.x & 1;  // 0: key, 1: value
  const int h = (int)(blockIdx.x >> 1);
  const int64_t t = blockIdx.y;
  const bool on = 4 * lane < p.head_dim;
  // The row load does not depend on the slot: both go out together (lanes
  // past the row read its first chunk, which exists, and drop it).
  float x[4];
  load4<Tag>(p.src[which] + t * p.src_st[which] + h * p.src_sh[which] + (on ? 4 * lane * EB : 0), x);
  const int64_t slot = (int64_t)reinterpret_cast<const IdxT *>(p.slots)[t];
  asm volatile("" ::"v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size;
  const int64_t off = slot - blk * p.block_size;
  store_fp8_row(p.dst[which] + blk * p.dst_sb[which] + off * p.dst_st[which] + h * p.dst_sh[which],
                p.scale[which] + blk * p.scale_sb + h * p.scale_sh + off, lane, on, x);
}

bool aligned(const void *ptr, int64_t n) { return ((uintptr_t)ptr % (uintptr_t)n) == 0; }

// Validates an FP8 append and fills its launch parameters (IKL_OK or an
// IKL_E* code with the message set).
int fp8_params(const ikl_append_args *a, Fp8AppendParams &p) {
  int eb;
  switch (a->dtype) {
    case IKL_F16:
    case IKL_BF16: eb = 2; break;
    case IKL_F32: eb = 4; break;
    default: return fail(IKL_EINVAL, "append: unsupported dtype");
  }
  if (a->head_dim % 4 != 0 || a->head_dim > 256)
    return fail(IKL_EUNSUPPORTED, "append: the FP8 cache needs head_dim a multiple of 4, at most 256");
  if (!a->k_scale || !a->v_scale) return fail(IKL_EINVAL, "append: the FP8 cache needs k_scale and v_scale");
  p.src[0] = (const char *)a->key;
  p.src[1] = (const char *)a->value;
  p.src_st[0] = a->key_stride_t * eb;
  p.src_sh[0] = a->key_stride_h * eb;
  p.src_st[1] = a->value_stride_t * eb;
  p.src_sh[1] = a->value_stride_h * eb;
  p.slots = a->slots;
  p.dst[0] = (char *)a->k_cache;
  p.dst[1] = (char *)a->v_cache;
  p.dst_sb[0] = a->k_stride_block;
  p.dst_st[0] = a->k_stride_token;
  p.dst_sh[0] = a->k_stride_head;
  p.dst_sb[1] = a->v_stride_block;
  p.dst_st[1] = a->v_stride_token;
  p.dst_sh[1] = a->v_stride_head;
  p.scale[0] = (float *)a->k_scale;
  p.scale[1] = (float *)a->v_scale;
  p.scale_sb = a->scale_stride_block;
  p.scale_sh = a->scale_stride_head;
  p.num_slots = a->num_blocks * (int64_t)a->block_size;
  p.block_size = a->block_size;
  p.head_dim = a->head_dim;
  // every row the kernel touches is read 4 elements and written 4 codes at a time
  const int64_t in_steps[] = {p.src_st[0], p.src_sh[0], p.src_st[1], p.src_sh[1]};
  for (int64_t st : in_steps)
    if (st % (4 * eb) != 0) return fail(IKL_EINVAL, "append: key/value rows must be aligned to 4 elements");
  const int64_t out_steps[] = {p.dst_sb[0], p.dst_st[0], p.dst_sh[0], p.dst_sb[1], p.dst_st[1], p.dst_sh[1]};
  for (int64_t st : out_steps)
    if (st % 4 != 0) return fail(IKL_EINVAL, "append: FP8 cache rows must be 4-byte aligned");
  if (!aligned(a->key, 4 * eb) || !aligned(a->value, 4 * eb) || !aligned(a->k_cache, 4) ||
      !aligned(a->v_cache, 4) || !aligned(a->k_scale, 4) || !aligned(a->v_scale, 4))
    return fail(IKL_EINVAL, "append: misaligned tensor pointer");
  if ((int64_t)a->num_kv_heads * 2 > 0x7fffffffLL) return fail(IKL_EINVAL, "append: too many heads");
  return IKL_OK;
}

int append_fp8(const ikl_append_args *a, hipStream_t s) {
  Fp8AppendParams p;
  const int rc = fp8_params(a, p);
  if (rc != IKL_OK) return rc;
  const dim3 grid((unsigned)(2 * a->num_kv_heads), (unsigned)a->num_tokens);
#define IKL_FP8_LAUNCH(TAG, IDX) append_kv_fp8_kernel<TAG, IDX><<<grid, 64, 0, s>>>(p)
  const bool i32 = a->slot_type == IKL_I32;
  if (a->dtype == IKL_BF16) {
    if (i32) IKL_FP8_LAUNCH(bf16_tag, int32_t);
    else IKL_FP8_LAUNCH(bf16_tag, int64_t);
  } else if (a->dtype == IKL_F16) {
    if (i32) IKL_FP8_LAUNCH(f16_tag, int32_t);
    else IKL_FP8_LAUNCH(f16_tag, int64_t);
  } else {
    if (i32) IKL_FP8_LAUNCH(f32_tag, int32_t);
    else IKL_FP8_LAUNCH(f32_tag, int64_t);
  }
#undef IKL_FP8_LAUNCH
  return check_launch("append_kv_fp8_kernel");
}

}  // namespace
}  // namespace ikl

using namespace ikl;

namespace ikl {
namespace {

// Checks shared by ikl_append_kv and the fused append of a decode step.
int check_append(const ikl_append_args *a) {
  if (!a) return fail(IKL_EINVAL, "append: null argument struct");
  if (a->num_tokens < 0) return fail(IKL_EINVAL, "append: num_tokens must be non-negative");
  if (a->num_tokens > 0x7fffffffLL) return fail(IKL_EINVAL, "append: too many tokens for one launch");
  if (a->num_tokens == 0) return IKL_OK;
  if (a->block_size <= 0 || a->num_blocks <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0)
    return fail(IKL_EINVAL, "append: cache dimensions must be positive");
  if (!a->key || !a->value || !a->slots || !a->k_cache || !a->v_cache)
    return fail(IKL_EINVAL, "append: null tensor pointer");
  if (a->slot_type != IKL_I32 && a->slot_type != IKL_I64)
    return fail(IKL_EINVAL, "append: slots must use int32 or int64");
  if (a->cache_dtype != 0 && a->cache_dtype != a->dtype && a->cache_dtype != IKL_FP8_E4M3)
    return fail(IKL_EINVAL, "append: cache_dtype must be 0, the key dtype or IKL_FP8_E4M3");
  return IKL_OK;
}

// Byte-stride parameters of a plain-copy append and the widest chunk (16, 4
// or the element size) that every row start and the row length allow.
int copy_params(const ikl_append_args *a, AppendParams &p, int &chunk) {
  int eb;
  switch (a->dtype) {
    case IKL_F16:
    case IKL_BF16: eb = 2; break;
    case IKL_F32: eb = 4; break;
    default: return fail(IKL_EINVAL, "append: unsupported dtype");
  }
  p.key = (const char *)a->key;
  p.value = (const char *)a->value;
  p.key_st = a->key_stride_t * eb;
  p.key_sh = a->key_stride_h * eb;
  p.value_st = a->value_stride_t * eb;
  p.value_sh = a->value_stride_h * eb;
  p.slots = a->slots;
  p.kc = (char *)a->k_cache;
  p.vc = (char *)a->v_cache;
  p.kc_sb = a->k_stride_block * eb;
  p.kc_st = a->k_stride_token * eb;
  p.kc_sh = a->k_stride_head * eb;
  p.vc_sb = a->v_stride_block * eb;
  p.vc_st = a->v_stride_token * eb;
  p.vc_sh = a->v_stride_head * eb;
  p.num_slots = a->num_blocks * (int64_t)a->block_size;
  p.block_size = a->block_size;
  p.num_kv_heads = a->num_kv_heads;
  const int64_t row_bytes = (int64_t)a->head_dim * eb;
  auto fits = [&](int64_t n) {
    return row_bytes % n == 0 && p.key_st % n == 0 && p.key_sh % n == 0 && p.value_st % n == 0 &&
           p.value_sh % n == 0 && p.kc_sb % n == 0 && p.kc_st % n == 0 && p.kc_sh % n == 0 &&
           p.vc_sb % n == 0 && p.vc_st % n == 0 && p.vc_sh % n == 0 && aligned(a->key, n) &&
           aligned(a->value, n) && aligned(a->k_cache, n) && aligned(a->v_cache, n);
  };
  chunk = fits(16) ? 16 : fits(4) ? 4 : eb;
  if (!fits(chunk)) return fail(IKL_EINVAL, "append: tensors are not element aligned");
  p.chunks_per_head = (int32_t)(row_bytes / chunk);
  return IKL_OK;
}

}  // namespace

int prepare_fused_append(const ikl_append_args *a, FusedAppend &f) {
  f = FusedAppend{};
  const int rc = check_append(a);
  if (rc != IKL_OK || a->num_tokens == 0) return rc;
  if (a->cache_dtype == IKL_FP8_E4M3) {
    // quantised rows, one reduce workgroup (one wave) per (token, head, K or V)
    Fp8AppendParams q;
    const int qrc = fp8_params(a, q);
    if (qrc != IKL_OK) return qrc;
    f.fp8 = 1;
    f.src_dtype = a->dtype;
    f.head_dim = a->head_dim;
    f.key = q.src[0];
    f.value = q.src[1];
    f.key_st = q.src_st[0];
    f.key_sh = q.src_sh[0];
    f.value_st = q.src_st[1];
    f.value_sh = q.src_sh[1];
    f.slots = q.slots;
    f.kc = q.dst[0];
    f.vc = q.dst[1];
    f.kc_sb = q.dst_sb[0];
    f.kc_st = q.dst_st[0];
    f.kc_sh = q.dst_sh[0];
    f.vc_sb = q.dst_sb[1];
    f.vc_st = q.dst_st[1];
    f.vc_sh = q.dst_sh[1];
    f.k_scale = q.scale[0];
    f.v_scale = q.scale[1];
    f.s_sb = q.scale_sb;
    f.s_sh = q.scale_sh;
    f.rows = a->num_tokens * (int64_t)a->num_kv_heads;
    f.num_slots = q.num_slots;
    f.kv_heads = a->num_kv_heads;
    f.block_size = a->block_size;
    f.slots_i64 = a->slot_type == IKL_I64;
    return IKL_OK;
  }
  AppendParams p;
  int chunk = 0;
  const int prc = copy_params(a, p, chunk);
  if (prc != IKL_OK) return prc;
  if (chunk != 16 || p.chunks_per_head > 32) return 1;
  f.key = p.key;
  f.value = p.value;
  f.key_st = p.key_st;
  f.key_sh = p.key_sh;
  f.value_st = p.value_st;
  f.value_sh = p.value_sh;
  f.slots = p.slots;
  f.kc = p.kc;
  f.vc = p.vc;
  f.kc_sb = p.kc_sb;
  f.kc_st = p.kc_st;
  f.kc_sh = p.kc_sh;
  f.vc_sb = p.vc_sb;
  f.vc_st = p.vc_st;
  f.vc_sh = p.vc_sh;
  f.rows = a->num_tokens * (int64_t)a->num_kv_heads;
  f.num_slots = p.num_slots;
  f.kv_heads = a->num_kv_heads;
  f.chunks = p.chunks_per_head;
  f.block_size = a->block_size;
  f.slots_i64 = a->slot_type == IKL_I64;
  return IKL_OK;
}

}  // namespace ikl

using namespace ikl;

extern "C" int ikl_append_kv(const ikl_append_args *a, void *stream) {
  const int rc = check_append(a);
  if (rc != IKL_OK || a->num_tokens == 0) return rc;
  if (a->cache_dtype == IKL_FP8_E4M3) return append_fp8(a, (hipStream_t)stream);
  AppendParams p;
  int chunk = 0;
  const int prc = copy_params(a, p, chunk);
  if (prc != IKL_OK) return prc;
  const int total = a->num_kv_heads * p.chunks_per_head;
  int threads = total >= 256 ? 256 : ((total + 63) / 64) * 64;
  dim3 grid((unsigned)a->num_tokens);
  hipStream_t s = (hipStream_t)stream;
#define IKL_APPEND_LAUNCH(IDX, CH) append_kv_kernel<IDX, CH><<<grid, threads, 0, s>>>(p)
  if (a->slot_type == IKL_I32) {
    if (chunk == 16) IKL_APPEND_LAUNCH(int32_t, 16);
    else if (chunk == 4) IKL_APPEND_LAUNCH(int32_t, 4);
    else IKL_APPEND_LAUNCH(int32_t, 2);
  } else {
    if (chunk == 16) IKL_APPEND_LAUNCH(int64_t, 16);
    else if (chunk == 4) IKL_APPEND_LAUNCH(int64_t, 4);
    else IKL_APPEND_LAUNCH(int64_t, 2);
  }
#undef IKL_APPEND_LAUNCH
  return check_launch("append_kv_kernel");
}
