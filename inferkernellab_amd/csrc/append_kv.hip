// KV append: scatter [T, Hkv, D] key/value rows into the paged cache
// [num_blocks, block_size, Hkv, D] at physical slots.
//
// Same result as cache.py:156-189 (write_slots: k[layer, slot//bs, slot%bs]
// = key) and append.py:19-66 (_append_kv_kernel), re-laid out for gfx950:
// one workgroup per token moves the token's whole Hkv*D row (2 KiB for
// 8x128 bf16) with 16-byte vector loads/stores, so a wave touches 1 KiB of
// contiguous cache memory per instruction instead of one head_dim row per
// program. Slots outside the cache are skipped (the reference's Triton
// kernel has no bound check, append.py:44-66).
#include "ikl_common.h"

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
  using type = u32x4;
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
  const int64_t slot = (int64_t)reinterpret_cast<const IdxT *>(p.slots)[t];
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size;
  const int64_t off = slot - blk * p.block_size;
  const int total = p.num_kv_heads * p.chunks_per_head;
  const char *ksrc = p.key + t * p.key_st;
  const char *vsrc = p.value + t * p.value_st;
  char *kdst = p.kc + blk * p.kc_sb + off * p.kc_st;
  char *vdst = p.vc + blk * p.vc_sb + off * p.vc_st;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int h = i / p.chunks_per_head;
    const int c = i - h * p.chunks_per_head;
    const C kv = *reinterpret_cast<const C *>(ksrc + h * p.key_sh + c * CHUNK);
    const C vv = *reinterpret_cast<const C *>(vsrc + h * p.value_sh + c * CHUNK);
    *reinterpret_cast<C *>(kdst + h * p.kc_sh + c * CHUNK) = kv;
    *reinterpret_cast<C *>(vdst + h * p.vc_sh + c * CHUNK) = vv;
  }
}

bool aligned(const void *ptr, int64_t n) { return ((uintptr_t)ptr % (uintptr_t)n) == 0; }

}  // namespace
}  // namespace ikl

using namespace ikl;

extern "C" int ikl_append_kv(const ikl_append_args *a, void *stream) {
  if (!a) return fail(IKL_EINVAL, "append: null argument struct");
  if (a->num_tokens < 0) return fail(IKL_EINVAL, "append: num_tokens must be non-negative");
  if (a->num_tokens == 0) return IKL_OK;
  if (a->num_tokens > 0x7fffffffLL) return fail(IKL_EINVAL, "append: too many tokens for one launch");
  if (a->block_size <= 0 || a->num_blocks <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0)
    return fail(IKL_EINVAL, "append: cache dimensions must be positive");
  if (!a->key || !a->value || !a->slots || !a->k_cache || !a->v_cache)
    return fail(IKL_EINVAL, "append: null tensor pointer");
  if (a->slot_type != IKL_I32 && a->slot_type != IKL_I64)
    return fail(IKL_EINVAL, "append: slots must use int32 or int64");
  int eb;
  switch (a->dtype) {
    case IKL_F16:
    case IKL_BF16: eb = 2; break;
    case IKL_F32: eb = 4; break;
    default: return fail(IKL_EINVAL, "append: unsupported dtype");
  }
  AppendParams p;
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
  // Widest chunk that every row start and the row length allow.
  auto fits = [&](int64_t n) {
    return row_bytes % n == 0 && p.key_st % n == 0 && p.key_sh % n == 0 && p.value_st % n == 0 &&
           p.value_sh % n == 0 && p.kc_sb % n == 0 && p.kc_st % n == 0 && p.kc_sh % n == 0 &&
           p.vc_sb % n == 0 && p.vc_st % n == 0 && p.vc_sh % n == 0 && aligned(a->key, n) &&
           aligned(a->value, n) && aligned(a->k_cache, n) && aligned(a->v_cache, n);
  };
  int chunk = fits(16) ? 16 : fits(4) ? 4 : eb;
  if (!fits(chunk)) return fail(IKL_EINVAL, "append: tensors are not element aligned");
  p.chunks_per_head = (int32_t)(row_bytes / chunk);
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
