/*
 * ikl_paged.h — C ABI of the MI355X (gfx950) paged-KV decode library
 * (libikl_paged.so).
 *
 * The library holds two hot operations of paged-KV decoding:
 *   - KV append: scatter new K/V rows into physical cache slots;
 *   - paged decode attention for MHA / GQA / MQA over a block-table
 *     addressed cache, with optional split-context partitions and a
 *     log-sum-exp reduce kernel.
 *
 * Conventions
 *   - Every pointer is a device pointer (HBM) except the argument structs
 *     themselves, which live in host memory and are read during the call.
 *   - Strides are in ELEMENTS of the tensor they describe, not bytes.
 *   - The cache layout is the reference's [layers, blocks, block_size,
 *     kv_heads, head_dim]; callers pass the base pointer of ONE layer
 *     (cache.k[layer], cache.v[layer]) plus its block/token/head strides.
 *   - The last dimension (head_dim) of every tensor is contiguous.
 *   - All work is enqueued on `stream` (a hipStream_t, NULL = default
 *     stream). No call synchronises the host, allocates device memory or
 *     keeps device state between calls.
 *   - Return value: 0 on success, a negative IKL_E* code otherwise; the
 *     message of the last failure on the calling thread is returned by
 *     ikl_last_error().
 */
#ifndef IKL_PAGED_H
#define IKL_PAGED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of query / cache / key / value / output tensors.
 * IKL_FP8_E4M3 is a cache format only (cache_dtype): OCP E4M3 codes with
 * one power-of-two fp32 scale per (token, kv head) row, value =
 * decode(code) * scale (exact in fp32, bf16 and fp16). */
enum ikl_dtype {
  IKL_F16 = 0,
  IKL_BF16 = 1,
  IKL_F32 = 2,
  IKL_FP8_E4M3 = 3,
};

/* Element types of index tensors (slots, block tables, context lengths). */
enum ikl_index_type {
  IKL_I32 = 0,
  IKL_I64 = 1,
};

/* Status codes. */
enum ikl_status {
  IKL_OK = 0,
  IKL_EINVAL = -1,      /* bad argument (shape, stride, alignment, dtype) */
  IKL_EUNSUPPORTED = -2,/* valid but not compiled in (e.g. head_dim 200) */
  IKL_ELAUNCH = -3,     /* HIP launch / runtime error */
  IKL_EWORKSPACE = -4,  /* workspace missing or too small */
};

/* Kernel family chosen for a grouped-attention launch
 * (ikl_paged_attention_path). */
enum ikl_attention_path {
  IKL_PATH_MHA_FALLBACK = 0,  /* heads_per_kv == 1: one query head per K/V tile */
  IKL_PATH_SCALAR_GROUPED = 1,/* VALU path: query group shares each K/V tile */
  IKL_PATH_MFMA_GROUPED = 2,  /* MFMA QK^T/PV tiles (dense group x tile) */
};

/* Arguments of ikl_append_kv.
 * Replaces the launch in append.py:69-106 (append_kv_triton ->
 * _append_kv_kernel, append.py:19-66) and the torch index_put of
 * cache.py:156-189 (PagedKVCache.write_slots). */
typedef struct ikl_append_args {
  const void *key;           /* [num_tokens, num_kv_heads, head_dim] */
  const void *value;         /* same shape as key */
  int64_t key_stride_t, key_stride_h;
  int64_t value_stride_t, value_stride_h;
  const void *slots;         /* [num_tokens] physical slot = block*block_size + offset */
  int32_t slot_type;         /* enum ikl_index_type */
  void *k_cache;             /* base of cache.k[layer]: [num_blocks, block_size, kv_heads, head_dim] */
  void *v_cache;             /* base of cache.v[layer] */
  int64_t k_stride_block, k_stride_token, k_stride_head;
  int64_t v_stride_block, v_stride_token, v_stride_head;
  int64_t num_tokens;
  int64_t num_blocks;
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t dtype;             /* enum ikl_dtype of key and value (and of the cache unless cache_dtype) */
  /* FP8 KV (no counterpart in the reference): cache_dtype IKL_FP8_E4M3
   * quantises each appended (token, head) row — scale = 2^ceil(log2(amax /
   * 448)) from the bits of the rounded amax / 448 (at least 2^-126, 1 for a
   * zero row), codes = e4m3(x / scale), round to nearest even, saturating at
   * 448 — and writes the scale to k_scale / v_scale [num_blocks,
   * num_kv_heads, block_size] fp32 (strides in elements; the token stride is
   * 1). 0 = same as dtype. */
  int32_t cache_dtype;
  void *k_scale;
  void *v_scale;
  int64_t scale_stride_block, scale_stride_head;
} ikl_append_args;

/* Arguments of ikl_paged_attention.
 * Replaces paged_decode_attention_triton (triton_ops.py:404-478, kernel
 * triton_ops.py:88-167) and paged_decode_attention_triton_grouped
 * (triton_ops.py:481-610, kernels triton_ops.py:178-283 and 294-401). */
typedef struct ikl_paged_attention_args {
  const void *query;         /* [batch, num_heads, head_dim] */
  int64_t q_stride_b, q_stride_h;
  const void *k_cache;       /* base of cache.k[layer] */
  const void *v_cache;       /* base of cache.v[layer] */
  int64_t k_stride_block, k_stride_token, k_stride_head;
  int64_t v_stride_block, v_stride_token, v_stride_head;
  const void *block_tables;  /* [batch, table_width] physical block ids */
  int32_t table_type;        /* enum ikl_index_type */
  int64_t table_stride_b;
  int64_t table_width;
  const void *context_lens;  /* [batch] */
  int32_t lens_type;         /* enum ikl_index_type */
  void *out;                 /* [batch, num_heads, head_dim], dtype of query */
  int64_t out_stride_b, out_stride_h;
  int64_t batch;
  int64_t num_blocks;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t dtype;             /* enum ikl_dtype (query, cache and out share it) */
  float scale;               /* softmax scale; the reference default is head_dim**-0.5 */
  /* Query heads that share one K/V tile inside a workgroup: 0 = all heads
   * of a KV head (capped by the kernel family), else 1..heads_per_kv. */
  int32_t query_group_size;
  /* Tokens per split-context partition: 0 = pick automatically (fixed
   * partitions or the balanced split; on the VALU family a request needing
   * at most 4 partitions runs them unsplit as one multi-wave workgroup),
   * -1 = never split (one pass per request), -2 = the balanced split (MFMA
   * family: equal runs of the batch's tiles per resident workgroup; with
   * path -1 an MHA launch moves to the MFMA family for it where that
   * supports the shape), else a positive multiple of 64. */
  int32_t partition_size;
  /* Host-known upper bound of context_lens (0 = table_width*block_size);
   * only sizes the grid, never read from device memory. Contract: every
   * context_lens[b] <= max_context_len. The fixed partitions cover
   * [0, max_context_len) only, so positions of a longer context past it are
   * not attended (no fault, no error: the device lengths are not read on
   * the host). The balanced split and the unsplit launch read the device
   * lengths and are unaffected. */
  int64_t max_context_len;
  /* Kernel family: -1 = automatic (ikl_paged_attention_path), else an
   * enum ikl_attention_path value. */
  int32_t path;
  /* Scratch for split partials; size from ikl_paged_attention_workspace_size. */
  void *workspace;
  int64_t workspace_bytes;
  /* Optional hipEvent_t handles recorded on `stream` for timing single
   * kernels of the launch: [0] before the attention kernel, [1] after it,
   * [2] after the split reduce kernel. NULL entries are skipped. */
  void *events[3];
  /* FP8 KV cache (cache_dtype IKL_FP8_E4M3; 0 = same as dtype): the cache
   * holds E4M3 codes with per-(token, head) fp32 scales k_scale / v_scale
   * [num_blocks, num_kv_heads, block_size] (the layout ikl_append_kv writes).
   * MFMA family only (dtype fp16 / bf16, head_dim in {32, 64, 96, 128}). */
  int32_t cache_dtype;
  const void *k_scale;
  const void *v_scale;
  int64_t scale_stride_block, scale_stride_head;
} ikl_paged_attention_args;

/* Arguments of ikl_rope_append_kv: rotary embedding of q and k fused with
 * the KV append. Replaces the step of hf_benchmark.py:419-436 (rotate-half
 * RoPE of hf_benchmark.py:69-85, then _write_kv -> append_kv_triton /
 * cache.write): one launch instead of the elementwise RoPE ops plus the
 * append. */
typedef struct ikl_rope_append_args {
  const void *query;         /* [num_tokens, num_heads, head_dim]; NULL when num_heads == 0 */
  int64_t q_stride_t, q_stride_h;
  void *query_out;           /* rotated query (may be `query`) */
  int64_t q_out_stride_t, q_out_stride_h;
  const void *key;           /* [num_tokens, num_kv_heads, head_dim], before rotation */
  int64_t key_stride_t, key_stride_h;
  const void *value;         /* [num_tokens, num_kv_heads, head_dim] */
  int64_t value_stride_t, value_stride_h;
  const void *cos;           /* [num_tokens, head_dim] of each token's position, tensor dtype */
  int64_t cos_stride_t;
  const void *sin;           /* [num_tokens, head_dim] */
  int64_t sin_stride_t;
  const void *slots;         /* [num_tokens] physical slot per token */
  int32_t slot_type;         /* enum ikl_index_type */
  void *k_cache;             /* base of cache.k[layer] */
  void *v_cache;             /* base of cache.v[layer] */
  int64_t k_stride_block, k_stride_token, k_stride_head;
  int64_t v_stride_block, v_stride_token, v_stride_head;
  int64_t num_tokens;
  int64_t num_blocks;
  int32_t block_size;
  int32_t num_heads;         /* 0: rotate and append keys only */
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t dtype;             /* enum ikl_dtype of every tensor (of the cache unless cache_dtype) */
  /* FP8 KV cache (cache_dtype IKL_FP8_E4M3; 0 = same as dtype): rope(k) and
   * v are quantised per (token, head) row as ikl_append_kv does, scales to
   * k_scale / v_scale [num_blocks, num_kv_heads, block_size]. */
  int32_t cache_dtype;
  void *k_scale;
  void *v_scale;
  int64_t scale_stride_block, scale_stride_head;
} ikl_rope_append_args;

/* Rotary embedding + KV append in one launch: query_out = rope(query);
 * cache.k[slot] = rope(key); cache.v[slot] = value; rope(x) = x * cos +
 * rotate_half(x) * sin with rotate_half(x) = [-x2, x1]. Bit-exact with the
 * torch elementwise sequence on the same cos / sin rows (each product and
 * the sum rounded to the tensor dtype); into an FP8 cache, equal to that
 * rotation followed by ikl_append_kv. Slots outside the cache are skipped;
 * query rows are rotated regardless. */
int ikl_rope_append_kv(const ikl_rope_append_args *args, void *stream);

/* Arguments of ikl_paged_prefill_attention.
 * Replaces paged_prefill_attention_sdpa (attention.py:230-321, called by the
 * batched prefill at hf_benchmark.py:491-498): the gather of the whole
 * prefix into dense K/V plus a masked SDPA, per layer. */
typedef struct ikl_paged_prefill_args {
  const void *query;         /* [batch, num_heads, query_width, head_dim] */
  int64_t q_stride_b, q_stride_h, q_stride_t;
  const void *k_cache;       /* base of cache.k[layer] */
  const void *v_cache;       /* base of cache.v[layer] */
  int64_t k_stride_block, k_stride_token, k_stride_head;
  int64_t v_stride_block, v_stride_token, v_stride_head;
  const void *block_tables;  /* [batch, table_width] physical block ids */
  int32_t table_type;        /* enum ikl_index_type */
  int64_t table_stride_b;
  int64_t table_width;
  const void *query_starts;  /* [batch] position of query row 0 */
  const void *context_lens;  /* [batch] end of the prefill range (exclusive) */
  int32_t lens_type;         /* enum ikl_index_type of query_starts and context_lens */
  void *out;                 /* [batch, num_heads, query_width, head_dim], dtype of query */
  int64_t out_stride_b, out_stride_h, out_stride_t;
  int64_t batch;
  int64_t query_width;
  int64_t num_blocks;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t dtype;             /* enum ikl_dtype (query, cache and out share it) */
  float scale;               /* softmax scale; <= 0 selects head_dim**-0.5 */
  /* Kernel family: -1 = automatic (ikl_paged_prefill_path), else
   * IKL_PATH_MFMA_GROUPED or IKL_PATH_SCALAR_GROUPED. */
  int32_t path;
  /* Optional hipEvent_t handles recorded on `stream` before [0] and after
   * [1] the attention kernel. NULL entries are skipped. */
  void *events[2];
  /* FP8 KV cache (cache_dtype IKL_FP8_E4M3; 0 = same as dtype), as in
   * ikl_paged_attention_args; MFMA kernel only. */
  int32_t cache_dtype;
  const void *k_scale;
  const void *v_scale;
  int64_t scale_stride_block, scale_stride_head;
} ikl_paged_prefill_args;

/* Causal prefill attention over the paged cache. Row t of request b sits at
 * position query_starts[b] + t; rows t < context_lens[b] - query_starts[b]
 * attend the positions <= their own, the other rows of the query width
 * receive the value at position 0 (what the reference's mask leaves them).
 * The cache must already hold positions [0, context_lens[b]). Positions
 * whose block id is outside [0, num_blocks) are masked; the kernels never
 * read outside the cache. Replaces attention.py:230-321. */
int ikl_paged_prefill_attention(const ikl_paged_prefill_args *args, void *stream);

/* Kernel family a prefill launch uses: IKL_PATH_MFMA_GROUPED for fp16/bf16
 * with head_dim in {32, 64, 96, 128} and block_size a multiple of 16, else
 * IKL_PATH_SCALAR_GROUPED. dtype: enum ikl_dtype. */
int32_t ikl_paged_prefill_path(int32_t dtype, int32_t head_dim, int32_t block_size);

/* Message of the last failed call on this thread ("" if none). */
const char *ikl_last_error(void);

/* Library version string. */
const char *ikl_version(void);

/* Reads `bytes` of a contiguous device buffer once (16-byte aligned, a
 * multiple of 16 bytes) with streaming vector loads, and writes nothing of
 * note: `sink` (sink_bytes >= 4 x 8 x CU count) only receives a word in the
 * case its loads XOR to a fixed tag, which keeps them from being optimised
 * away. Timing it on a buffer larger than the MALL states the plain-stream
 * HBM read rate of the device, the ceiling for the attention kernels'
 * algorithmic GB/s. A measurement aid with no counterpart in the
 * reference. */
int ikl_hbm_read_probe(const void *buffer, int64_t bytes, void *sink, int64_t sink_bytes, void *stream);

/* Version of this C ABI (the argument structs and entry points declared
 * here). A caller compares it with IKL_ABI_VERSION of the header it was
 * built against and refuses to run on a mismatch. No counterpart in the
 * reference, whose operators are Python functions. */
#define IKL_ABI_VERSION 3
int32_t ikl_abi_version(void);

/* KV append (in place). Slots outside [0, num_blocks*block_size) are skipped,
 * never written. Replaces append.py:69-106 / cache.py:156-189. */
int ikl_append_kv(const ikl_append_args *args, void *stream);

/* Bytes of workspace the launch described by `args` needs (0 when it runs
 * without split partials). Negative on invalid arguments. */
int64_t ikl_paged_attention_workspace_size(const ikl_paged_attention_args *args);

/* Resolved split partition size (tokens) for `args`, or 0 when the launch
 * runs without splitting. Negative on invalid arguments. */
int32_t ikl_paged_attention_partition_size(const ikl_paged_attention_args *args);

/* Paged decode attention. Positions p < context_lens[b] whose physical block
 * id is outside [0, num_blocks) are masked (like triton_ops.py:138); the
 * kernels never read outside the cache. Replaces triton_ops.py:404-610. */
int ikl_paged_attention(const ikl_paged_attention_args *args, void *stream);

/* Bytes of the per-device scratch array behind ikl_paged_attention_noalloc. */
#define IKL_NOALLOC_SCRATCH_BYTES (16u << 20)

/* ikl_paged_attention without a caller workspace and without any device
 * allocation: the split partials go to a 16 MiB array the library holds on
 * each device for the life of the process (found once per device with
 * hipGetSymbolAddress, on the first call with that device current). No
 * counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The first call on each device must run outside stream
 * capture: it looks the array's address up with hipGetSymbolAddress; later
 * calls only enqueue kernels and may be captured.
 * args->workspace / workspace_bytes are ignored. A launch whose
 * split needs more than IKL_NOALLOC_SCRATCH_BYTES (see
 * ikl_paged_attention_workspace_size) fails with IKL_EWORKSPACE. All calls
 * on one device share the array: calls that overlap on that device (on
 * different streams, or concurrently from several threads) race. */
int ikl_paged_attention_noalloc(const ikl_paged_attention_args *args, void *stream);

/* One decode step of the synthetic runner's order (decode.py:480-487):
 * paged decode attention over context_lens, then the KV append of the
 * step's new rows. When the attention splits (a reduce kernel runs) and the
 * append is a plain copy in 16-byte pieces (16-bit or fp32 cache, aligned
 * rows of at most 512 bytes) or a quantising append into an FP8 cache whose
 * key / value rows are in the attention's dtype, the reduce kernel's
 * workgroups also do the append: one launch less per step, with the same
 * result as ikl_paged_attention followed by ikl_append_kv, codes and scales
 * included (the reduce runs after the attention kernel has read the cache).
 * Otherwise the two run as separate launches in that order. Both argument
 * structs are validated before anything is enqueued. No counterpart in the
 * reference, which launches the two operators separately. */
int ikl_paged_decode_step(const ikl_paged_attention_args *attention, const ikl_append_args *append,
                          void *stream);

/* 1 when ikl_paged_decode_step with these arguments fuses the append into
 * the reduce kernel, 0 when it launches it separately, negative on invalid
 * arguments. Planning only: launches nothing. */
int32_t ikl_paged_decode_step_fused(const ikl_paged_attention_args *attention,
                                    const ikl_append_args *append);

/* Workspace bytes that ikl_paged_decode_step uses with these arguments:
 * the attention's (ikl_paged_attention_workspace_size); an unsplit
 * attention, folded multi-wave workgroups included, is followed by the
 * append's own launch. Negative on invalid arguments. Planning only. No
 * counterpart in the reference (see ikl_paged_decode_step). */
int64_t ikl_paged_decode_step_workspace_size(const ikl_paged_attention_args *attention,
                                             const ikl_append_args *append);

/* Static path selection for a grouped launch; mirrors the role of
 * paged_decode_grouped_path (triton_ops.py:56-75) for this library's
 * kernel families. Name mapping to the reference's strings:
 * IKL_PATH_MHA_FALLBACK = "mha_fallback" and IKL_PATH_SCALAR_GROUPED =
 * "scalar_grouped" in both; IKL_PATH_MFMA_GROUPED ("mfma_grouped" in the
 * Python wrapper) is the counterpart of the reference's
 * "tensorcore_short_context" (the dense group x tile contraction on the
 * matrix cores). The two rules differ where the reference's kernel has
 * limits this one does not: the reference answers "scalar_grouped" for
 * table_width > 16 or an effective group below 4 heads, where this library
 * still runs the matrix cores, and it takes any head_dim >= 16 where this
 * one needs 32, 64, 96 or 128; the other rows of the reference's truth
 * table (tests/test_attention.py:22-42) agree under the mapping.
 * Rule: MHA (heads_per_kv == 1) -> IKL_PATH_MHA_FALLBACK;
 * fp16/bf16 with head_dim in {32, 64, 96, 128} and block_size a multiple of
 * 16 -> IKL_PATH_MFMA_GROUPED; otherwise IKL_PATH_SCALAR_GROUPED. The
 * reference's selector has no block_size argument; this one needs it
 * because the MFMA tiles assume 16-token block alignment. table_width does
 * not influence the choice (the MFMA path has no context-length limit).
 * dtype: enum ikl_dtype. Returns enum ikl_attention_path. */
int32_t ikl_paged_attention_path(int32_t dtype, int32_t head_dim, int32_t block_size,
                                 int64_t table_width, int32_t heads_per_kv,
                                 int32_t query_group_size);

/* Resolved launch of an ikl_paged_attention call (filled by
 * ikl_paged_attention_launch_config). The caller sets struct_size to
 * sizeof(ikl_launch_config) of the header it was built against; the library
 * fills only the fields that fit in it, so the struct can grow at its end
 * without older callers being written past. */
typedef struct ikl_launch_config {
  int32_t struct_size;         /* in: bytes the caller allocated (>= IKL_LAUNCH_CONFIG_MIN_BYTES) */
  int32_t path;                /* enum ikl_attention_path */
  int32_t tile_tokens;         /* positions one wave takes per loop step */
  int32_t waves_per_workgroup;
  int32_t stages;              /* tiles in flight per wave (software pipeline depth) */
  int32_t split;               /* 0 = none, 1 = fixed partitions, 2 = balanced split */
  int32_t partition_size;      /* as ikl_paged_attention_partition_size */
  int64_t workgroups;          /* grid size of the attention kernel */
  int32_t group_size;          /* query heads that share each K/V tile (one unit) */
} ikl_launch_config;

/* Smallest struct_size accepted: the struct up to and including `workgroups`
 * (group_size and later fields are filled when struct_size covers them). */
#define IKL_LAUNCH_CONFIG_MIN_BYTES 40

/* Launch configuration `args` resolves to, without launching. Replaces the
 * autotune-config reporters of triton_ops.py:17-53 (block_n / num_warps /
 * num_stages of the last autotuned launch): these kernels are not
 * autotuned, their configuration follows from the arguments. Returns 0 or
 * a negative IKL_E* code (IKL_EINVAL when out->struct_size is below
 * IKL_LAUNCH_CONFIG_MIN_BYTES). */
int ikl_paged_attention_launch_config(const ikl_paged_attention_args *args, ikl_launch_config *out);

#ifdef __cplusplus
}
#endif

#endif /* IKL_PAGED_H */
