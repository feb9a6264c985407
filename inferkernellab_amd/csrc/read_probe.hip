// HBM read-rate probe: streams a contiguous device buffer once with 16-byte
// non-temporal vector loads and writes nothing (a result word is stored
// only if the XOR of every loaded dword equals a fixed tag, which keeps the
// loads live without adding write traffic). The benchmark times it on a
// buffer larger than the 256 MB MALL to state, in the same run, the read
// rate the memory system delivers to a plain stream: the ceiling the
// attention kernels' GB/s sit under.
#include <algorithm>

#include "ikl_common.h"
#include "paged_attn.h"

namespace ikl {
namespace {

constexpr int PROBE_THREADS = 64;  // one wave per workgroup, one chunk per wave
constexpr int PROBE_UNROLL = 4;  // 16-byte loads in flight per thread
constexpr uint32_t PROBE_TAG = 0x9e3779b9u;

// Workgroup (one wave) w streams its own contiguous chunk [w n16 / G,
// (w + 1) n16 / G) of 16-byte pieces front to back (PROBE_UNROLL loads in
// flight per lane). On MI355X, 1 GiB: one-wave chunks at 8 waves per CU
// read 7.06 TB/s, 256-thread chunks 6.6-6.7, and a grid-stride sweep of the
// same buffer, which interleaves every wave's loads over all of it,
// 5.1-5.9.
__global__ __launch_bounds__(PROBE_THREADS) void hbm_read_probe_kernel(const v4u32 *__restrict__ src, int64_t n16,
                                                                        uint32_t *sink) {
  const int64_t lo = (int64_t)blockIdx.x * n16 / gridDim.x, hi = ((int64_t)blockIdx.x + 1) * n16 / gridDim.x;
  constexpr int STEP = PROBE_THREADS * PROBE_UNROLL;
  uint32_t acc = 0;
  int64_t i = lo + threadIdx.x;
  for (; i + (PROBE_UNROLL - 1) * PROBE_THREADS < hi; i += STEP) {
    v4u32 v[PROBE_UNROLL];
#pragma unroll
    for (int u = 0; u < PROBE_UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * PROBE_THREADS);
#pragma unroll
    for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < hi; i += PROBE_THREADS) {
    const v4u32 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == PROBE_TAG) sink[blockIdx.x] = acc;
}

}  // namespace
}  // namespace ikl

using namespace ikl;

extern "C" int ikl_hbm_read_probe(const void *buffer, int64_t bytes, void *sink, int64_t sink_bytes,
                                  void *stream) {
  if (!buffer || !sink || bytes <= 0) return fail(IKL_EINVAL, "read probe: null buffer or empty size");
  if (((uintptr_t)buffer & 15u) != 0 || bytes % 16 != 0)
    return fail(IKL_EINVAL, "read probe: the buffer must be 16-byte aligned and a multiple of 16 bytes");
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  const int64_t n16 = bytes / 16;
  // 8 one-wave workgroups per CU (2 waves per SIMD), fewer for a buffer
  // that cannot feed them one unrolled pass each
  const int64_t want = (n16 + PROBE_THREADS * PROBE_UNROLL - 1) / (PROBE_THREADS * PROBE_UNROLL);
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)cus * 8));
  if (sink_bytes < grid * 4)
    return fail(IKL_EINVAL, "read probe: the sink needs " + std::to_string(grid * 4) + " bytes");
  hbm_read_probe_kernel<<<dim3((unsigned)grid), dim3(PROBE_THREADS), 0, (hipStream_t)stream>>>(
      (const v4u32 *)buffer, n16, (uint32_t *)sink);
  return check_launch("read probe");
}
