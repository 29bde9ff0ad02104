// HBM read-bandwidth probe: the practical read ceiling that the paged decode
// kernel's bandwidth is compared with.  A grid-stride stream of streaming
// (non-temporal) 16-byte loads, the form the decode kernel reads K/V with,
// kProbeUnroll in flight per lane, folded by XOR into one word per lane so
// that no load can be dropped.  No counterpart in the reference.

#include "lvamd_common.h"

namespace lvamd {

constexpr int kProbeUnroll = 8;

__global__ __launch_bounds__(64) void hbm_read_probe_kernel(gptr<const u32x4> p, int64_t n16, gptr<uint32_t> sink) {
  const int64_t nthr = (int64_t)gridDim.x * 64;
  const int64_t tid = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  u32x4 acc = {0u, 0u, 0u, 0u};
  int64_t i = tid;
  for (; i + (kProbeUnroll - 1) * nthr < n16; i += kProbeUnroll * nthr) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * nthr);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += nthr) acc ^= p[i];
  sink[tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace lvamd

using namespace lvamd;

extern "C" int lvamd_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int32_t workgroups,
                                    lvamd_stream_t stream) {
  if (!buf || !sink || bytes < 0 || bytes % 16 != 0 || workgroups <= 0 || workgroups > 65536)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)buf & 15u) != 0 || ((uintptr_t)sink & 3u) != 0) return LVAMD_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(hbm_read_probe_kernel, dim3((unsigned)workgroups), dim3(64), 0,
                     static_cast<hipStream_t>(stream), (gptr<const u32x4>)(buf), bytes / 16,
                     (gptr<uint32_t>)(sink));
  return launch_status();
}
