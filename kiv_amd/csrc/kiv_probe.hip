// Read-bandwidth probes: the achievable bandwidth of HBM and of the host
// link (mapped pinned host memory read by the GPU), measured with the same
// kind of 16-byte streaming loads the retrieval kernels issue.  They have
// no counterpart in the reference; they give the retrieval kernels'
// bandwidth figures a measured ceiling on the same machine.
#include <string.h>

#include <algorithm>

#include "kiv_common.h"
#include "kiv_internal.h"

namespace kiv {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;
constexpr size_t kScrubBytes = size_t(512) << 20;  // > L2 + MALL

// Each thread reads kProbeUnroll 16-byte words per step (all issued before
// any is used), grid-stride over the buffer, and folds them into one word.
// The fold is stored only when it hits a constant no real buffer is
// expected to produce, which keeps the loads without writing memory.
__global__ void __launch_bounds__(kProbeThreads) probe_read_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                                   uint32_t *sink) {
  const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
  uint32_t acc = 0;
  int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

}  // namespace kiv

using namespace kiv;

extern "C" {

int kiv_probe_read_bandwidth(int32_t where, size_t bytes, int32_t blocks, int32_t iters, int32_t cold,
                             double *gbps, kiv_stream_t stream) {
  if (!gbps || bytes < 16 || iters < 1 || blocks < 0 || (where != KIV_TIER_HOST && where != KIV_TIER_HBM))
    return fail(KIV_ERR_INVALID, "kiv_probe_read_bandwidth: bad argument");
  bytes &= ~size_t(15);
  hipStream_t st = (hipStream_t)stream;
  void *host = nullptr, *buf = nullptr, *scrub = nullptr;
  uint32_t *sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = KIV_OK;
  const int nb = blocks > 0 ? blocks : 1024;
  auto check = [&](hipError_t e, const char *what) {
    if (e != hipSuccess && rc == KIV_OK) rc = hip_fail(e, what);
    return rc == KIV_OK;
  };
  if (where == KIV_TIER_HOST) {
    if (check(hipHostMalloc(&host, bytes, hipHostMallocMapped), "hipHostMalloc"))
      check(hipHostGetDevicePointer(&buf, host, 0), "hipHostGetDevicePointer");
    if (rc == KIV_OK) memset(host, 0x5a, bytes);
  } else if (check(hipMalloc(&buf, bytes), "hipMalloc")) {
    check(hipMemsetAsync(buf, 0x5a, bytes, st), "hipMemsetAsync");
  }
  if (rc == KIV_OK && cold && check(hipMalloc(&scrub, kScrubBytes), "hipMalloc"))
    check(hipMemsetAsync(scrub, 0x33, kScrubBytes, st), "hipMemsetAsync");
  if (rc == KIV_OK) check(hipMalloc((void **)&sink, (size_t)std::max(nb, 4096) * 4), "hipMalloc");
  // Timing-only events: no system-scope fence to time with the reads.
  if (rc == KIV_OK) check(hipEventCreateWithFlags(&e0, hipEventDisableSystemFence), "hipEventCreateWithFlags");
  if (rc == KIV_OK) check(hipEventCreateWithFlags(&e1, hipEventDisableSystemFence), "hipEventCreateWithFlags");
  if (rc == KIV_OK) {
    const int64_t n16 = (int64_t)(bytes / 16);
    hipLaunchKernelGGL(probe_read_kernel, dim3(nb), dim3(kProbeThreads), 0, st, (const uint4 *)buf, n16, sink);
    double total_ms = 0.0;
    // Warm: one interval over all launches.  Cold: each launch timed on its
    // own, after a streaming read of kScrubBytes that evicts the caches.
    const int rounds = cold ? iters : 1, per_round = cold ? 1 : iters;
    for (int it = 0; it < rounds && rc == KIV_OK; ++it) {
      if (cold)
        hipLaunchKernelGGL(probe_read_kernel, dim3(4096), dim3(kProbeThreads), 0, st, (const uint4 *)scrub,
                           (int64_t)(kScrubBytes / 16), sink);
      check(hipEventRecord(e0, st), "hipEventRecord");
      for (int k = 0; k < per_round; ++k)
        hipLaunchKernelGGL(probe_read_kernel, dim3(nb), dim3(kProbeThreads), 0, st, (const uint4 *)buf, n16, sink);
      check(hipGetLastError(), "probe_read_kernel");
      check(hipEventRecord(e1, st), "hipEventRecord");
      check(hipEventSynchronize(e1), "hipEventSynchronize");
      float ms = 0.f;
      if (check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime")) total_ms += ms;
    }
    if (rc == KIV_OK) *gbps = (double)bytes * iters / (total_ms * 1e-3) / 1e9;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (sink) (void)hipFree(sink);
  if (scrub) (void)hipFree(scrub);
  if (host) (void)hipHostFree(host);
  else if (buf) (void)hipFree(buf);
  return rc;
}

}  // extern "C"
