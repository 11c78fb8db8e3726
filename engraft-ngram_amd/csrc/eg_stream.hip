// Streaming copy: the device's HBM streaming ceiling, measured with a kernel of
// this library rather than a runtime copy.  One 16-byte non-temporal load and
// one 16-byte non-temporal store per lane, one wavefront per 1 KiB, the grid
// sized to the copy: the shape that moved the most bytes per second among the
// one-shot and grid-stride shapes (1-8 vectors per lane) on MI355X.  The
// forward kernels stream their residual the same way, so this copy at the
// forward's traffic is the reference point of its roofline.
#include "eg_common.h"

namespace eg {

__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace eg

using namespace eg;

extern "C" {

int eg_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  EG_CHECK_ARG(bytes >= 0 && bytes % 16 == 0, "bytes=%lld must be a non-negative multiple of 16", (long long)bytes);
  EG_CHECK_ARG(bytes == 0 || (src != nullptr && dst != nullptr), "src/dst is NULL");
  EG_CHECK_ARG(((uintptr_t)src | (uintptr_t)dst) % 16 == 0, "src/dst must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  if (n16 == 0) return EG_OK;
  EG_CHECK_ARG((n16 + 255) / 256 < (1LL << 31), "bytes=%lld too large for one launch", (long long)bytes);
  hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)src, (u32x4*)dst, n16);
  return launch_status("stream_copy_kernel");
}

}  // extern "C"
