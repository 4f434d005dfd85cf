// wc_lib.hip -- library-level entry points: version, errors, workspace.
#include <atomic>

#include "wc_common.h"

namespace wc {

static thread_local std::string g_error;

int set_error(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return status;
}

const char* last_error() { return g_error.c_str(); }

int device_cus(int* cus) {
  static std::atomic<int> cache[64];  // 0 = not yet queried
  int dev = 0;
  WC_HIP(hipGetDevice(&dev));
  int n = dev >= 0 && dev < 64 ? cache[dev].load(std::memory_order_relaxed) : 0;
  if (n == 0) {
    WC_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  }
  *cus = n;
  return WC_OK;
}

// zero-fill with plain vector stores (graph-safe replacement for hipMemsetAsync)
__global__ void k_fill_zero(uint4* __restrict__ p, size_t n16, unsigned char* __restrict__ tail, size_t ntail) {
  const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t j = i; j < n16; j += stride) p[j] = make_uint4(0, 0, 0, 0);
  if (i < ntail) tail[i] = 0;
}

}  // namespace wc

extern "C" {

int wc_version(void) { return WC_ABI_VERSION; }

const char* wc_last_error(void) { return wc::last_error(); }

size_t wc_workspace_bytes(void) { return wc::kVerifyWorkspace; }

int wc_workspace_init(void* workspace, size_t bytes, wc_stream_t stream) {
  WC_REQUIRE(workspace != nullptr, "wc_workspace_init: workspace is NULL");
  WC_REQUIRE(wc::aligned(workspace, 16), "wc_workspace_init: workspace must be 16-byte aligned");
  if (bytes == 0) return WC_OK;
  const size_t n16 = bytes / 16, ntail = bytes % 16;
  unsigned char* tail = static_cast<unsigned char*>(workspace) + n16 * 16;
  size_t blocks = (n16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(wc::k_fill_zero, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<uint4*>(workspace), n16, tail, ntail);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
