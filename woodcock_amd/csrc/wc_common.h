// wc_common.h -- shared host/device helpers of the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <string>

#include "../../include/woodcock_hip.h"

namespace wc {

// ------------------------------------------------------------------ host-side errors

int set_error(int status, const char* fmt, ...);
const char* last_error();

#define WC_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return ::wc::set_error(WC_E_INVALID, __VA_ARGS__); \
  } while (0)

#define WC_HIP(expr)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) return ::wc::set_error(WC_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

// after a launch: report launch-configuration errors without synchronising
#define WC_LAUNCHED()                                                                   \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess) return ::wc::set_error(WC_E_HIP, "launch: %s", hipGetErrorString(e_)); \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ------------------------------------------------------------------ workspace layout
// The verify kernels share one small zero-initialised workspace:
//   [0, 8*WC_MAX_NODES)            per-row argmax slots (uint64 keys)
//   [+0, +64)                      completion counters (uint32), one per kernel family
constexpr size_t kSlotBytes = 8 * WC_MAX_NODES;
constexpr size_t kCounterOff = kSlotBytes;
constexpr int kNumCounters = 16;
constexpr size_t kVerifyWorkspace = kCounterOff + 4 * kNumCounters + 64;
enum Counter { kCtrArgmax = 0, kCtrStochastic = 1, kCtrHead = 2 };

// ------------------------------------------------------------------ device helpers

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int m = kWave / 2; m > 0; m >>= 1) {
    unsigned long long o = __shfl_xor(v, m);
    v = o > v ? o : v;
  }
  return v;
}

// Monotone map float -> uint32 (larger float => larger key).  NaN maps above +inf,
// so a NaN wins an argmax as it does for numpy.argmax.
__device__ __forceinline__ uint32_t float_order(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (value, index) packed so that the max key is the max value at its LOWEST index
// (sampling.cpp:47 max_element, numpy argmax).  Key 0 means "empty".
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
  return (static_cast<unsigned long long>(float_order(v)) << 32) | static_cast<uint32_t>(0x7fffffff - idx);
}
__device__ __forceinline__ int argmax_key_index(unsigned long long k) {
  return 0x7fffffff - static_cast<int>(static_cast<uint32_t>(k & 0xffffffffu));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_float(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint16_t float_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Device-scope ("agent") atomics: coherent across the XCDs of one GPU.
__device__ __forceinline__ unsigned long long atomic_max_u64(unsigned long long* p, unsigned long long v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long atomic_load_u64(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u32(unsigned int* p, unsigned int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// "Last block done" handshake: every block calls this once after publishing its
// partial results (all threads of the block must call it).  Returns true in
// exactly one block -- the last to arrive -- after an acquire fence, so that
// block sees every other block's published writes.  That block must reset
// *counter to 0 (atomic_store_u32) before it exits, which makes the kernel
// re-launchable without a host-side clear.
__device__ __forceinline__ bool last_block_done(unsigned int* counter, unsigned int total) {
  __shared__ bool s_last;
  __threadfence();  // every thread releases its own writes (device scope: other XCDs' L2s)
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned int prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == total - 1);
  }
  __syncthreads();
  if (s_last) __threadfence();  // acquire the other blocks' writes
  return s_last;
}

}  // namespace wc
