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
// compute units of the current device (queried once per device)
int device_cus(int* cus);

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
// The verify kernels share one zero-initialised workspace:
//   [0, 8*WC_MAX_NODES)                  per-row argmax slots (uint64 keys)
//   then kNumCounters tree counters      (kTreeCounterBytes each, see last_block_done)
//   then the stochastic / softmax scratch (kStochRowOff ... kVerifyWorkspace)
constexpr size_t kSlotBytes = 8 * WC_MAX_NODES;
constexpr size_t kCounterOff = kSlotBytes;
constexpr int kNumCounters = 4;
enum Counter { kCtrArgmax = 0, kCtrStochastic = 1, kCtrTree = 2, kCtrStochStats = 3 };

// ------------------------------------------------------------------ device helpers

constexpr int kWave = 64;
constexpr int kSlots = 32;       // draft-head argmax atomics are spread over kSlots addresses per row
constexpr int kSlotStride = 16;  // uint64s between slots: one 128-byte line each

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

// Wave-wide sum with DPP lane moves (VALU, no LDS round trip): pairwise and
// quad exchanges, two rotations complete each 16-lane row, the row broadcasts
// of lanes 15 and 31 fold the four rows into lane 63, which is read back
// uniformly.  Same value on every lane on return.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_move<0x124>(v);       // row_ror:4
  v += dpp_move<0x128>(v);       // row_ror:8
  v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_move<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave-wide max (exact in any order) with DPP moves; lanes outside a
// broadcast's rows keep their own value.  Every lane of the wave must be active.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move_keep(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x124>(v));
  v = fmaxf(v, dpp_move<0x128>(v));
  v = fmaxf(v, dpp_move_keep<0x142, 0xA>(v));
  v = fmaxf(v, dpp_move_keep<0x143, 0xC>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// fp64 lane moves: the two halves moved alike.  BC: lanes whose source lies
// outside the row (or wave) receive 0.
template <int CTRL, int ROW_MASK = 0xf, bool BC = false>
__device__ __forceinline__ double dpp_move_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), CTRL, ROW_MASK, 0xf, BC);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), CTRL, ROW_MASK, 0xf, BC);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), lane);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
// fp64 wave sum, the association of wave_sum_dpp; same value on every lane.
// Every lane of the wave must be active.
__device__ __forceinline__ double wave_sum_dpp(double v) {
  v += dpp_move_f64<0xB1>(v);
  v += dpp_move_f64<0x4E>(v);
  v += dpp_move_f64<0x124>(v);
  v += dpp_move_f64<0x128>(v);
  v += dpp_move_f64<0x142, 0xA>(v);
  v += dpp_move_f64<0x143, 0xC>(v);
  return readlane_f64(v, 63);
}
// Inclusive prefix sum over the lanes in lane order: Hillis-Steele steps of 1,
// 2, 4, 8 lanes within each 16-lane row, then the row totals carried by the
// lane-15 and lane-31 broadcasts.  Every lane of the wave must be active.
__device__ __forceinline__ double wave_incl_scan_dpp(double x) {
  x += dpp_move_f64<0x111, 0xf, true>(x);  // row_shr:1
  x += dpp_move_f64<0x112, 0xf, true>(x);  // row_shr:2
  x += dpp_move_f64<0x114, 0xf, true>(x);  // row_shr:4
  x += dpp_move_f64<0x118, 0xf, true>(x);  // row_shr:8
  x += dpp_move_f64<0x142, 0xA>(x);        // row_bcast:15 into rows 1 and 3
  x += dpp_move_f64<0x143, 0xC>(x);        // row_bcast:31 into rows 2 and 3
  return x;
}
// the inclusive scan moved up one lane (lane 0: 0)
__device__ __forceinline__ double wave_excl_from_incl(double incl) {
  return dpp_move_f64<0x138, 0xf, true>(incl);  // wave_shr:1
}

// Reductions over the 16 lanes of a DPP row (lanes 16r .. 16r + 15); every
// lane of the row receives the result.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_move<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_move<0x128>(v));  // row_ror:8
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x124>(v);
  v += dpp_move<0x128>(v);
  return v;
}

// Ties a loaded value to this point: its load cannot be sunk into a later
// conditional block, where it would wait on its own, one load after another.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(unsigned long long& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }

// Wait states between the last MFMA of a loop and the first instruction that
// reads its result registers (LDS / memory stores, VALU): 24, beyond the 19 the
// longest XDL operation needs.  Issued explicitly after MFMA loops because the
// compiler's own count has fallen short on gfx950: with ~13 instructions
// between a v_mfma_f32_16x16x32_bf16 and the ds_write of its result, elements
// 2-3 of the tile were read stale, differently from run to run.
__device__ __forceinline__ void mfma_settle() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Workgroup barrier that orders LDS only: global loads in flight stay in flight
// (the plain __syncthreads() fence would wait for every outstanding load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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

// Philox4x64-10 (Salmon et al., SC'11): same stream as the host oracle.
__device__ __forceinline__ void philox4x64(unsigned long long c[4], unsigned long long k0, unsigned long long k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B97F4A7C15ull;
      k1 += 0xBB67AE8584CAA73Bull;
    }
    const unsigned long long lo0 = 0xD2E7470EE14C6C93ull * c[0], hi0 = __umul64hi(0xD2E7470EE14C6C93ull, c[0]);
    const unsigned long long lo1 = 0xCA5A826395121157ull * c[2], hi1 = __umul64hi(0xCA5A826395121157ull, c[2]);
    const unsigned long long n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

// uniform i of (seed, round, purpose): counter (i/4, round, purpose, 0), key (seed, 0), word i%4
__device__ __forceinline__ double philox_uniform(unsigned long long seed, unsigned long long round, int purpose,
                                                 unsigned long long i) {
  unsigned long long c[4] = {i >> 2, round, static_cast<unsigned long long>(purpose), 0ull};
  philox4x64(c, seed, 0ull);
  return static_cast<double>(c[i & 3] >> 11) * (1.0 / 9007199254740992.0);
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

// Device-coherent publish / fetch of single words: agent-scope atomic stores and
// loads (sc1 on gfx950), visible across the XCDs of the GPU without an L2
// write-back or invalidate.
__device__ __forceinline__ void publish_f32(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<unsigned int*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch_f32(const float* p) {
  return __uint_as_float(
      __hip_atomic_load(reinterpret_cast<const unsigned int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// "Last block done" handshake.  Every block calls this once (all threads) after
// handing its partial results over with publish_*() or device-scope RMW atomics;
// returns true in exactly one block, the last to arrive, which then reads them
// with fetch_*() / atomic loads.  Each thread first waits until its own
// published stores and atomics have completed, the block barriers, and relaxed
// RMWs on counters order the blocks -- no cache write-back or invalidate is
// involved.  Plain stores are NOT handed over (they become visible at the end
// of the kernel).
//
// The counters form a two-level tree so that no address takes more than
// ~total/64 RMWs: block b increments group counter b % G; the block completing
// a group increments the root; the block completing the root is the last.
// Every counter sits on its own 128-byte line and is reset by the block that
// completes it, so the kernel can be replayed without a host-side clear.
constexpr int kTreeGroups = 64;
constexpr int kCounterStride = 32;  // uints: one 128-byte line per counter
constexpr size_t kTreeCounterBytes = 4 * kCounterStride * (kTreeGroups + 1);

// Stochastic verification and probability kernels, after the counters:
//   per verify row (Q = draft mass, p(x), q(x) at the drafted token) as fp64,
//   per vocabulary chunk (residual mass, target mass) as fp64,
//   per (row, chunk) (max, sum of exp) of the softmax kernels as fp32.
constexpr int kVocabChunk = 4096;
constexpr int kMaxVocabChunks = 512;  // vocabularies up to 2,097,152 entries
constexpr size_t kStochRowOff = kCounterOff + kNumCounters * kTreeCounterBytes;
constexpr size_t kStochRowBytes = 8 * 4 * WC_MAX_NODES;
constexpr size_t kStochChunkOff = kStochRowOff + kStochRowBytes;
constexpr size_t kStochChunkBytes = 8 * 2 * kMaxVocabChunks;
constexpr size_t kProbsOff = kStochChunkOff + kStochChunkBytes;
constexpr size_t kProbsBytes = 4 * 2 * static_cast<size_t>(WC_MAX_NODES) * kMaxVocabChunks;
constexpr size_t kTreeStateOff = kProbsOff + kProbsBytes;  // stochastic tree walk state
constexpr size_t kTreeStateBytes = 4096;
// head row where each vocabulary chunk's ids start (d2t ascending), then the
// stochastic chain's decision (n, residual, uniforms) and the chosen row's
// softmax (max, sum) for the sampling launch
constexpr size_t kChunkRowsOff = kTreeStateOff + kTreeStateBytes;
constexpr size_t kChunkRowsBytes = 4 * (kMaxVocabChunks + 4);
constexpr size_t kStochDecOff = kChunkRowsOff + kChunkRowsBytes;
constexpr size_t kStochDecBytes = 64;
// the one-launch stochastic chain's two mailbox sets (one per call parity), then
// its control word (call counter | sticky failure flag << 32); each set ends with
// one arrival word per chunk block (at most 3 row groups per chunk)
constexpr int kMailRows = 8, kMailChunks = 256, kMailOther = 64, kMailRep = 4;
constexpr int kMailArrive = 3 * kMailChunks;
constexpr size_t kMailSetWords = kMailRep * (kMailRows * kMailChunks + 2 * kMailChunks + kMailOther) + kMailArrive;
// top-k warping: the k-th largest scaled logit of each row, as its order key
constexpr size_t kWarpOff = kStochDecOff + kStochDecBytes;
constexpr size_t kWarpBytes = 4 * WC_MAX_NODES;
constexpr size_t kGridBarOff = kWarpOff + kWarpBytes;
constexpr size_t kGridBarBytes = 2 * 8 * kMailSetWords + 128;
constexpr size_t kVerifyWorkspace = kGridBarOff + kGridBarBytes;
inline unsigned int* verify_counter(void* ws, int which) {
  return reinterpret_cast<unsigned int*>(static_cast<char*>(ws) + kCounterOff + which * kTreeCounterBytes);
}

__device__ __forceinline__ unsigned int linear_block() { return blockIdx.y * gridDim.x + blockIdx.x; }

// idx: this block's index among the `total` blocks counted on ctr.
__device__ __forceinline__ bool last_block_done(unsigned int* ctr, unsigned int total, unsigned int idx) {
  __shared__ bool s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int G = total < kTreeGroups ? total : kTreeGroups;
    const unsigned int g = idx % G;
    const unsigned int gsize = total / G + (g < total % G ? 1u : 0u);
    unsigned int* leaf = ctr + kCounterStride * (1 + g);
    bool last = false;
    if (__hip_atomic_fetch_add(leaf, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1) {
      __hip_atomic_store(leaf, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == G - 1) {
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = true;
      }
    }
    s_last = last;
  }
  __syncthreads();
  return s_last;
}

__device__ __forceinline__ bool last_block_done(unsigned int* ctr, unsigned int total) {
  return last_block_done(ctr, total, linear_block());
}

}  // namespace wc
