// kv_compact.hip -- in-place KV compaction of the accepted entries, all layers in one launch.
//
// compact_cache (python/woodcock/target.py:159-175) gathers rows start+keep[i]
// and writes them to start+i in every layer; KVCache::compact
// (src/cache/kv_cache.cpp:21-31) does the same with ascending memmoves.  Here
// one workgroup owns one (layer, K|V, kv head) slice [capacity][row_bytes]:
// it loads every kept row of its slice into registers with coalesced 16-byte
// loads, waits at a barrier, then stores them to their destinations, so the
// in-place move is hazard-free for any strictly increasing keep.  Slices are
// disjoint, so no inter-block ordering is needed.  keep / n_keep / start are
// read from device memory (e.g. straight out of a wc_verdict).
#include "wc_common.h"

namespace wc {

struct KVPtrs {
  void* k[WC_MAX_LAYERS];
  void* v[WC_MAX_LAYERS];
};

constexpr int kCompactBlock = 256;

template <typename U, int PER>
__global__ __launch_bounds__(kCompactBlock) void k_kv_compact(KVPtrs ptrs, int kv_heads, int cap, int row_bytes,
                                                              const int32_t* __restrict__ start_dev,
                                                              const int32_t* __restrict__ keep_dev,
                                                              const int32_t* __restrict__ n_keep_dev, int max_keep,
                                                              int32_t* __restrict__ offset_dev,
                                                              int32_t* __restrict__ status_dev) {
  __shared__ int s_keep[WC_MAX_NODES + 1];
  __shared__ int s_n, s_start, s_ok, s_ident;
  const int tid = threadIdx.x;
  if (tid == 0) {
    const int n = *n_keep_dev, start = *start_dev;
    s_n = n;
    s_start = start;
    s_ok = (n >= 0 && n <= max_keep && start >= 0);
  }
  __syncthreads();
  if (s_ok && tid < s_n) s_keep[tid] = keep_dev[tid];
  __syncthreads();
  if (tid == 0) {
    int ok = s_ok, ident = 1;
    const int n = ok ? s_n : 0;
    for (int i = 0; i < n; ++i) {
      const int k = s_keep[i];
      ok &= (k >= i) && (i == 0 || k > s_keep[i - 1]);
      ident &= (k == i);
    }
    if (n > 0) ok &= (s_start + s_keep[n - 1] < cap);
    s_ok = ok;
    s_ident = ident;
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      if (!ok && status_dev) *status_dev = WC_E_INVALID;
      if (ok && offset_dev) *offset_dev = s_start + n;
    }
  }
  __syncthreads();
  if (!s_ok || s_ident) return;  // identity keep: nothing moves (target.py:170)

  const int layer = blockIdx.y >> 1;
  char* base = static_cast<char*>((blockIdx.y & 1) ? ptrs.v[layer] : ptrs.k[layer]) +
               static_cast<int64_t>(blockIdx.x) * cap * row_bytes;
  const int units = row_bytes / static_cast<int>(sizeof(U));
  const int total = s_n * units;
  U reg[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = tid + j * kCompactBlock;
    if (idx < total) {
      const int i = idx / units, u = idx - i * units;
      reg[j] = reinterpret_cast<const U*>(base + static_cast<int64_t>(s_start + s_keep[i]) * row_bytes)[u];
    }
  }
  __syncthreads();  // every read of the slice precedes every write
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = tid + j * kCompactBlock;
    if (idx < total) {
      const int i = idx / units, u = idx - i * units;
      if (s_keep[i] != i) reinterpret_cast<U*>(base + static_cast<int64_t>(s_start + i) * row_bytes)[u] = reg[j];
    }
  }
}

template <typename U>
static int launch_compact(const KVPtrs& p, int n_layers, int kv_heads, int cap, int row_bytes, const int32_t* start,
                          const int32_t* keep, const int32_t* n_keep, int max_keep, int32_t* offset, int32_t* status,
                          hipStream_t stream) {
  const int units = row_bytes / static_cast<int>(sizeof(U));
  const int per = (max_keep * units + kCompactBlock - 1) / kCompactBlock;
  const dim3 grid(kv_heads, 2 * n_layers), block(kCompactBlock);
#define WC_COMPACT(N)                                                                                       \
  hipLaunchKernelGGL((k_kv_compact<U, N>), grid, block, 0, stream, p, kv_heads, cap, row_bytes, start, keep, \
                     n_keep, max_keep, offset, status)
  if (per <= 1)
    WC_COMPACT(1);
  else if (per <= 2)
    WC_COMPACT(2);
  else if (per <= 4)
    WC_COMPACT(4);
  else if (per <= 8)
    WC_COMPACT(8);
  else if (per <= 16)
    WC_COMPACT(16);
  else
    return set_error(WC_E_INVALID, "wc_kv_compact: max_keep*row_bytes = %d exceeds %d bytes", max_keep * row_bytes,
                     16 * kCompactBlock * static_cast<int>(sizeof(U)));
#undef WC_COMPACT
  WC_LAUNCHED();
  return WC_OK;
}

}  // namespace wc

extern "C" int wc_kv_compact(void* const* k_layers, void* const* v_layers, int n_layers, int kv_heads, int capacity,
                             int row_bytes, const int32_t* start_dev, const int32_t* keep_dev,
                             const int32_t* n_keep_dev, int max_keep, int32_t* offset_dev, int32_t* status_dev,
                             wc_stream_t stream) {
  WC_REQUIRE(k_layers && v_layers, "wc_kv_compact: layer pointer arrays are NULL");
  WC_REQUIRE(n_layers >= 1 && n_layers <= WC_MAX_LAYERS, "wc_kv_compact: n_layers must be in 1..%d (got %d)",
             WC_MAX_LAYERS, n_layers);
  WC_REQUIRE(kv_heads >= 1 && capacity >= 1, "wc_kv_compact: kv_heads and capacity must be positive");
  WC_REQUIRE(row_bytes > 0 && row_bytes % 4 == 0, "wc_kv_compact: row_bytes must be a positive multiple of 4");
  WC_REQUIRE(max_keep >= 1 && max_keep <= WC_MAX_NODES + 1, "wc_kv_compact: max_keep must be in 1..%d",
             WC_MAX_NODES + 1);
  WC_REQUIRE(start_dev && keep_dev && n_keep_dev, "wc_kv_compact: start/keep/n_keep are NULL");
  WC_REQUIRE(offset_dev == nullptr || (offset_dev != start_dev && offset_dev != n_keep_dev &&
                                       (offset_dev < keep_dev || offset_dev >= keep_dev + max_keep)),
             "wc_kv_compact: offset must not alias start, keep or n_keep (blocks read them concurrently)");
  wc::KVPtrs p{};
  bool vec16 = row_bytes % 16 == 0;
  for (int l = 0; l < n_layers; ++l) {
    WC_REQUIRE(k_layers[l] && v_layers[l], "wc_kv_compact: layer %d pointer is NULL", l);
    p.k[l] = k_layers[l];
    p.v[l] = v_layers[l];
    vec16 = vec16 && wc::aligned(k_layers[l], 16) && wc::aligned(v_layers[l], 16);
    WC_REQUIRE(wc::aligned(k_layers[l], 4) && wc::aligned(v_layers[l], 4), "wc_kv_compact: layer %d misaligned", l);
  }
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (vec16)
    return wc::launch_compact<uint4>(p, n_layers, kv_heads, capacity, row_bytes, start_dev, keep_dev, n_keep_dev,
                                     max_keep, offset_dev, status_dev, s);
  return wc::launch_compact<uint32_t>(p, n_layers, kv_heads, capacity, row_bytes, start_dev, keep_dev, n_keep_dev,
                                      max_keep, offset_dev, status_dev, s);
}
