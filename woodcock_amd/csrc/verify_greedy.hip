// verify_greedy.hip -- target argmax fused with greedy chain / tree acceptance.
//
// One launch covers the whole round's verification (python/woodcock/spec.py:355-361,
// python/woodcock/sampling.py:60-66,131-140): a grid of (chunk, row) blocks streams
// the fp32 logits once with 128-bit loads, each block folds its chunk into a
// packed (value, lowest index) key and publishes it with one device-scope
// atomicMax per row; the last block to finish runs the acceptance scan with
// wave-wide ballots and writes a wc_verdict, then clears the slots and its
// counter so the kernel can be replayed (graph-safe, no memset).
#include <mutex>

#include "wc_common.h"

namespace wc {

constexpr int kArgBlock = 256;
constexpr int kArgItems = 4;                            // float4 loads per thread
constexpr int kArgChunk = kArgBlock * 4 * kArgItems;    // 4096 logits per block

enum VerifyMode { kModeArgmax = 0, kModeChain = 1, kModeTree = 2 };

template <bool VEC>
__device__ __forceinline__ unsigned long long chunk_argmax(const float* __restrict__ row, int begin, int end) {
  unsigned long long best = 0;
  if (VEC) {
    float4 v[kArgItems];
    int idx[kArgItems];
#pragma unroll
    for (int j = 0; j < kArgItems; ++j) {
      idx[j] = begin + (j * kArgBlock + static_cast<int>(threadIdx.x)) * 4;
      if (idx[j] + 3 < end) v[j] = *reinterpret_cast<const float4*>(row + idx[j]);
    }
#pragma unroll
    for (int j = 0; j < kArgItems; ++j) {
      const int i = idx[j];
      if (i + 3 < end) {
        unsigned long long k0 = argmax_key(v[j].x, i), k1 = argmax_key(v[j].y, i + 1);
        unsigned long long k2 = argmax_key(v[j].z, i + 2), k3 = argmax_key(v[j].w, i + 3);
        k0 = k1 > k0 ? k1 : k0;
        k2 = k3 > k2 ? k3 : k2;
        k0 = k2 > k0 ? k2 : k0;
        best = k0 > best ? k0 : best;
      } else {
        for (int t = i; t < end && t < i + 4; ++t) {
          const unsigned long long k = argmax_key(row[t], t);
          best = k > best ? k : best;
        }
      }
    }
  } else {
    for (int i = begin + static_cast<int>(threadIdx.x); i < end; i += kArgBlock) {
      const unsigned long long k = argmax_key(row[i], i);
      best = k > best ? k : best;
    }
  }
  return best;
}

template <bool VEC>
__global__ __launch_bounds__(kArgBlock) void k_argmax_verify(
    const float* __restrict__ logits, int rows, int vocab, int64_t ld, unsigned long long* __restrict__ slots,
    unsigned int* __restrict__ counter, int mode, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ tree_parents, int32_t* __restrict__ argmax_out,
    wc_verdict* __restrict__ verdict) {
  const int r = blockIdx.y;
  const int begin = blockIdx.x * kArgChunk;
  const int end = min(vocab, begin + kArgChunk);
  unsigned long long best = chunk_argmax<VEC>(logits + static_cast<int64_t>(r) * ld, begin, end);

  __shared__ unsigned long long s_part[kArgBlock / kWave];
  best = wave_max_u64(best);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_part[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgBlock / kWave; ++w) best = s_part[w] > best ? s_part[w] : best;
    atomic_max_u64(&slots[r], best);
  }
  if (!last_block_done(counter, gridDim.x * gridDim.y)) return;
  if (wave != 0) return;

  // ---- last block, wave 0: lane c owns row / node c (rows <= 64)
  const int c = lane;
  int t = -1;
  if (c < rows) {
    t = argmax_key_index(atomic_load_u64(&slots[c]));
    atomic_store_u64(&slots[c], 0ull);
    if (argmax_out) argmax_out[c] = t;
  }
  if (mode == kModeChain) {
    const int K = rows - 1;
    const bool match = c < K && drafts[c] == t;
    const unsigned long long m = __ballot(match);
    int a = __ffsll(static_cast<long long>(~m)) - 1;  // leading matches
    if (a < 0 || a > K) a = K;
    const int next = __shfl(t, a);
    if (c < a) {
      verdict->tokens[c] = drafts[c];
      verdict->keep[c] = c;
    }
    if (c == a) {
      verdict->tokens[c] = next;
      verdict->keep[c] = c;
      verdict->n_accepted = a;
      verdict->next = next;
      verdict->n_keep = a + 1;
      verdict->n_uniforms = 0;
      verdict->status = 0;
    }
  } else if (mode == kModeTree) {
    const int N = rows;
    const int tok = c < N ? tree_tokens[c] : -1;
    const int par = c < N ? tree_parents[c] : -2;
    const bool bad = c < N && (c == 0 ? par != -1 : (par < 0 || par >= N));
    const bool any_bad = __ballot(bad) != 0ull;
    int v = 0, len = 0, want = __shfl(t, 0);
    if (!any_bad) {
      for (int step = 0; step < N; ++step) {  // a path has at most N-1 edges
        want = __shfl(t, v);
        const unsigned long long m = __ballot(c < N && par == v && tok == want);
        if (m == 0ull) break;
        const int nxt = __ffsll(static_cast<long long>(m)) - 1;  // first child in draw order
        const int nxt_tok = __shfl(tok, nxt);                   // whole wave participates
        if (c == 0) {
          verdict->keep[1 + len] = nxt;
          verdict->tokens[len] = nxt_tok;
        }
        ++len;
        v = nxt;
      }
      want = __shfl(t, v);
    }
    if (c == 0) {
      verdict->keep[0] = 0;
      verdict->tokens[len] = want;
      verdict->n_accepted = len;
      verdict->next = want;
      verdict->n_keep = len + 1;
      verdict->n_uniforms = 0;
      verdict->status = any_bad ? WC_E_INVALID : 0;
    }
  }
}

static int launch_argmax_verify(const float* logits, int rows, int vocab, int64_t ld, int mode, const int32_t* drafts,
                                const int32_t* tree_tokens, const int32_t* tree_parents, int32_t* argmax_out,
                                wc_verdict* verdict, void* workspace, hipStream_t stream) {
  WC_REQUIRE(logits != nullptr, "logits is NULL");
  WC_REQUIRE(workspace != nullptr && aligned(workspace, 16), "workspace is NULL or not 16-byte aligned");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "rows must be in 1..%d (got %d)", WC_MAX_NODES, rows);
  WC_REQUIRE(vocab >= 1, "vocab must be positive (got %d)", vocab);
  WC_REQUIRE(ld >= vocab, "row stride %lld smaller than vocab %d", static_cast<long long>(ld), vocab);
  auto* slots = static_cast<unsigned long long*>(workspace);
  auto* counter = verify_counter(workspace, kCtrArgmax);
  const dim3 grid((vocab + kArgChunk - 1) / kArgChunk, rows);
  const bool vec = aligned(logits, 16) && (ld % 4) == 0;
  if (vec)
    hipLaunchKernelGGL(k_argmax_verify<true>, grid, dim3(kArgBlock), 0, stream, logits, rows, vocab, ld, slots,
                       counter, mode, drafts, tree_tokens, tree_parents, argmax_out, verdict);
  else
    hipLaunchKernelGGL(k_argmax_verify<false>, grid, dim3(kArgBlock), 0, stream, logits, rows, vocab, ld, slots,
                       counter, mode, drafts, tree_tokens, tree_parents, argmax_out, verdict);
  WC_LAUNCHED();
  return WC_OK;
}

// ------------------------------------------------------------------ scratch without allocation
// wc_verify_chain_greedy_static keeps its scratch -- the argmax slots of up to
// WC_MAX_NODES rows, then the argmax counter tree, laid out as in a verify
// workspace -- in this file-scope device array: one copy per GPU, alive until
// the process ends.  Host code never passes the array's name to a kernel (in
// host code it is only a stand-in for the symbol); it passes the device
// address hipGetSymbolAddress returns, queried once per device with that
// device current.
constexpr size_t kStaticScratchBytes = kCounterOff + (kCtrArgmax + 1) * kTreeCounterBytes;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];

static int static_scratch(void** out) {
  int dev = 0;
  WC_HIP(hipGetDevice(&dev));
  WC_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "static scratch: device %d beyond the %d supported", dev,
             kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(WC_E_HIP, "static scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WC_OK;
}

}  // namespace wc

extern "C" {

int wc_verify_chain_greedy_static(const float* logits, int rows, int vocab, int64_t ld,
                                  const int32_t* draft_tokens_dev, wc_verdict* verdict_dev, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(verdict_dev != nullptr, "wc_verify_chain_greedy_static: verdict is NULL");
  WC_REQUIRE(rows == 1 || draft_tokens_dev != nullptr, "wc_verify_chain_greedy_static: draft tokens are NULL");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES,
             "wc_verify_chain_greedy_static: %d rows exceed the %d rows its static scratch holds", rows,
             WC_MAX_NODES);
  void* ws = nullptr;
  if (int rc = static_scratch(&ws)) return rc;
  // slots and counters start at zero: cleared by a kernel (no memset node, so
  // a captured call stays valid), whatever an earlier call left
  if (int rc = wc_workspace_init(ws, kStaticScratchBytes, stream)) return rc;
  return launch_argmax_verify(logits, rows, vocab, ld, kModeChain, draft_tokens_dev, nullptr, nullptr, nullptr,
                              verdict_dev, ws, reinterpret_cast<hipStream_t>(stream));
}

int wc_argmax_rows(const float* logits, int rows, int vocab, int64_t ld, int32_t* out_dev, void* workspace,
                   wc_stream_t stream) {
  WC_REQUIRE(out_dev != nullptr, "wc_argmax_rows: out is NULL");
  return wc::launch_argmax_verify(logits, rows, vocab, ld, wc::kModeArgmax, nullptr, nullptr, nullptr, out_dev,
                                  nullptr, workspace, reinterpret_cast<hipStream_t>(stream));
}

int wc_verify_chain_greedy(const float* logits, int rows, int vocab, int64_t ld, const int32_t* draft_tokens_dev,
                           wc_verdict* verdict_dev, void* workspace, wc_stream_t stream) {
  WC_REQUIRE(verdict_dev != nullptr, "wc_verify_chain_greedy: verdict is NULL");
  WC_REQUIRE(rows == 1 || draft_tokens_dev != nullptr, "wc_verify_chain_greedy: draft tokens are NULL");
  return wc::launch_argmax_verify(logits, rows, vocab, ld, wc::kModeChain, draft_tokens_dev, nullptr, nullptr,
                                  nullptr, verdict_dev, workspace, reinterpret_cast<hipStream_t>(stream));
}

int wc_verify_tree_greedy(const float* logits, int rows, int vocab, int64_t ld, const int32_t* tree_tokens_dev,
                          const int32_t* tree_parents_dev, wc_verdict* verdict_dev, void* workspace,
                          wc_stream_t stream) {
  WC_REQUIRE(verdict_dev != nullptr, "wc_verify_tree_greedy: verdict is NULL");
  WC_REQUIRE(tree_tokens_dev != nullptr && tree_parents_dev != nullptr, "wc_verify_tree_greedy: tree is NULL");
  return wc::launch_argmax_verify(logits, rows, vocab, ld, wc::kModeTree, nullptr, tree_tokens_dev, tree_parents_dev,
                                  nullptr, verdict_dev, workspace, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
