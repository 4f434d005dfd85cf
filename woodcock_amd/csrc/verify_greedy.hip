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

#include "argmax_verify.h"

namespace wc {

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
