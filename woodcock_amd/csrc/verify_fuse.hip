// verify_fuse.hip -- the greedy chain verify and the drafter's fuse in one launch.
//
// A chain round keeps the prefix [0..a] of its verify block
// (python/woodcock/spec.py:362-366), and the fuse is row-wise
// (python/woodcock/drafter.py:149-153), so the fuse of every one of the k + 1
// tap rows can run before the verdict is known; the drafter pass that follows
// reads rows 0..a of it.  Here the two share one grid sized to be resident at
// once (one twelve-wave block per CU): blocks [0, nv) are the verify's, each
// folding a chunk of up to three 12,288-logit batches of one logits row
// (loads for all batches issued before any is folded) into a packed (value,
// lowest index) key with one atomicMax, the last of them running the
// acceptance scan (argmax_verify.h); blocks [nv, grid) are the few-row GEMV's
// (gemvk.h, R output rows each, twelve waves: one 512-wide step of one tap
// each).  R = 10 (8 in the fuse's own launch) leaves the verify 51 of 256
// CUs at hidden 2048: a block per CU lets the verify's load -> atomic -> scan
// chain run beside the fuse's weight stream instead of after it or in a
// launch of its own.  The products and their summation order do not depend
// on R, so the results equal those of the two launches in sequence.
#include "argmax_verify.h"
#include "gemvk.h"

namespace wc {

int fuse_gemv_args(const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps, int tap_dtype,
                   int64_t tap_ld, int rows, float* g_out, int64_t g_ld, GemvArgs* out);

constexpr int kVfThreads = 12 * kWave;            // the fuse's twelve waves
constexpr int kVfBatch = arg_chunk<kVfThreads>();  // 12,288 logits: four float4 per thread
constexpr int kVfBatches = 3;                      // batches per verify block at most
constexpr int kVfRowsMax = 8;                      // input rows (k + 1) of the one-launch path
constexpr int kVfGemvRows = 10;                    // output rows per GEMV block (8 in the fuse's own launch)

struct VerifyFuseArgs {
  const float* logits;
  int rows, vocab;
  int64_t ld;
  unsigned long long* slots;
  unsigned int* counter;
  const int32_t* drafts;
  wc_verdict* verdict;
  int nvx;    // verify blocks per logits row
  int chunk;  // logits per verify block (a multiple of kVfBatch, at most kVfBatches of them)
};

template <int R, int MM, int XB, int GB>
__global__ __launch_bounds__(kVfThreads) void k_verify_fuse(VerifyFuseArgs v, GemvArgs a) {
  const int b = blockIdx.x;
  const int nv = v.nvx * v.rows;
  if (b >= nv) {
    gemvk_block<R, false, 3, 1, MM, XB, GB, 12>(a, b - nv, static_cast<int>(gridDim.x) - nv);
    return;
  }
  __shared__ unsigned long long s_part[kVfThreads / kWave];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int r = b / v.nvx;
  const float* row = v.logits + static_cast<int64_t>(r) * v.ld;
  const int begin = (b % v.nvx) * v.chunk, end = min(v.vocab, begin + v.chunk);
  // every full float4 of the chunk requested at once, then folded
  float4 x[kVfBatches][kArgItems];
#pragma unroll
  for (int q = 0; q < kVfBatches; ++q)
#pragma unroll
    for (int j = 0; j < kArgItems; ++j) {
      const int i = begin + q * kVfBatch + (j * kVfThreads + t) * 4;
      if (i + 3 < end) x[q][j] = *reinterpret_cast<const float4*>(row + i);
    }
  unsigned long long best = 0;
#pragma unroll
  for (int q = 0; q < kVfBatches; ++q)
#pragma unroll
    for (int j = 0; j < kArgItems; ++j) {
      const int i = begin + q * kVfBatch + (j * kVfThreads + t) * 4;
      if (i + 3 < end) {
        unsigned long long k0 = argmax_key(x[q][j].x, i), k1 = argmax_key(x[q][j].y, i + 1);
        unsigned long long k2 = argmax_key(x[q][j].z, i + 2), k3 = argmax_key(x[q][j].w, i + 3);
        k0 = k1 > k0 ? k1 : k0;
        k2 = k3 > k2 ? k3 : k2;
        k0 = k2 > k0 ? k2 : k0;
        best = k0 > best ? k0 : best;
      } else {
        for (int e = i; e < end && e < i + 4; ++e) {  // the ragged end of the row
          const unsigned long long k = argmax_key(row[e], e);
          best = k > best ? k : best;
        }
      }
    }
  best = wave_max_u64(best);
  if (lane == 0) s_part[wave] = best;
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kVfThreads / kWave; ++w) best = s_part[w] > best ? s_part[w] : best;
    atomic_max_u64(&v.slots[r], best);
  }
  if (!last_block_done(v.counter, nv, b)) return;
  if (wave != 0) return;
  verify_finish(lane, v.slots, v.rows, kModeChain, v.drafts, nullptr, nullptr, nullptr, v.verdict);
}

template <int R, int XB, int GB>
static void launch_vf_m(const VerifyFuseArgs& v, const GemvArgs& a, dim3 grid, hipStream_t s) {
  if (a.M <= 4)
    hipLaunchKernelGGL((k_verify_fuse<R, 4, XB, GB>), grid, dim3(kVfThreads), 0, s, v, a);
  else if (a.M <= 6)
    hipLaunchKernelGGL((k_verify_fuse<R, 6, XB, GB>), grid, dim3(kVfThreads), 0, s, v, a);
  else
    hipLaunchKernelGGL((k_verify_fuse<R, 8, XB, GB>), grid, dim3(kVfThreads), 0, s, v, a);
}

template <int XB, int GB>
static void launch_vf(const VerifyFuseArgs& v, const GemvArgs& a, dim3 grid, hipStream_t s) {
  launch_vf_m<kVfGemvRows, XB, GB>(v, a, grid, s);
}

}  // namespace wc

extern "C" {

int wc_verify_chain_greedy_fuse(const float* logits, int rows, int vocab, int64_t ld,
                                const int32_t* draft_tokens_dev, wc_verdict* verdict_dev, void* verify_workspace,
                                const wc_drafter_dims* dims, const wc_drafter_weights* w, const void* const* taps,
                                int tap_dtype, int64_t tap_ld, float* g_out, int64_t g_ld, void* drafter_workspace,
                                wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(verdict_dev != nullptr, "wc_verify_chain_greedy_fuse: verdict is NULL");
  WC_REQUIRE(rows == 1 || draft_tokens_dev != nullptr, "wc_verify_chain_greedy_fuse: draft tokens are NULL");
  WC_REQUIRE(logits != nullptr && vocab >= 1 && ld >= vocab, "wc_verify_chain_greedy_fuse: bad logits");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_STEP_ROWS, "wc_verify_chain_greedy_fuse: rows must be in 1..%d",
             WC_MAX_STEP_ROWS);
  WC_REQUIRE(verify_workspace != nullptr && aligned(verify_workspace, 16),
             "wc_verify_chain_greedy_fuse: verify workspace is NULL or not 16-byte aligned");
  GemvArgs a;
  if (int rc = fuse_gemv_args(dims, w, taps, tap_dtype, tap_ld, rows, g_out, g_ld, &a)) return rc;
  int gb = 0;
  for (int f = 0; f < a.n_in; ++f)
    if (a.in[f].gain) gb |= 1 << f;
  // one launch: two to eight rows (the few-row GEMV's range, which the fuse
  // launch uses for them too, so the fused rows round alike), three taps of
  // 2048 (one 512-wide step per wave, twelve waves), gains on every tap or
  // none, 16-byte logits rows, and CUs left beside the GEMV's blocks for
  // verify chunks of at most kVfBatches batches
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  const int ngemv = (dims->hidden + kVfGemvRows - 1) / kVfGemvRows;
  const int per_row = (cus - ngemv) / rows;
  int nvx = 0, chunk = 0;
  if (per_row >= 1) {
    chunk = ((vocab + per_row - 1) / per_row + kVfBatch - 1) / kVfBatch * kVfBatch;
    nvx = (vocab + chunk - 1) / chunk;
  }
  const bool one = nvx > 0 && chunk <= kVfBatches * kVfBatch && rows >= 2 && rows <= kVfRowsMax && dims->num_features == 3 &&
                   dims->target_hidden == 2048 && (gb == 0 || gb == 7) && aligned(logits, 16) && ld % 4 == 0;
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (!one) {
    if (int rc = wc_verify_chain_greedy(logits, rows, vocab, ld, draft_tokens_dev, verdict_dev, verify_workspace,
                                        stream))
      return rc;
    return wc_drafter_fuse(dims, w, taps, tap_dtype, tap_ld, nullptr, 0, rows, nullptr, g_out, g_ld,
                           drafter_workspace, stream);
  }
  VerifyFuseArgs v{};
  v.logits = logits;
  v.rows = rows;
  v.vocab = vocab;
  v.ld = ld;
  v.slots = static_cast<unsigned long long*>(verify_workspace);
  v.counter = verify_counter(verify_workspace, kCtrArgmax);
  v.drafts = draft_tokens_dev;
  v.verdict = verdict_dev;
  v.nvx = nvx;
  v.chunk = chunk;
  const dim3 grid(nvx * rows + ngemv);
  const bool bf = tap_dtype == WC_BF16;
  if (bf && gb)
    launch_vf<7, 7>(v, a, grid, s);
  else if (bf)
    launch_vf<7, 0>(v, a, grid, s);
  else if (gb)
    launch_vf<0, 7>(v, a, grid, s);
  else
    launch_vf<0, 0>(v, a, grid, s);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
