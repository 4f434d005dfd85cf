// argmax_verify.h -- the greedy verify's device code (target argmax fused with
// chain / tree acceptance): a block streams one chunk of one logits row, folds
// it into a packed (value, lowest index) key published by one device-scope
// atomicMax per row; the last block to finish runs the acceptance scan with
// wave-wide ballots and writes a wc_verdict, then clears the slots and its
// counter (graph-safe, no memset).  Shared by the verify launch and by the
// launch that runs the verify beside the drafter's fuse.
#pragma once

#include "wc_common.h"

namespace wc {

constexpr int kArgBlock = 256;
constexpr int kArgItems = 4;                            // float4 loads per thread
constexpr int kArgChunk = kArgBlock * 4 * kArgItems;    // 4096 logits per block
template <int NT>
constexpr int arg_chunk() { return NT * 4 * kArgItems; }  // logits per block of NT threads

enum VerifyMode { kModeArgmax = 0, kModeChain = 1, kModeTree = 2 };

template <bool VEC, int NT = kArgBlock>
__device__ __forceinline__ unsigned long long chunk_argmax(const float* __restrict__ row, int begin, int end) {
  unsigned long long best = 0;
  if (VEC) {
    float4 v[kArgItems];
    int idx[kArgItems];
#pragma unroll
    for (int j = 0; j < kArgItems; ++j) {
      idx[j] = begin + (j * NT + static_cast<int>(threadIdx.x)) * 4;
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
    for (int i = begin + static_cast<int>(threadIdx.x); i < end; i += NT) {
      const unsigned long long k = argmax_key(row[i], i);
      best = k > best ? k : best;
    }
  }
  return best;
}

// The acceptance scan of the last block's wave 0 (lane c owns row / node c,
// rows <= 64): reads and clears the per-row argmax slots, then writes the
// verdict of a chain (leading draft matches) or a tree (greedy path walk).
__device__ __forceinline__ void verify_finish(int lane, unsigned long long* __restrict__ slots, int rows, int mode,
                                              const int32_t* __restrict__ drafts,
                                              const int32_t* __restrict__ tree_tokens,
                                              const int32_t* __restrict__ tree_parents,
                                              int32_t* __restrict__ argmax_out, wc_verdict* __restrict__ verdict) {
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

// One (chunk bx, row r) block of NT threads among nblk (block index idx).
template <bool VEC, int NT>
__device__ __forceinline__ void argmax_verify_block(
    const float* __restrict__ logits, int rows, int vocab, int64_t ld, unsigned long long* __restrict__ slots,
    unsigned int* __restrict__ counter, int mode, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ tree_parents, int32_t* __restrict__ argmax_out,
    wc_verdict* __restrict__ verdict, int bx, int r, int idx, int nblk) {
  const int begin = bx * arg_chunk<NT>();
  const int end = min(vocab, begin + arg_chunk<NT>());
  unsigned long long best = chunk_argmax<VEC, NT>(logits + static_cast<int64_t>(r) * ld, begin, end);

  __shared__ unsigned long long s_part[NT / kWave];
  best = wave_max_u64(best);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_part[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NT / kWave; ++w) best = s_part[w] > best ? s_part[w] : best;
    atomic_max_u64(&slots[r], best);
  }
  if (!last_block_done(counter, nblk, idx)) return;
  if (wave != 0) return;
  verify_finish(lane, slots, rows, mode, drafts, tree_tokens, tree_parents, argmax_out, verdict);
}

template <bool VEC>
__global__ __launch_bounds__(kArgBlock) void k_argmax_verify(
    const float* __restrict__ logits, int rows, int vocab, int64_t ld, unsigned long long* __restrict__ slots,
    unsigned int* __restrict__ counter, int mode, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ tree_tokens, const int32_t* __restrict__ tree_parents, int32_t* __restrict__ argmax_out,
    wc_verdict* __restrict__ verdict) {
  argmax_verify_block<VEC, kArgBlock>(logits, rows, vocab, ld, slots, counter, mode, drafts, tree_tokens, tree_parents,
                                      argmax_out, verdict, blockIdx.x, blockIdx.y, linear_block(),
                                      gridDim.x * gridDim.y);
}

}  // namespace wc
