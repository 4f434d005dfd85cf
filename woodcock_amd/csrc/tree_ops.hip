// tree_ops.hip -- device-side helpers of tree drafting and verification.
//
// wc_tree_mask: the verify block's attention mask for a flattened draft tree
// (python/woodcock/sampling.py:118-128; src/sampling/sampling.cpp:85-93):
// row v sees the prefix slots [0, prefix) and its ancestors (itself included)
// at prefix + u.
//
// wc_sample_without_replacement: Gumbel-top-k over the nonzero entries of a
// draft distribution (python/woodcock/sampling.py:196-203): one uniform per
// nonzero entry in vocabulary order, key log q(x) - log(-log u), the k largest
// keys in descending order.  Rows consume the stream one after another (the
// reference draws every frontier node from one generator, spec.py:238-249).
#include "wc_common.h"

namespace wc {

// ------------------------------------------------------------------ tree mask

constexpr int kMaskThreads = 256;

// Block (row v, column range): prefix columns are 1; a tree column prefix + u
// is 1 when u lies on v's parent chain.  The chain is walked once per block
// into a 64-bit ancestor set (parents must satisfy parents[i] < i; the walk
// stops at the first parent that does not).
__global__ __launch_bounds__(kMaskThreads) void k_tree_mask(const int32_t* __restrict__ parents, int n, int prefix,
                                                           uint8_t* __restrict__ mask, int64_t ld) {
  __shared__ unsigned long long s_anc;
  const int v = blockIdx.y;
  if (threadIdx.x == 0) {
    unsigned long long anc = 0;
    int u = v;
    for (int step = 0; step < WC_MAX_NODES && u >= 0 && u < n; ++step) {
      anc |= 1ull << u;
      const int par = parents[u];
      if (par >= u) break;
      u = par;
    }
    s_anc = anc;
  }
  __syncthreads();
  const unsigned long long anc = s_anc;
  uint8_t* row = mask + static_cast<int64_t>(v) * ld;
  const int cols = prefix + n;
  for (int c = blockIdx.x * kMaskThreads + threadIdx.x; c < cols; c += gridDim.x * kMaskThreads)
    row[c] = c < prefix ? 1 : static_cast<uint8_t>((anc >> (c - prefix)) & 1ull);
}

// ------------------------------------------------------------------ Gumbel-top-k

constexpr int kGkThreads = 512;
constexpr int kGkMaxK = 16;  // draws per row

__global__ __launch_bounds__(kGkThreads) void k_gumbel_topk(const float* __restrict__ q, int rows, int head_rows,
                                                            int64_t ld_q, const int32_t* __restrict__ d2t,
                                                            const int32_t* __restrict__ k_dev, int k_max,
                                                            unsigned long long seed, const int32_t* round_dev,
                                                            int purpose, long long base, int32_t* __restrict__ out,
                                                            int32_t* __restrict__ counts) {
  __shared__ double red_d[kGkThreads / kWave];
  __shared__ int red_i[kGkThreads / kWave];
  __shared__ int s_scan[kGkThreads];
  __shared__ int s_win;
  const int t = threadIdx.x;
  const unsigned long long round = static_cast<unsigned long long>(*round_dev);
  const int per = (head_rows + kGkThreads - 1) / kGkThreads;  // consecutive entries per thread
  long long used = base;  // uniforms consumed before this row
  for (int r = 0; r < rows; ++r) {
    const float* qr = q + static_cast<int64_t>(r) * ld_q;
    const int r0 = min(t * per, head_rows), r1 = min(r0 + per, head_rows);
    // the row's mass (the reference renormalises q over the vocabulary)
    double ms = 0.0;
    int nz = 0;
    for (int i = r0; i < r1; ++i) {
      const float x = qr[i];
      ms += static_cast<double>(x);
      nz += x > 0.f ? 1 : 0;
    }
    ms = wave_sum(ms);
    if (t % kWave == 0) red_d[t / kWave] = ms;
    s_scan[t] = nz;
    __syncthreads();
    double Q = 0.0;
    for (int w = 0; w < kGkThreads / kWave; ++w) Q += red_d[w];
    if (t == 0) {  // exclusive scan of the per-thread nonzero counts, in vocabulary order
      int run = 0;
      for (int i = 0; i < kGkThreads; ++i) {
        const int c = s_scan[i];
        s_scan[i] = run;
        run += c;
      }
      red_i[0] = run;
    }
    __syncthreads();
    const int total_nz = red_i[0];
    int rank = s_scan[t];
    const int k = min(min(k_dev ? k_dev[r] : k_max, k_max), total_nz);
    // keys of this thread's entries, log q(x) - log(-log u) with u the entry's
    // uniform, kept as a descending list of the thread's kGkMaxK best
    double lk[kGkMaxK];
    int li[kGkMaxK];
#pragma unroll
    for (int e = 0; e < kGkMaxK; ++e) {
      lk[e] = -INFINITY;
      li[e] = 0x7fffffff;
    }
    for (int i = r0; i < r1; ++i) {
      const float x = qr[i];
      if (!(x > 0.f)) continue;
      const double u = philox_uniform(seed, round, purpose, static_cast<unsigned long long>(used + rank));
      ++rank;
      double kk = log(static_cast<double>(x) / Q) - log(-log(u));
      int ki = i;
      if (!(kk > lk[kGkMaxK - 1])) continue;
#pragma unroll
      for (int e = 0; e < kGkMaxK; ++e) {  // insert, keeping the list sorted (earlier index first on ties)
        if (kk > lk[e]) {
          const double tk = lk[e];
          const int ti = li[e];
          lk[e] = kk;
          li[e] = ki;
          kk = tk;
          ki = ti;
        }
      }
    }
    // k rounds of a block argmax over the list heads (largest key, then the lowest index)
    for (int sel = 0; sel < k; ++sel) {
      double bk = lk[0];
      int bi = li[0];
      for (int m = kWave / 2; m > 0; m >>= 1) {
        const double ok = __shfl_xor(bk, m);
        const int oi = __shfl_xor(bi, m);
        if (ok > bk || (ok == bk && oi < bi)) {
          bk = ok;
          bi = oi;
        }
      }
      __syncthreads();
      if (t % kWave == 0) {
        red_d[t / kWave] = bk;
        red_i[t / kWave] = bi;
      }
      __syncthreads();
      if (t == 0) {
        double wk = -INFINITY;
        int wi = 0x7fffffff;
        for (int w = 0; w < kGkThreads / kWave; ++w)
          if (red_d[w] > wk || (red_d[w] == wk && red_i[w] < wi)) {
            wk = red_d[w];
            wi = red_i[w];
          }
        s_win = wi;
        out[static_cast<int64_t>(r) * k_max + sel] = d2t ? d2t[wi] : wi;
      }
      __syncthreads();
      if (li[0] == s_win) {  // the winner pops its head
#pragma unroll
        for (int e = 0; e + 1 < kGkMaxK; ++e) {
          lk[e] = lk[e + 1];
          li[e] = li[e + 1];
        }
        lk[kGkMaxK - 1] = -INFINITY;
        li[kGkMaxK - 1] = 0x7fffffff;
      }
    }
    if (t == 0 && counts) counts[r] = k;
    used += total_nz;
    __syncthreads();
  }
}

}  // namespace wc

extern "C" {

int wc_tree_mask(const int32_t* parents_dev, int n, int prefix, uint8_t* mask_out, int64_t ld, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(parents_dev && mask_out, "wc_tree_mask: NULL buffer");
  WC_REQUIRE(n >= 1 && n <= WC_MAX_NODES, "wc_tree_mask: n must be in 1..%d (got %d)", WC_MAX_NODES, n);
  WC_REQUIRE(prefix >= 0 && ld >= static_cast<int64_t>(prefix) + n, "wc_tree_mask: row stride below prefix + n");
  const int cols = prefix + n;
  const int gx = std::max(1, std::min(64, (cols + kMaskThreads * 4 - 1) / (kMaskThreads * 4)));
  hipLaunchKernelGGL(k_tree_mask, dim3(gx, n), dim3(kMaskThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     parents_dev, n, prefix, mask_out, ld);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_sample_without_replacement(const float* q, int rows, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                                  const int32_t* k_dev, int k_max, const wc_uniforms* rng, int64_t uniform_base,
                                  int32_t* tokens_out, int32_t* counts_out, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(q && rng && rng->round_dev && tokens_out, "wc_sample_without_replacement: NULL buffer");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "wc_sample_without_replacement: rows must be in 1..%d",
             WC_MAX_NODES);
  WC_REQUIRE(head_rows >= 1 && ld_q >= head_rows,
             "wc_sample_without_replacement: head_rows must be positive with ld_q >= head_rows");
  WC_REQUIRE(k_max >= 1 && k_max <= kGkMaxK, "wc_sample_without_replacement: k_max must be in 1..%d", kGkMaxK);
  WC_REQUIRE(uniform_base >= 0, "wc_sample_without_replacement: negative uniform offset");
  hipLaunchKernelGGL(k_gumbel_topk, dim3(1), dim3(kGkThreads), 0, reinterpret_cast<hipStream_t>(stream), q, rows,
                     head_rows, ld_q, d2t_dev, k_dev, k_max, static_cast<unsigned long long>(rng->seed),
                     rng->round_dev, rng->purpose, static_cast<long long>(uniform_base), tokens_out, counts_out);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
