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
//
// Greedy tree drafting on the device (python/woodcock/spec.py:216-303 with
// StaticPolicy, python/woodcock/policies.py:49-75): a node table in a
// caller-owned state buffer, filled level by level without a host round trip.
//   wc_tree_draft_begin     node 0 = the root token;
//   wc_tree_draft_expand    the `width` most probable head rows of each
//                           frontier row's draft distribution become children
//                           (token = d2t[row], phat = phat(parent) * q), in
//                           descending q order, the lower head row first on a tie;
//   wc_tree_draft_frontier  the `width` level nodes of largest phat (ties: the
//                           earlier node) become the next frontier, with the
//                           drafter inputs of that forward: tokens, the rows of
//                           their parents' feedback, positions base - 1 + depth
//                           and the attention mask (the prefix within the
//                           window, the cache slots of the ancestors below the
//                           root, the node's own slot);
//   wc_tree_draft_select    the verified tree: every node, or the root plus the
//                           `budget` nodes of largest phat (ties: shallower,
//                           then earlier) in node order, parents remapped.
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

// ------------------------------------------------------------------ greedy tree drafting

constexpr int kTdMaxNodes = 512;
constexpr int kTdMaxWidth = 8;
constexpr int kTdThreads = 256;

constexpr int kTdParts = 16;  // blocks per frontier row in the expansion

struct TreeDraftState {
  double phat[kTdMaxNodes];
  int32_t token[kTdMaxNodes], parent[kTdMaxNodes], depth[kTdMaxNodes];
  int32_t slot[kTdMaxNodes];   // drafter cache slot once forwarded
  int32_t store[kTdMaxNodes];  // row of the node's out / feedback once forwarded (the root: 0)
  int32_t front[kTdMaxWidth];  // node ids of the current frontier, in frontier-row order
  // expansion: each part's top-width keys per frontier row, and a counter per
  // row (own 128-byte line; reset by the block that completes it)
  unsigned long long cand[kTdMaxWidth][kTdParts][kTdMaxWidth];
  unsigned int ctr[kTdMaxWidth][32];
};

__global__ void k_td_begin(TreeDraftState* st, const int32_t* __restrict__ root_token) {
  if (threadIdx.x == 0) {
    st->token[0] = *root_token;
    st->parent[0] = -1;
    st->depth[0] = 0;
    st->phat[0] = 1.0;
    st->slot[0] = -1;
    st->store[0] = 0;
    st->front[0] = 0;
  }
}

// Largest key over the block (every thread receives it).
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* red) {
  v = wave_max_u64(v);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  unsigned long long b = 0;
#pragma unroll
  for (int w = 0; w < kTdThreads / kWave; ++w) b = red[w] > b ? red[w] : b;
  return b;
}

// Block r: the `width` largest (q, lowest row first) entries of q row r.  Each
// thread keeps a sorted top-width list of its share of the row, read as
// 16-byte vectors kTdVec at a time (all loads of a pass issued before the
// first insert); `width` block-wide maxima then pop the winners in order.
constexpr int kTdVec = 8;
__global__ __launch_bounds__(kTdThreads) void k_td_expand(TreeDraftState* st, const float* __restrict__ q,
                                                          int head_rows, int64_t ld_q,
                                                          const int32_t* __restrict__ d2t, int width,
                                                          int node_base) {
  __shared__ unsigned long long red[kTdThreads / kWave];
  __shared__ bool s_last;
  const int r = blockIdx.x, p = blockIdx.y, P = gridDim.y, t = threadIdx.x;
  const float* qr = q + static_cast<int64_t>(r) * ld_q;
  // part p: the rows [i0, i1) of the head (a multiple of 4 long, so aligned rows stay aligned)
  const int span = ((head_rows + P - 1) / P + 3) & ~3;
  const int i0 = min(p * span, head_rows), i1 = min(i0 + span, head_rows);
  unsigned long long top[kTdMaxWidth];
#pragma unroll
  for (int j = 0; j < kTdMaxWidth; ++j) top[j] = 0;
  auto insert = [&](float v, int i) {
    unsigned long long k = argmax_key(v, i);
#pragma unroll
    for (int j = 0; j < kTdMaxWidth; ++j) {
      const bool take = j < width && k > top[j];
      const unsigned long long o = top[j];
      top[j] = take ? k : o;
      k = take ? o : k;
    }
  };
  // 16-byte vectors where the row is 16-byte aligned, the tail (and unaligned rows) element-wise
  const bool al = (reinterpret_cast<uintptr_t>(qr) & 15) == 0;
  const int b4 = i0 / 4, e4 = al ? i1 / 4 : b4;
  const float4* q4 = reinterpret_cast<const float4*>(qr);
  for (int b = b4; b < e4; b += kTdThreads * kTdVec) {
    float4 v[kTdVec];
#pragma unroll
    for (int u = 0; u < kTdVec; ++u) v[u] = q4[min(b + u * kTdThreads + t, e4 - 1)];
#pragma unroll
    for (int u = 0; u < kTdVec; ++u) {
      const int i4 = b + u * kTdThreads + t;
      if (i4 < e4) {
        insert(v[u].x, 4 * i4);
        insert(v[u].y, 4 * i4 + 1);
        insert(v[u].z, 4 * i4 + 2);
        insert(v[u].w, 4 * i4 + 3);
      }
    }
  }
  for (int i = 4 * e4 + t; i < i1; i += kTdThreads) insert(qr[i], i);
  // the part's top keys, largest first (keys are unique: the row is in the key)
  for (int j = 0; j < width; ++j) {
    const unsigned long long best = block_max_u64(top[0], red);
    if (best != 0 && top[0] == best) {
#pragma unroll
      for (int i = 0; i + 1 < kTdMaxWidth; ++i) top[i] = top[i + 1];
      top[kTdMaxWidth - 1] = 0;
    }
    if (t == 0) atomic_store_u64(&st->cand[r][p][j], best);
  }
  // the last part of the row to finish merges every part's keys
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const bool last = __hip_atomic_fetch_add(&st->ctr[r][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      static_cast<unsigned int>(P - 1);
    if (last) __hip_atomic_store(&st->ctr[r][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  unsigned long long k = t < P * width ? atomic_load_u64(&st->cand[r][t / width][t % width]) : 0ull;
  const int v = st->front[r];
  for (int j = 0; j < width; ++j) {
    const unsigned long long best = block_max_u64(k, red);
    if (best != 0 && k == best) k = 0;
    if (t == 0) {
      const int row = argmax_key_index(best);
      const int c = node_base + r * width + j;
      st->token[c] = d2t ? d2t[row] : row;
      st->parent[c] = v;
      st->depth[c] = st->depth[v] + 1;
      st->phat[c] = st->phat[v] * static_cast<double>(qr[row]);
      st->slot[c] = -1;
      st->store[c] = -1;
    }
  }
}

// One block: next frontier among the level's nodes [lb, le) and the inputs of
// its drafter forward.
__global__ __launch_bounds__(kTdThreads) void k_td_frontier(TreeDraftState* st, int lb, int le, int width,
                                                            const int32_t* __restrict__ offset_dev, int tree_cache,
                                                            int window, int store_base, int32_t* __restrict__ tokens,
                                                            int32_t* __restrict__ feat_rows,
                                                            int32_t* __restrict__ positions,
                                                            uint8_t* __restrict__ mask, int64_t mask_ld) {
  __shared__ int s_front[kTdMaxWidth];
  __shared__ int s_anc[kTdMaxWidth][kTdMaxNodes / kTdMaxWidth];
  __shared__ int s_nanc[kTdMaxWidth];
  __shared__ double s_ph[kTdMaxNodes];
  const int t = threadIdx.x;
  const int n = le - lb, m = min(width, n);
  for (int i = t; i < n; i += kTdThreads) s_ph[i] = st->phat[lb + i];
  __syncthreads();
  for (int i = t; i < n; i += kTdThreads) {
    const double ph = s_ph[i];
    int rank = 0;
    for (int u = 0; u < n; ++u) {
      const double pu = s_ph[u];
      rank += (pu > ph || (pu == ph && u < i)) ? 1 : 0;
    }
    if (rank < m) s_front[rank] = lb + i;
  }
  __syncthreads();
  const int base = *offset_dev;
  if (t < m) {
    const int v = s_front[t];
    st->front[t] = v;
    tokens[t] = st->token[v];
    feat_rows[t] = st->store[st->parent[v]];
    positions[t] = base - 1 + st->depth[v];
    st->slot[v] = base + tree_cache + t;
    st->store[v] = store_base + t;
    // cache slots of the ancestors below the root
    int na = 0;
    for (int u = st->parent[v]; u > 0 && na < kTdMaxNodes / kTdMaxWidth; u = st->parent[u]) s_anc[t][na++] = st->slot[u];
    s_nanc[t] = na;
  }
  __syncthreads();
  for (int r = 0; r < m; ++r) {
    const int v = s_front[r];
    const int pos = base - 1 + st->depth[v];
    const int lo = window > 0 ? max(0, pos - window + 1) : 0;
    const int self = base + tree_cache + r, na = s_nanc[r];
    uint8_t* row = mask + static_cast<int64_t>(r) * mask_ld;
    for (int64_t c = t; c < mask_ld; c += kTdThreads) {
      bool on = (c >= lo && c < base) || c == self;
      for (int k = 0; k < na; ++k) on = on || c == s_anc[r][k];
      row[c] = on ? 1 : 0;
    }
  }
}

// One block: the verified subset in node order with parents remapped.
__global__ __launch_bounds__(kTdThreads) void k_td_select(const TreeDraftState* st, int n_nodes, int budget,
                                                          int32_t* __restrict__ tokens, int32_t* __restrict__ parents,
                                                          int32_t* __restrict__ depth, int32_t* __restrict__ count) {
  __shared__ int s_pos[kTdMaxNodes];
  __shared__ double s_ph[kTdMaxNodes];
  __shared__ int s_dep[kTdMaxNodes];
  const int t = threadIdx.x;
  const bool all = n_nodes - 1 <= budget;
  for (int v = t; v < n_nodes; v += kTdThreads) {
    s_ph[v] = st->phat[v];
    s_dep[v] = st->depth[v];
  }
  __syncthreads();
  for (int v = t; v < n_nodes; v += kTdThreads) {
    bool keep = v == 0 || all;
    if (!keep) {
      const double ph = s_ph[v];
      const int dv = s_dep[v];
      int rank = 0;
      for (int u = 1; u < n_nodes; ++u) {
        const double pu = s_ph[u];
        const int du = s_dep[u];
        rank += (pu > ph || (pu == ph && (du < dv || (du == dv && u < v)))) ? 1 : 0;
      }
      keep = rank < budget;
    }
    s_pos[v] = keep ? 1 : 0;
  }
  __syncthreads();
  if (t == 0) {  // exclusive scan; -1 marks a dropped node
    int k = 0;
    for (int v = 0; v < n_nodes; ++v) {
      const int kept = s_pos[v];
      s_pos[v] = kept ? k : -1;
      k += kept;
    }
    *count = k;
  }
  __syncthreads();
  for (int v = t; v < n_nodes; v += kTdThreads) {
    const int i = s_pos[v];
    if (i < 0) continue;
    const int p = st->parent[v];
    tokens[i] = st->token[v];
    depth[i] = st->depth[v];
    parents[i] = p < 0 ? -1 : s_pos[p];
  }
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

size_t wc_tree_draft_state_bytes(void) { return sizeof(wc::TreeDraftState); }

int wc_tree_draft_begin(void* state, const int32_t* root_token_dev, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && root_token_dev, "wc_tree_draft_begin: NULL buffer");
  hipLaunchKernelGGL(k_td_begin, dim3(1), dim3(kWave), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<TreeDraftState*>(state), root_token_dev);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_expand(void* state, const float* q, int rows, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                         int width, int node_base, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && q, "wc_tree_draft_expand: NULL buffer");
  WC_REQUIRE(width >= 1 && width <= kTdMaxWidth, "wc_tree_draft_expand: width must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(rows >= 1 && rows <= kTdMaxWidth, "wc_tree_draft_expand: rows must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(head_rows >= width && ld_q >= head_rows, "wc_tree_draft_expand: need head_rows >= width, ld_q >= head_rows");
  WC_REQUIRE(node_base >= 1 && node_base + rows * width <= kTdMaxNodes,
             "wc_tree_draft_expand: nodes %d..%d outside the table of %d", node_base, node_base + rows * width,
             kTdMaxNodes);
  // parts of at least 1024 head rows each, at most kTdParts per frontier row
  const int parts = std::max(1, std::min(kTdParts, head_rows / 1024));
  hipLaunchKernelGGL(k_td_expand, dim3(rows, parts), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<TreeDraftState*>(state), q, head_rows, ld_q, d2t_dev, width, node_base);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_frontier(void* state, int level_begin, int level_end, int width, const int32_t* offset_dev,
                           int tree_cache, int window, int store_base, int32_t* tokens_out, int32_t* feat_rows_out,
                           int32_t* positions_out, uint8_t* mask_out, int64_t mask_ld, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && offset_dev && tokens_out && feat_rows_out && positions_out && mask_out,
             "wc_tree_draft_frontier: NULL buffer");
  WC_REQUIRE(width >= 1 && width <= kTdMaxWidth, "wc_tree_draft_frontier: width must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(level_begin >= 1 && level_end > level_begin && level_end <= kTdMaxNodes,
             "wc_tree_draft_frontier: bad level range %d..%d", level_begin, level_end);
  WC_REQUIRE(tree_cache >= 0 && store_base >= 1 && mask_ld >= 1, "wc_tree_draft_frontier: bad offsets");
  hipLaunchKernelGGL(k_td_frontier, dim3(1), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<TreeDraftState*>(state), level_begin, level_end, width, offset_dev, tree_cache,
                     window, store_base, tokens_out, feat_rows_out, positions_out, mask_out, mask_ld);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_select(const void* state, int n_nodes, int budget, int32_t* tokens_out, int32_t* parents_out,
                         int32_t* depth_out, int32_t* count_out, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && tokens_out && parents_out && depth_out && count_out, "wc_tree_draft_select: NULL buffer");
  WC_REQUIRE(n_nodes >= 1 && n_nodes <= kTdMaxNodes, "wc_tree_draft_select: n_nodes must be in 1..%d", kTdMaxNodes);
  WC_REQUIRE(budget >= 0, "wc_tree_draft_select: negative budget");
  hipLaunchKernelGGL(k_td_select, dim3(1), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const TreeDraftState*>(state), n_nodes, budget, tokens_out, parents_out, depth_out,
                     count_out);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
