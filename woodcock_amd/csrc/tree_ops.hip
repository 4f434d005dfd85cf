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
// Sampled drafting at T > 0 (spec.py:238-249; policies.py:25-36) shares the
// table: wc_tree_draft_expand_sample draws each frontier row's children
// without replacement (their number fixed before drawing, within the budget)
// and appends them; wc_tree_draft_frontier then takes the level range from the
// state; wc_tree_draft_select_all returns every node with the row of its draft
// distribution.  Node counts are data-dependent there (a row with fewer nonzero
// entries than draws yields fewer children), so they live in the state and the
// host's launch shapes are upper bounds.
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
  // sampled drafting (T > 0): the table's node count, the last expansion's
  // node range, the current frontier's row count and the draws granted so far
  // (Plan.children_for)
  int32_t n_nodes, lvl_begin, lvl_end, n_front, granted, pad_[3];
  // per frontier row and part: the part's best keys (fp64 bits), their head
  // rows and the part's q mass; per row: the drawn children (token, phat bits)
  // and their number; the level's completion counter (own 128-byte line)
  unsigned long long skey[kTdMaxWidth][kTdParts][kTdMaxWidth];
  unsigned int srow[kTdMaxWidth][kTdParts][kTdMaxWidth];
  unsigned long long smass[kTdMaxWidth][kTdParts];
  unsigned int stok[kTdMaxWidth][kTdMaxWidth];
  unsigned long long sphat[kTdMaxWidth][kTdMaxWidth];
  unsigned int scount[kTdMaxWidth];
  unsigned int lvl_ctr[32];
  // greedy expansion from the logits: per frontier row and part, the part's
  // maximum and its sum of exp(z - maximum) (two fp32 bit patterns)
  unsigned long long zstat[kTdMaxWidth][kTdParts];
};

__device__ __forceinline__ unsigned int atomic_load_u32(const unsigned int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_td_begin(TreeDraftState* st, const int32_t* __restrict__ root_token) {
  if (threadIdx.x == 0) {
    st->token[0] = *root_token;
    st->parent[0] = -1;
    st->depth[0] = 0;
    st->phat[0] = 1.0;
    st->slot[0] = -1;
    st->store[0] = 0;
    st->front[0] = 0;
    st->n_nodes = 1;
    st->lvl_begin = 0;
    st->lvl_end = 1;
    st->n_front = 1;
    st->granted = 0;
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
// LOGITS: the row holds the head logits z and q = softmax(z) (T = 1) is never
// written: softmax is monotone, so the top-width of q are the top-width of z
// (same tie rule), and a child's q = exp(z - M) / S comes from the row's
// maximum M and sum S = sum_p S_p exp(m_p - M), combined in part order by the
// last part from each part's maximum m_p and sum S_p of exp(z - m_p).  The
// exponential and the in-part sums follow k_softmax_row (expf; lane sums, the
// wave sums, then the waves in order): only the association of the row sum
// differs, a few ulps of q.
constexpr int kTdVec = 8;
template <bool LOGITS>
__global__ __launch_bounds__(kTdThreads) void k_td_expand(TreeDraftState* st, const float* __restrict__ q,
                                                          int head_rows, int64_t ld_q,
                                                          const int32_t* __restrict__ d2t, int width,
                                                          int node_base) {
  __shared__ unsigned long long red[kTdThreads / kWave];
  __shared__ float s_f[kTdThreads / kWave];
  __shared__ float s_row[2];
  __shared__ bool s_last;
  const int r = blockIdx.x, p = blockIdx.y, P = gridDim.y, t = threadIdx.x;
  const float* qr = q + static_cast<int64_t>(r) * ld_q;
  // part p: the rows [i0, i1) of the head (a multiple of 4 long, so aligned rows stay aligned)
  const int span = ((head_rows + P - 1) / P + 3) & ~3;
  const int i0 = min(p * span, head_rows), i1 = min(i0 + span, head_rows);
  unsigned long long top[kTdMaxWidth];
#pragma unroll
  for (int j = 0; j < kTdMaxWidth; ++j) top[j] = 0;
  float mloc = -INFINITY;  // LOGITS: this thread's maximum
  auto insert = [&](float v, int i) {
    if constexpr (LOGITS) mloc = fmaxf(mloc, v);
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
  if constexpr (LOGITS) {
    // the part's maximum, then its sum of exp(z - maximum) over a second pass
    // of the part (L2-resident after the first; a single pass with running
    // sums rescaled at each new maximum measured slower)
    const int lane = t % kWave, wave = t / kWave;
    const float mw = wave_max_dpp(mloc);
    if (lane == 0) s_f[wave] = mw;
    __syncthreads();
    float mp = s_f[0];
#pragma unroll
    for (int w = 1; w < kTdThreads / kWave; ++w) mp = fmaxf(mp, s_f[w]);
    __syncthreads();
    float sl = 0.f;
    for (int i = i0 + t; i < i1; i += kTdThreads) {
      const float v = qr[i];
      sl += v == -INFINITY ? 0.f : expf(v - mp);
    }
    sl = wave_sum_dpp(sl);
    if (lane == 0) s_f[wave] = sl;
    __syncthreads();
    float sp = 0.f;
#pragma unroll
    for (int w = 0; w < kTdThreads / kWave; ++w) sp += s_f[w];
    if (t == 0)
      atomic_store_u64(&st->zstat[r][p], (static_cast<unsigned long long>(__float_as_uint(mp)) << 32) |
                                             static_cast<unsigned long long>(__float_as_uint(sp)));
  }
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
  if constexpr (LOGITS) {
    if (t == 0) {
      float mp[kTdParts], sp[kTdParts], M = -INFINITY;
      for (int j = 0; j < P; ++j) {
        const unsigned long long w = atomic_load_u64(&st->zstat[r][j]);
        mp[j] = __uint_as_float(static_cast<uint32_t>(w >> 32));
        sp[j] = __uint_as_float(static_cast<uint32_t>(w & 0xffffffffu));
        M = fmaxf(M, mp[j]);
      }
      float S = 0.f;
      for (int j = 0; j < P; ++j) S += sp[j] == 0.f ? 0.f : sp[j] * expf(mp[j] - M);
      s_row[0] = M;
      s_row[1] = S;
    }
    __syncthreads();
  }
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
      const float qc = LOGITS ? expf(qr[row] - s_row[0]) / s_row[1] : qr[row];
      st->phat[c] = st->phat[v] * static_cast<double>(qc);
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
  __shared__ int s_nanc[kTdMaxWidth], s_pos[kTdMaxWidth];
  __shared__ double s_ph[kTdMaxNodes];
  const int t = threadIdx.x;
  // level_begin 0: the level the last sampled expansion appended (its range is
  // in the state); rows [m, width) then get inputs of a harmless padding row
  const bool dyn = lb == 0;
  if (dyn) {
    lb = st->lvl_begin;
    le = st->lvl_end;
  }
  const int n = min(max(le - lb, 0), kTdMaxNodes), m = min(width, n);
  const int rows = dyn ? width : m;
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
  if (t == 0) st->n_front = m;
  if (t < m) {
    const int v = s_front[t];
    st->front[t] = v;
    tokens[t] = st->token[v];
    feat_rows[t] = st->store[st->parent[v]];
    s_pos[t] = positions[t] = base - 1 + st->depth[v];
    st->slot[v] = base + tree_cache + t;
    st->store[v] = store_base + t;
    // cache slots of the ancestors below the root
    int na = 0;
    for (int u = st->parent[v]; u > 0 && na < kTdMaxNodes / kTdMaxWidth; u = st->parent[u]) s_anc[t][na++] = st->slot[u];
    s_nanc[t] = na;
  } else if (t < rows) {  // padding: the root token on the root's feedback at depth 1, seeing the prefix and itself
    tokens[t] = st->token[0];
    feat_rows[t] = 0;
    s_pos[t] = positions[t] = base;
    s_nanc[t] = 0;
  }
  __syncthreads();
  for (int r = 0; r < rows; ++r) {
    const int pos = s_pos[r];
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
  __shared__ int s_grp[kTdMaxNodes / kWave];  // kept nodes per 64-node group
  const int t = threadIdx.x, lane = t % kWave;
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
  // exclusive scan of the keep flags in node order, -1 marking a dropped node:
  // within each 64-node group from the wave's ballot, then the groups' counts
  int flag[kTdMaxNodes / kTdThreads], below[kTdMaxNodes / kTdThreads];
#pragma unroll
  for (int j = 0; j < kTdMaxNodes / kTdThreads; ++j) {
    const int v = t + j * kTdThreads;
    flag[j] = v < n_nodes ? s_pos[v] : 0;
    const unsigned long long b = __ballot(flag[j] != 0);
    below[j] = __popcll(b & ((1ull << lane) - 1ull));
    if (lane == 0) s_grp[v / kWave] = __popcll(b);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kTdMaxNodes / kTdThreads; ++j) {
    const int v = t + j * kTdThreads;
    int off = 0;
    for (int g = 0; g < v / kWave; ++g) off += s_grp[g];
    if (v < n_nodes) s_pos[v] = flag[j] ? off + below[j] : -1;
  }
  if (t == 0) {
    int k = 0;
    for (int g = 0; g < kTdMaxNodes / kWave; ++g) k += s_grp[g];
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

// ------------------------------------------------------------------ sampled tree drafting (T > 0)

// (key, head row) order of the draws: the larger key first, the lower row on a tie.
__device__ __forceinline__ bool key_before(double ka, int ia, double kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// The best (key, row) over the block; every thread receives it.
__device__ __forceinline__ void block_best_key(double& k, int& i, double* red_k, int* red_i) {
  for (int s = kWave / 2; s > 0; s >>= 1) {
    const double ok = __shfl_xor(k, s);
    const int oi = __shfl_xor(i, s);
    if (key_before(ok, oi, k, i)) {
      k = ok;
      i = oi;
    }
  }
  __syncthreads();
  if (threadIdx.x % kWave == 0) {
    red_k[threadIdx.x / kWave] = k;
    red_i[threadIdx.x / kWave] = i;
  }
  __syncthreads();
  k = red_k[0];
  i = red_i[0];
  for (int w = 1; w < kTdThreads / kWave; ++w)
    if (key_before(red_k[w], red_i[w], k, i)) {
      k = red_k[w];
      i = red_i[w];
    }
}

constexpr int kNoRow = 0x7fffffff;

// Block (r, p): part p of frontier row r (rows past the state's frontier count
// return at once).  Row r's draw count m = min(width, budget left after the
// rows before it) is fixed before drawing (Plan.children_for,
// policies.py:32-36).  Every nonzero entry i gets the key
// log q(i) - log(-log u), u = value v * H4 + i of the drafting stream (v the
// frontier node, H4 = head_rows rounded up to 4), and the m largest keys are the
// children in descending key order: Gumbel-top-k = m draws without replacement
// (sampling.py:196-203; spec.py:238-249).  Each entry owns its uniform, so all
// rows and parts draw at once.  The part's best m keys and its q mass go to
// the row's last part, which keeps the best m overall with
// phat = phat(parent) * q(i) / sum(q); the last row to finish appends every
// row's children to the node table in frontier order.
__global__ __launch_bounds__(kTdThreads) void k_td_sample(TreeDraftState* st, const float* __restrict__ q,
                                                          int head_rows, int64_t ld_q,
                                                          const int32_t* __restrict__ d2t, int width, int budget,
                                                          unsigned long long seed, const int32_t* __restrict__ round_dev,
                                                          int purpose) {
  __shared__ double red_k[kTdThreads / kWave];
  __shared__ int red_i[kTdThreads / kWave];
  __shared__ double red_m[kTdThreads / kWave];
  __shared__ bool s_last;
  const int r = blockIdx.x, p = blockIdx.y, P = gridDim.y, t = threadIdx.x;
  const int nf = min(st->n_front, static_cast<int>(gridDim.x));
  if (nf <= 0) {  // an empty frontier: the level is empty
    if (r == 0 && p == 0 && t == 0) {
      st->lvl_begin = st->n_nodes;
      st->lvl_end = st->n_nodes;
    }
    return;
  }
  if (r >= nf) return;
  const int rem = max(0, budget - st->granted);
  const int m = min(width, max(0, rem - r * width));
  const int v = st->front[r];
  const float* qr = q + static_cast<int64_t>(r) * ld_q;
  const int span = ((head_rows + P - 1) / P + 3) & ~3;
  const int i0 = min(p * span, head_rows), i1 = min(i0 + span, head_rows);
  const unsigned long long round = static_cast<unsigned long long>(*round_dev);
  const unsigned long long ubase =
      static_cast<unsigned long long>(v) * static_cast<unsigned long long>((head_rows + 3) & ~3);
  double lk[kTdMaxWidth];
  int li[kTdMaxWidth];
#pragma unroll
  for (int e = 0; e < kTdMaxWidth; ++e) {
    lk[e] = -INFINITY;
    li[e] = kNoRow;
  }
  double mass = 0.0;
  if (m > 0) {
    // four consecutive entries per thread share one Philox block (i0 is a multiple of 4)
    for (int g = i0 + 4 * t; g < i1; g += 4 * kTdThreads) {
      unsigned long long c[4] = {(ubase + static_cast<unsigned long long>(g)) >> 2, round,
                                 static_cast<unsigned long long>(purpose), 0ull};
      philox4x64(c, seed, 0ull);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = g + e;
        if (i >= i1) break;
        const float x = qr[i];
        mass += static_cast<double>(x);
        if (!(x > 0.f)) continue;
        const double u = static_cast<double>(c[e] >> 11) * (1.0 / 9007199254740992.0);
        double kk = log(static_cast<double>(x)) - log(-log(u));
        int ki = i;
#pragma unroll
        for (int j = 0; j < kTdMaxWidth; ++j) {  // sorted insert into the thread's best list
          const bool take = j < m && key_before(kk, ki, lk[j], li[j]);
          const double tk = lk[j];
          const int ti = li[j];
          lk[j] = take ? kk : tk;
          li[j] = take ? ki : ti;
          kk = take ? tk : kk;
          ki = take ? ti : ki;
        }
      }
    }
  }
  // the part's best m, popped from the list heads in order
  for (int sel = 0; sel < m; ++sel) {
    double bk = lk[0];
    int bi = li[0];
    block_best_key(bk, bi, red_k, red_i);
    if (t == 0) {
      atomic_store_u64(&st->skey[r][p][sel], static_cast<unsigned long long>(__double_as_longlong(bk)));
      atomic_store_u32(&st->srow[r][p][sel], static_cast<unsigned int>(bi));
    }
    if (bi != kNoRow && li[0] == bi) {
#pragma unroll
      for (int e = 0; e + 1 < kTdMaxWidth; ++e) {
        lk[e] = lk[e + 1];
        li[e] = li[e + 1];
      }
      lk[kTdMaxWidth - 1] = -INFINITY;
      li[kTdMaxWidth - 1] = kNoRow;
    }
  }
  mass = wave_sum(mass);
  __syncthreads();
  if (t % kWave == 0) red_m[t / kWave] = mass;
  __syncthreads();
  if (t == 0) {
    double ms = 0.0;
    for (int w = 0; w < kTdThreads / kWave; ++w) ms += red_m[w];
    atomic_store_u64(&st->smass[r][p], static_cast<unsigned long long>(__double_as_longlong(ms)));
  }
  // the row's last part merges the parts' candidates
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
  double ck = -INFINITY;
  int ci = kNoRow;
  if (t < P * m) {
    ck = __longlong_as_double(static_cast<long long>(atomic_load_u64(&st->skey[r][t / m][t % m])));
    ci = static_cast<int>(atomic_load_u32(&st->srow[r][t / m][t % m]));
  }
  double Q = 0.0;  // the row's q mass, parts summed in order
  for (int pp = 0; pp < P; ++pp)
    Q += __longlong_as_double(static_cast<long long>(atomic_load_u64(&st->smass[r][pp])));
  const double ph = st->phat[v];
  int cnt = 0;
  for (int sel = 0; sel < m; ++sel) {
    double bk = ck;
    int bi = ci;
    block_best_key(bk, bi, red_k, red_i);
    if (bi == kNoRow) break;  // fewer nonzero entries than draws
    if (t == 0) {
      atomic_store_u32(&st->stok[r][sel], static_cast<unsigned int>(d2t ? d2t[bi] : bi));
      const double phc = ph * (static_cast<double>(qr[bi]) / Q);
      atomic_store_u64(&st->sphat[r][sel], static_cast<unsigned long long>(__double_as_longlong(phc)));
    }
    if (ci == bi) {
      ck = -INFINITY;
      ci = kNoRow;
    }
    ++cnt;
  }
  if (t == 0) atomic_store_u32(&st->scount[r], static_cast<unsigned int>(cnt));
  // the last row appends the level
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const bool last = __hip_atomic_fetch_add(&st->lvl_ctr[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      static_cast<unsigned int>(nf - 1);
    if (last) __hip_atomic_store(&st->lvl_ctr[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last || t != 0) return;
  int c = st->n_nodes;
  const int begin = c;
  int granted = 0;
  for (int rr = 0; rr < nf; ++rr) {
    const int vv = st->front[rr];
    granted += min(width, max(0, rem - rr * width));
    const int cr = static_cast<int>(atomic_load_u32(&st->scount[rr]));
    for (int j = 0; j < cr && c < kTdMaxNodes; ++j, ++c) {
      st->token[c] = static_cast<int32_t>(atomic_load_u32(&st->stok[rr][j]));
      st->parent[c] = vv;
      st->depth[c] = st->depth[vv] + 1;
      st->phat[c] = __longlong_as_double(static_cast<long long>(atomic_load_u64(&st->sphat[rr][j])));
      st->slot[c] = -1;
      st->store[c] = -1;
    }
  }
  st->lvl_begin = begin;
  st->lvl_end = c;
  st->n_nodes = c;
  st->granted += granted;
}

// One block: every node of a sampled tree (StaticPolicy.select_verify keeps all
// of them at T > 0, policies.py:67-69) in node order, with the row of each
// node's draft distribution (its feedback-store row; 0 for nodes never
// expanded), padded to max_nodes rows with root-token children of the root.
__global__ __launch_bounds__(kTdThreads) void k_td_select_all(const TreeDraftState* st, int max_nodes,
                                                              int32_t* __restrict__ tokens,
                                                              int32_t* __restrict__ parents,
                                                              int32_t* __restrict__ depth,
                                                              int32_t* __restrict__ q_rows,
                                                              int32_t* __restrict__ count) {
  const int n = min(st->n_nodes, max_nodes);
  for (int v = threadIdx.x; v < max_nodes; v += kTdThreads) {
    if (v < n) {
      tokens[v] = st->token[v];
      parents[v] = st->parent[v];
      depth[v] = st->depth[v];
      q_rows[v] = max(st->store[v], 0);
    } else {
      tokens[v] = st->token[0];
      parents[v] = 0;
      depth[v] = 1;
      q_rows[v] = 0;
    }
  }
  if (threadIdx.x == 0) *count = n;
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
  hipLaunchKernelGGL(k_td_expand<false>, dim3(rows, parts), dim3(kTdThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<TreeDraftState*>(state), q, head_rows, ld_q,
                     d2t_dev, width, node_base);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_expand_logits(void* state, const float* logits, int rows, int head_rows, int64_t ld,
                                const int32_t* d2t_dev, int width, int node_base, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && logits, "wc_tree_draft_expand_logits: NULL buffer");
  WC_REQUIRE(width >= 1 && width <= kTdMaxWidth, "wc_tree_draft_expand_logits: width must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(rows >= 1 && rows <= kTdMaxWidth, "wc_tree_draft_expand_logits: rows must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(head_rows >= width && ld >= head_rows,
             "wc_tree_draft_expand_logits: need head_rows >= width, ld >= head_rows");
  WC_REQUIRE(node_base >= 1 && node_base + rows * width <= kTdMaxNodes,
             "wc_tree_draft_expand_logits: nodes %d..%d outside the table of %d", node_base, node_base + rows * width,
             kTdMaxNodes);
  const int parts = std::max(1, std::min(kTdParts, head_rows / 1024));
  hipLaunchKernelGGL(k_td_expand<true>, dim3(rows, parts), dim3(kTdThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<TreeDraftState*>(state), logits, head_rows, ld,
                     d2t_dev, width, node_base);
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
  WC_REQUIRE(level_begin == 0 || (level_begin >= 1 && level_end > level_begin && level_end <= kTdMaxNodes),
             "wc_tree_draft_frontier: bad level range %d..%d", level_begin, level_end);
  WC_REQUIRE(tree_cache >= 0 && store_base >= 1 && mask_ld >= 1, "wc_tree_draft_frontier: bad offsets");
  hipLaunchKernelGGL(k_td_frontier, dim3(1), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<TreeDraftState*>(state), level_begin, level_end, width, offset_dev, tree_cache,
                     window, store_base, tokens_out, feat_rows_out, positions_out, mask_out, mask_ld);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_expand_sample(void* state, const float* q, int rows, int head_rows, int64_t ld_q,
                                const int32_t* d2t_dev, int width, int budget, const wc_uniforms* rng,
                                wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && q && rng && rng->round_dev, "wc_tree_draft_expand_sample: NULL buffer");
  WC_REQUIRE(width >= 1 && width <= kTdMaxWidth, "wc_tree_draft_expand_sample: width must be in 1..%d",
             kTdMaxWidth);
  WC_REQUIRE(rows >= 1 && rows <= kTdMaxWidth, "wc_tree_draft_expand_sample: rows must be in 1..%d", kTdMaxWidth);
  WC_REQUIRE(head_rows >= 1 && ld_q >= head_rows, "wc_tree_draft_expand_sample: need head_rows >= 1, ld_q >= head_rows");
  WC_REQUIRE(budget >= 0 && budget < kTdMaxNodes, "wc_tree_draft_expand_sample: budget must be in 0..%d",
             kTdMaxNodes - 1);
  const int parts = std::max(1, std::min(kTdParts, head_rows / 1024));
  hipLaunchKernelGGL(k_td_sample, dim3(rows, parts), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<TreeDraftState*>(state), q, head_rows, ld_q, d2t_dev, width, budget,
                     static_cast<unsigned long long>(rng->seed), rng->round_dev, rng->purpose);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_tree_draft_select_all(const void* state, int max_nodes, int32_t* tokens_out, int32_t* parents_out,
                             int32_t* depth_out, int32_t* q_rows_out, int32_t* count_out, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(state && tokens_out && parents_out && depth_out && q_rows_out && count_out,
             "wc_tree_draft_select_all: NULL buffer");
  WC_REQUIRE(max_nodes >= 1 && max_nodes <= kTdMaxNodes, "wc_tree_draft_select_all: max_nodes must be in 1..%d",
             kTdMaxNodes);
  hipLaunchKernelGGL(k_td_select_all, dim3(1), dim3(kTdThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const TreeDraftState*>(state), max_nodes, tokens_out, parents_out, depth_out,
                     q_rows_out, count_out);
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
