// verify_stochastic.hip -- temperature softmax and stochastic chain verification.
//
// wc_probs_from_logits: p = softmax(logits / max(T, 1e-6)) per row in fp32
// (python/woodcock/sampling.py:39-45; src/sampling/sampling.cpp:9-45), two
// launches: per-chunk (max, sum of exp), then every chunk merges its row's
// partials and writes its probabilities.
//
// wc_verify_chain_stochastic: the Leviathan / Chen rule of the engine's chain
// path (python/woodcock/spec.py:316-324 -> verify_tree_stochastic with width 1,
// sampling.py:143-177, which equals verify_chain_stochastic, sampling.py:69-82):
//   for i < K: x = d_i, q_i(x) = q_i[row(x)] / sum_r q_i[r] (the draft
//   distribution over the head rows scattered through d2t and renormalised in
//   fp64, spec.py:240-248); q_i(x) <= 0 rejects without a uniform, else
//   u < min(1, p_i(x) / q_i(x)) accepts;
//   on rejection at i the next token is drawn from max(p_i - q_i, 0)
//   (p_i itself when that mass is <= 1e-12, sampling.py:182-187), after K
//   acceptances from p_K; a draw is the first x whose running sum exceeds
//   u * total (sampling.py:190-193).
// Every decision is fp64.  Uniforms come from the Philox4x64-10 stream
// (seed, round, purpose) in consumption order.  Two launches: per verify row
// the draft mass and the values at the drafted token; then a grid over the
// vocabulary in which every block repeats the (tiny) accept scan, sums its
// chunk of the chosen row, and the last block locates the draw.
#include "wc_common.h"

namespace wc {

constexpr int kStThreads = 256;
constexpr int kPerThread = kVocabChunk / kStThreads;  // 16 entries of a chunk per thread

struct StochArgs {
  const float* p;  // [rows][ld_p] target probabilities
  int rows, vocab;
  int64_t ld_p;
  const float* q;  // [rows-1][ld_q] draft probabilities over the head rows
  int head_rows;
  int64_t ld_q;
  const int32_t* d2t;     // [head_rows] ascending target ids, or NULL = identity
  const int32_t* drafts;  // [rows-1]
  const int32_t* draft_rows;  // [rows-1] head rows of the drafts, or NULL = search d2t
  unsigned long long seed;
  const int32_t* round_dev;
  int purpose;
  double* row_data;    // [WC_MAX_NODES][4]: Q, p(x), q_raw(x), flags
  double* chunk_data;  // [kMaxVocabChunks][2]: residual mass, target mass
  unsigned int* counter;
  wc_verdict* verdict;
};

__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kStThreads / kWave; ++w) t += red[w];
  return t;
}

// first index r in [0, n) with d2t[r] >= x (d2t ascending)
__device__ __forceinline__ int lower_bound_i32(const int32_t* d2t, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (d2t[mid] < x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// ------------------------------------------------------------------ per-row prologue

// Block i < K: draft mass Q_i = sum_r q_i[r] (fp64), the head row of d_i, and
// p_i(d_i), q_i[row].  Block K validates d2t (ascending, within the vocabulary)
// and the drafted tokens.
__global__ __launch_bounds__(kStThreads) void k_stoch_rows(StochArgs a) {
  __shared__ double red[kStThreads / kWave];
  __shared__ int s_bad;
  const int i = blockIdx.x, K = a.rows - 1;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();
  if (i == K) {
    int bad = 0;
    if (a.d2t) {
      for (int r = threadIdx.x; r < a.head_rows; r += kStThreads) {
        const int t = a.d2t[r];
        if (t < 0 || t >= a.vocab || (r + 1 < a.head_rows && a.d2t[r + 1] <= t)) bad = 1;
      }
    }
    for (int k = threadIdx.x; k < K; k += kStThreads)
      if (a.drafts[k] < 0 || a.drafts[k] >= a.vocab) bad = 1;
    if (bad) s_bad = 1;
    __syncthreads();
    if (threadIdx.x == 0) a.row_data[4 * WC_MAX_NODES - 1] = s_bad ? 1.0 : 0.0;  // flags slot of the last row
    return;
  }
  const float* qr = a.q + static_cast<int64_t>(i) * a.ld_q;
  double s = 0.0;
#pragma unroll 8
  for (int r = threadIdx.x; r < a.head_rows; r += kStThreads) s += static_cast<double>(qr[r]);
  s = block_sum_f64(s, red);
  if (threadIdx.x == 0) {
    const int x = min(max(a.drafts[i], 0), a.vocab - 1);
    int row = -1;
    if (a.draft_rows) {
      row = a.draft_rows[i];
      if (row < 0 || row >= a.head_rows || (a.d2t ? a.d2t[row] : row) != x) row = -1;
    } else if (a.d2t) {
      const int r = lower_bound_i32(a.d2t, a.head_rows, x);
      row = (r < a.head_rows && a.d2t[r] == x) ? r : -1;
    } else {
      row = x < a.head_rows ? x : -1;
    }
    double* rd = a.row_data + 4 * i;
    rd[0] = s;
    rd[1] = static_cast<double>(a.p[static_cast<int64_t>(i) * a.ld_p + x]);
    rd[2] = row >= 0 ? static_cast<double>(qr[row]) : 0.0;
  }
}

// ------------------------------------------------------------------ accept scan

struct Decision {
  int n;          // accepted drafts (the rejected position, or K)
  int residual;   // 1: draw from max(p_n - q_n, 0); 0: from p_n
  int n_uniforms; // consumed by the accept tests
};

// Sequential accept tests (sampling.py:74-80 / 163-170 at width 1); plain loads
// of the prologue's results (a previous launch).
__device__ __forceinline__ Decision decide(const StochArgs& a, unsigned long long round) {
  const int K = a.rows - 1;
  Decision d{K, 0, 0};
  for (int i = 0; i < K; ++i) {
    const double* rd = a.row_data + 4 * i;
    const double Q = rd[0];
    const double qx = Q > 0.0 ? rd[2] / Q : 0.0;
    bool accept = false;
    if (qx > 0.0) {
      const double u = philox_uniform(a.seed, round, a.purpose, static_cast<unsigned long long>(d.n_uniforms++));
      accept = u < fmin(1.0, rd[1] / qx);
    }
    if (!accept) {
      d.n = i;
      d.residual = 1;
      return d;
    }
  }
  return d;
}

// Values of chunk c of the row to draw from: residual max(p - q, 0) and p, fp64.
// q is scattered into LDS from the head rows whose ids fall in the chunk.
__device__ __forceinline__ void chunk_values(const StochArgs& a, const Decision& d, int c, double* qchunk,
                                             double (&rv)[kPerThread], double (&pv)[kPerThread]) {
  const int x0 = c * kVocabChunk;
  const float* pr = a.p + static_cast<int64_t>(d.n) * a.ld_p;
  for (int j = threadIdx.x; j < kVocabChunk; j += kStThreads) qchunk[j] = 0.0;
  __syncthreads();
  if (d.residual) {
    const double Q = a.row_data[4 * d.n];
    const float* qr = a.q + static_cast<int64_t>(d.n) * a.ld_q;
    if (a.d2t) {
      const int r0 = lower_bound_i32(a.d2t, a.head_rows, x0);
      const int r1 = lower_bound_i32(a.d2t, a.head_rows, x0 + kVocabChunk);
      for (int r = r0 + threadIdx.x; r < r1; r += kStThreads) qchunk[a.d2t[r] - x0] = static_cast<double>(qr[r]) / Q;
    } else {
      for (int j = threadIdx.x; j < kVocabChunk && x0 + j < a.head_rows; j += kStThreads)
        qchunk[j] = static_cast<double>(qr[x0 + j]) / Q;
    }
  }
  __syncthreads();
  // thread t owns the 16 consecutive entries t*16 .. t*16+15 of the chunk
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int j = threadIdx.x * kPerThread + e, x = x0 + j;
    const double pd = x < a.vocab ? static_cast<double>(pr[x]) : 0.0;
    pv[e] = pd;
    rv[e] = fmax(pd - qchunk[j], 0.0);
  }
}

__global__ __launch_bounds__(kStThreads) void k_stoch_sample(StochArgs a) {
  __shared__ double red[kStThreads / kWave];
  __shared__ double qchunk[kVocabChunk];
  __shared__ double s_tsum[kStThreads];
  __shared__ int s_chunk, s_idx;
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  const Decision d = decide(a, round);
  const int c = blockIdx.x, nchunks = gridDim.x;

  double rv[kPerThread], pv[kPerThread];
  chunk_values(a, d, c, qchunk, rv, pv);
  double sr = 0.0, sp = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    sr += rv[e];
    sp += pv[e];
  }
  sr = block_sum_f64(sr, red);
  sp = block_sum_f64(sp, red);
  if (threadIdx.x == 0) {
    unsigned long long* cd = reinterpret_cast<unsigned long long*>(a.chunk_data + 2 * c);
    atomic_store_u64(cd, static_cast<unsigned long long>(__double_as_longlong(sr)));
    atomic_store_u64(cd + 1, static_cast<unsigned long long>(__double_as_longlong(sp)));
  }
  if (!last_block_done(a.counter, nchunks, c)) return;

  // ---- last block: totals, the chunk holding the draw, then the entry
  const bool bad = a.row_data[4 * WC_MAX_NODES - 1] != 0.0;
  double cr[2], cp[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = threadIdx.x + h * kStThreads;
    const unsigned long long* cd = reinterpret_cast<const unsigned long long*>(a.chunk_data + 2 * min(k, nchunks - 1));
    cr[h] = k < nchunks ? __longlong_as_double(static_cast<long long>(atomic_load_u64(cd))) : 0.0;
    cp[h] = k < nchunks ? __longlong_as_double(static_cast<long long>(atomic_load_u64(cd + 1))) : 0.0;
  }
  const double tot_r = block_sum_f64(cr[0] + cr[1], red);
  const double tot_p = block_sum_f64(cp[0] + cp[1], red);
  const bool use_r = d.residual && tot_r > 1e-12;  // sampling.py:184: residual mass <= 1e-12 -> p
  const double total = use_r ? tot_r : tot_p;
  const double u = philox_uniform(a.seed, round, a.purpose, static_cast<unsigned long long>(d.n_uniforms));
  const double target = u * total;
  // chunk with the first inclusive running sum above the target: the chunk
  // masses go to LDS (reusing qchunk), thread 0 walks them in order
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = threadIdx.x + h * kStThreads;
    if (k < nchunks) qchunk[k] = use_r ? cr[h] : cp[h];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double run = 0.0;
    int cs = nchunks - 1;
    for (int k = 0; k < nchunks; ++k) {
      const double v = qchunk[k];
      if (run + v > target) {
        cs = k;
        break;
      }
      run += v;
    }
    s_chunk = cs;
    red[0] = run;  // mass before the chunk
    s_idx = kVocabChunk;
  }
  __syncthreads();
  const int cs = s_chunk;
  const double before = red[0];
  __syncthreads();
  chunk_values(a, d, cs, qchunk, rv, pv);
  double tsum = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) tsum += use_r ? rv[e] : pv[e];
  s_tsum[threadIdx.x] = tsum;
  __syncthreads();
  if (threadIdx.x == 0) {  // exclusive running sums of the 256 thread ranges, in order
    double run = before;
    for (int t = 0; t < kStThreads; ++t) {
      const double v = s_tsum[t];
      s_tsum[t] = run;
      run += v;
    }
  }
  __syncthreads();
  double run = s_tsum[threadIdx.x];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    run += use_r ? rv[e] : pv[e];
    if (run > target) {
      atomicMin(&s_idx, static_cast<int>(threadIdx.x) * kPerThread + e);
      break;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int x = min(cs * kVocabChunk + s_idx, a.vocab - 1);  // searchsorted clamp (sampling.py:193)
    wc_verdict* v = a.verdict;
    for (int k = 0; k < d.n; ++k) {
      v->tokens[k] = a.drafts[k];
      v->keep[k] = k;
    }
    v->tokens[d.n] = x;
    v->keep[d.n] = d.n;
    v->n_accepted = d.n;
    v->next = x;
    v->n_keep = d.n + 1;
    v->n_uniforms = d.n_uniforms + 1;
    v->status = bad ? WC_E_INVALID : 0;
  }
}

// ------------------------------------------------------------------ stochastic tree

// wc_verify_tree_stochastic: recursive rejection down a draft tree whose
// children were drawn without replacement (python/woodcock/sampling.py:143-177;
// src/sampling/sampling.cpp:116-141).  At node v with children c_1, c_2, ...
// (ascending node index = draw order): x = token(c); q(x) <= 0 rejects without
// a uniform, else u < min(1, p(x) / q(x)) accepts and the walk moves to c; a
// rejection replaces p by norm(max(p - q, 0)) (p / sum p when that mass is
// <= 1e-12, sampling.py:182-187), zeroes q(x) and renormalises q by its new
// mass s, stopping when s <= 0.  With no child accepted (or at a leaf) the next
// token is drawn from the current p (sampling.py:190-193).
//
// After j rejections at v every entry is a fixed map of its own (p_i, q_i):
//   p <- mode_k ? max(p - q, 0) / div_k : p / div_k,   q <- (i == x_k) ? 0 : q / s_k
// for k = 1..j, so only the normalisers (div_k, s_k) need vocabulary-wide sums.
// q is zero outside the head rows, so each rejection's sums run over the head
// rows and the entries outside them contribute (sum of their p) / prod div_k.
// One block walks the tree (k_tree_walk); a grid over the vocabulary then sums
// the final distribution chunk by chunk and the last block locates the draw
// (k_tree_sample).

struct TreeState {
  double q_mass;  // Q of the final node: the sum of its draft probabilities
  int node, nsteps, n_uniforms, path_len, bad, pad[3];
  int path[WC_MAX_NODES];
  int x[WC_MAX_NODES];
  int mode[WC_MAX_NODES];
  double div[WC_MAX_NODES];
  double s[WC_MAX_NODES];
};
static_assert(sizeof(TreeState) <= kTreeStateBytes, "tree state exceeds its workspace slot");

struct TreeArgs {
  const float* p;  // [rows][ld_p] target probabilities per node
  int rows, vocab;
  int64_t ld_p;
  const float* q;  // [rows][ld_q] draft probabilities of each node's children, over the head rows
  int head_rows;
  int64_t ld_q;
  const int32_t* d2t;  // [head_rows] ascending target ids, or NULL = identity
  const int32_t* tokens;
  const int32_t* parents;
  unsigned long long seed;
  const int32_t* round_dev;
  int purpose;
  TreeState* st;
  double* chunk_data;  // [kMaxVocabChunks]
  unsigned int* counter;
  wc_verdict* verdict;
};

constexpr int kTwThreads = 1024;

// The map of j rejections applied to one entry (token id tok): returns p, sets q.
__device__ __forceinline__ double tree_chain(double p, double q, int tok, int j, const int* xs, const int* mode,
                                             const double* div, const double* sv, double& q_out) {
  for (int k = 0; k < j; ++k) {
    p = mode[k] ? fmax(p - q, 0.0) / div[k] : p / div[k];
    q = tok == xs[k] ? 0.0 : q / sv[k];
  }
  q_out = q;
  return p;
}

__device__ __forceinline__ double block_sum_tw(double v, double* red) {
  v = wave_sum(v);
  __syncthreads();
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kTwThreads / kWave; ++w) t += red[w];
  return t;
}

__device__ __forceinline__ int head_row_of(const TreeArgs& a, int x) {
  if (!a.d2t) return x < a.head_rows ? x : -1;
  const int r = lower_bound_i32(a.d2t, a.head_rows, x);
  return (r < a.head_rows && a.d2t[r] == x) ? r : -1;
}

__global__ __launch_bounds__(kTwThreads) void k_tree_walk(TreeArgs a) {
  __shared__ double red[kTwThreads / kWave];
  __shared__ int s_x[WC_MAX_NODES], s_mode[WC_MAX_NODES], s_path[WC_MAX_NODES];
  __shared__ double s_div[WC_MAX_NODES], s_s[WC_MAX_NODES];
  __shared__ int s_bad, s_acc, s_nu;
  __shared__ unsigned long long s_kids;
  const int t = threadIdx.x, N = a.rows;
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  if (t == 0) {
    s_bad = 0;
    s_nu = 0;
  }
  __syncthreads();
  {  // parents[0] = -1, 0 <= parents[i] < i, tokens inside the vocabulary, d2t ascending
    int bad = 0;
    for (int i = t; i < N; i += kTwThreads) {
      const int par = a.parents[i], tok = a.tokens[i];
      if (i == 0 ? par != -1 : (par < 0 || par >= i)) bad = 1;
      if (tok < 0 || tok >= a.vocab) bad = 1;
    }
    if (a.d2t)
      for (int r = t; r < a.head_rows; r += kTwThreads) {
        const int x = a.d2t[r];
        if (x < 0 || x >= a.vocab || (r + 1 < a.head_rows && a.d2t[r + 1] <= x)) bad = 1;
      }
    if (bad) s_bad = 1;
  }
  __syncthreads();
  const bool bad = s_bad != 0;
  int v = 0, plen = 0, j = 0;
  double Q = 1.0;
  while (!bad) {
    if (t < kWave) {
      const unsigned long long m = __ballot(t < N && a.parents[min(t, N - 1)] == v);
      if (t == 0) s_kids = m;
    }
    __syncthreads();
    unsigned long long kids = s_kids;
    j = 0;
    if (kids == 0) break;  // a leaf: the draw is from p[v]
    // node sums: Q, the target mass on the head rows and on the whole vocabulary
    const float* pr = a.p + static_cast<int64_t>(v) * a.ld_p;
    const float* qr = a.q + static_cast<int64_t>(v) * a.ld_q;
    double sq = 0.0, sph = 0.0, spa = 0.0;
    for (int r = t; r < a.head_rows; r += kTwThreads) {
      sq += static_cast<double>(qr[r]);
      sph += static_cast<double>(pr[a.d2t ? a.d2t[r] : r]);
    }
    for (int i = t; i < a.vocab; i += kTwThreads) spa += static_cast<double>(pr[i]);
    Q = block_sum_tw(sq, red);
    const double p_head = block_sum_tw(sph, red);
    const double p_out = block_sum_tw(spa, red) - p_head;  // mass where q = 0
    double divprod = 1.0;
    int accepted = -1;
    while (kids != 0) {
      const int c = __builtin_ctzll(kids);
      kids &= kids - 1;
      const int x = a.tokens[c];
      if (t == 0) {  // the accept test at x after j rejections
        const int rx = head_row_of(a, x);
        const double q0 = (rx >= 0 && Q > 0.0) ? static_cast<double>(qr[rx]) / Q : 0.0;
        double qx;
        const double px = tree_chain(static_cast<double>(pr[x]), q0, x, j, s_x, s_mode, s_div, s_s, qx);
        int acc = -1;
        if (qx > 0.0) {
          const double u = philox_uniform(a.seed, round, a.purpose, static_cast<unsigned long long>(s_nu++));
          if (u < fmin(1.0, px / qx)) acc = c;
        }
        s_acc = acc;
      }
      __syncthreads();
      accepted = s_acc;
      if (accepted >= 0) break;
      // rejection j + 1: residual mass, current p mass and the renormalising q mass
      double z = 0.0, ps = 0.0, ss = 0.0;
      for (int r = t; r < a.head_rows; r += kTwThreads) {
        const int tok = a.d2t ? a.d2t[r] : r;
        const double q0 = Q > 0.0 ? static_cast<double>(qr[r]) / Q : 0.0;
        double qj;
        const double pj = tree_chain(static_cast<double>(pr[tok]), q0, tok, j, s_x, s_mode, s_div, s_s, qj);
        z += fmax(pj - qj, 0.0);
        ps += pj;
        ss += tok == x ? 0.0 : qj;
      }
      z = block_sum_tw(z, red);
      ps = block_sum_tw(ps, red);
      ss = block_sum_tw(ss, red);
      const double outside = p_out / divprod;
      const double zt = outside + z;
      const bool normal = zt > 1e-12;
      const double div = normal ? zt : outside + ps;
      if (t == 0) {
        s_x[j] = x;
        s_mode[j] = normal ? 1 : 0;
        s_div[j] = div;
        s_s[j] = ss;
      }
      __syncthreads();
      divprod *= div;
      ++j;
      if (ss <= 0.0) break;
    }
    if (accepted < 0) break;  // every child rejected: the draw is from the current p at v
    if (t == 0) s_path[plen] = accepted;
    ++plen;
    v = accepted;
    __syncthreads();
  }
  __syncthreads();
  TreeState* st = a.st;
  if (t == 0) {
    st->q_mass = Q;
    st->node = bad ? 0 : v;
    st->nsteps = bad ? 0 : j;
    st->n_uniforms = s_nu;
    st->path_len = bad ? 0 : plen;
    st->bad = bad ? 1 : 0;
  }
  if (t < WC_MAX_NODES) {
    st->path[t] = s_path[t];
    st->x[t] = s_x[t];
    st->mode[t] = s_mode[t];
    st->div[t] = s_div[t];
    st->s[t] = s_s[t];
  }
}

__global__ __launch_bounds__(kStThreads) void k_tree_sample(TreeArgs a) {
  __shared__ double red[kStThreads / kWave];
  __shared__ double qchunk[kVocabChunk];
  __shared__ double s_tsum[kStThreads];
  __shared__ int s_x[WC_MAX_NODES], s_mode[WC_MAX_NODES];
  __shared__ double s_div[WC_MAX_NODES], s_s[WC_MAX_NODES];
  __shared__ int s_chunk, s_idx;
  const TreeState* st = a.st;
  const int t = threadIdx.x;
  const int v = st->node, j = st->nsteps;
  const double Q = st->q_mass;
  if (t < WC_MAX_NODES) {
    s_x[t] = st->x[t];
    s_mode[t] = st->mode[t];
    s_div[t] = st->div[t];
    s_s[t] = st->s[t];
  }
  const float* pr = a.p + static_cast<int64_t>(v) * a.ld_p;
  const float* qr = a.q ? a.q + static_cast<int64_t>(v) * a.ld_q : nullptr;
  // values of chunk c of the final distribution: q of the head rows in the chunk
  // scattered into LDS (zero elsewhere), then the j-step map per entry
  auto values = [&](int c, double (&val)[kPerThread]) {
    const int x0 = c * kVocabChunk;
    for (int k = t; k < kVocabChunk; k += kStThreads) qchunk[k] = 0.0;
    __syncthreads();
    if (j > 0 && qr && Q > 0.0) {
      if (a.d2t) {
        const int r0 = lower_bound_i32(a.d2t, a.head_rows, x0);
        const int r1 = lower_bound_i32(a.d2t, a.head_rows, x0 + kVocabChunk);
        for (int r = r0 + t; r < r1; r += kStThreads) qchunk[a.d2t[r] - x0] = static_cast<double>(qr[r]) / Q;
      } else {
        for (int k = t; k < kVocabChunk && x0 + k < a.head_rows; k += kStThreads)
          qchunk[k] = static_cast<double>(qr[x0 + k]) / Q;
      }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int k = t * kPerThread + e, x = x0 + k;
      double qo;
      val[e] = x < a.vocab ? tree_chain(static_cast<double>(pr[x]), qchunk[k], x, j, s_x, s_mode, s_div, s_s, qo)
                           : 0.0;
    }
  };
  const int c = blockIdx.x, nchunks = gridDim.x;
  double val[kPerThread];
  values(c, val);
  double sum = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) sum += val[e];
  sum = block_sum_f64(sum, red);
  if (t == 0)
    atomic_store_u64(reinterpret_cast<unsigned long long*>(a.chunk_data + c),
                     static_cast<unsigned long long>(__double_as_longlong(sum)));
  if (!last_block_done(a.counter, nchunks, c)) return;

  // ---- last block: the total, the chunk holding u * total, then the entry
  double cm[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = t + h * kStThreads;
    const unsigned long long* cd = reinterpret_cast<const unsigned long long*>(a.chunk_data + min(k, nchunks - 1));
    cm[h] = k < nchunks ? __longlong_as_double(static_cast<long long>(atomic_load_u64(cd))) : 0.0;
  }
  const double total = block_sum_f64(cm[0] + cm[1], red);
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  const int nu = st->n_uniforms;
  const double target = philox_uniform(a.seed, round, a.purpose, static_cast<unsigned long long>(nu)) * total;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = t + h * kStThreads;
    if (k < nchunks) qchunk[k] = cm[h];
  }
  __syncthreads();
  if (t == 0) {
    double run = 0.0;
    int cs = nchunks - 1;
    for (int k = 0; k < nchunks; ++k) {
      if (run + qchunk[k] > target) {
        cs = k;
        break;
      }
      run += qchunk[k];
    }
    s_chunk = cs;
    red[0] = run;
    s_idx = kVocabChunk;
  }
  __syncthreads();
  const int cs = s_chunk;
  const double before = red[0];
  __syncthreads();
  values(cs, val);
  double tsum = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) tsum += val[e];
  s_tsum[t] = tsum;
  __syncthreads();
  if (t == 0) {
    double run = before;
    for (int k = 0; k < kStThreads; ++k) {
      const double w = s_tsum[k];
      s_tsum[k] = run;
      run += w;
    }
  }
  __syncthreads();
  double run = s_tsum[t];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    run += val[e];
    if (run > target) {
      atomicMin(&s_idx, t * kPerThread + e);
      break;
    }
  }
  __syncthreads();
  if (t == 0) {
    const int x = min(cs * kVocabChunk + s_idx, a.vocab - 1);  // searchsorted clamp (sampling.py:193)
    const int plen = st->path_len;
    wc_verdict* out = a.verdict;
    out->keep[0] = 0;
    for (int k = 0; k < plen; ++k) {
      out->tokens[k] = a.tokens[st->path[k]];
      out->keep[k + 1] = st->path[k];
    }
    out->tokens[plen] = x;
    out->n_accepted = plen;
    out->next = x;
    out->n_keep = plen + 1;
    out->n_uniforms = nu + 1;
    out->status = st->bad ? WC_E_INVALID : 0;
  }
}

// ------------------------------------------------------------------ softmax

struct ProbsArgs {
  const float* logits;
  int rows, n;
  int64_t ld;
  float temperature;
  float* out;
  int64_t ld_out;
  float* part;  // [rows][kMaxVocabChunks][2]
};

__device__ __forceinline__ float scaled(const ProbsArgs& a, float v) { return v / a.temperature; }

// (max, sum of exp(x - max)) of chunk blockIdx.x of row blockIdx.y
__global__ __launch_bounds__(kStThreads) void k_softmax_part(ProbsArgs a) {
  __shared__ float s_m[kStThreads / kWave], s_s[kStThreads / kWave];
  const int r = blockIdx.y, x0 = blockIdx.x * kVocabChunk;
  const float* lr = a.logits + static_cast<int64_t>(r) * a.ld;
  float v[kPerThread];
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int x = x0 + e * kStThreads + threadIdx.x;
    v[e] = x < a.n ? scaled(a, lr[min(x, a.n - 1)]) : -INFINITY;
    m = fmaxf(m, v[e]);
  }
  m = wave_max(m);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  float M = s_m[0];
  for (int w = 1; w < kStThreads / kWave; ++w) M = fmaxf(M, s_m[w]);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) s += v[e] == -INFINITY ? 0.f : expf(v[e] - M);
  s = wave_sum(s);
  if (lane == 0) s_s[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int w = 0; w < kStThreads / kWave; ++w) t += s_s[w];
    float* pp = a.part + (static_cast<int64_t>(r) * kMaxVocabChunks + blockIdx.x) * 2;
    pp[0] = M;
    pp[1] = t;
  }
}

// merge the row's partials, then p = exp(x - M) / S for chunk blockIdx.x
__global__ __launch_bounds__(kStThreads) void k_softmax_write(ProbsArgs a) {
  __shared__ float s_M, s_S;
  const int r = blockIdx.y, x0 = blockIdx.x * kVocabChunk, nch = gridDim.x;
  const float* pp = a.part + static_cast<int64_t>(r) * kMaxVocabChunks * 2;
  if (threadIdx.x < kWave) {
    float m = -INFINITY;
    for (int c = threadIdx.x; c < nch; c += kWave) m = fmaxf(m, pp[2 * c]);
    m = wave_max(m);
    float s = 0.f;
    for (int c = threadIdx.x; c < nch; c += kWave) {
      const float mc = pp[2 * c];
      s += mc == -INFINITY ? 0.f : pp[2 * c + 1] * expf(mc - m);
    }
    s = wave_sum(s);
    if (threadIdx.x == 0) {
      s_M = m;
      s_S = s;
    }
  }
  __syncthreads();
  const float M = s_M, S = s_S;
  const float* lr = a.logits + static_cast<int64_t>(r) * a.ld;
  float* orow = a.out + static_cast<int64_t>(r) * a.ld_out;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int x = x0 + e * kStThreads + threadIdx.x;
    if (x < a.n) orow[x] = expf(scaled(a, lr[x]) - M) / S;
  }
}

}  // namespace wc

extern "C" {

int wc_probs_from_logits(const float* logits, int rows, int n, int64_t ld, float temperature, float* out,
                         int64_t ld_out, void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(logits && out, "wc_probs_from_logits: NULL buffer");
  WC_REQUIRE(workspace && aligned(workspace, 16), "wc_probs_from_logits: workspace is NULL or misaligned");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "wc_probs_from_logits: rows must be in 1..%d (got %d)",
             WC_MAX_NODES, rows);
  WC_REQUIRE(n >= 1 && n <= kVocabChunk * kMaxVocabChunks, "wc_probs_from_logits: width %d out of range", n);
  WC_REQUIRE(ld >= n && ld_out >= n, "wc_probs_from_logits: row stride smaller than the width");
  ProbsArgs a{};
  a.logits = logits;
  a.rows = rows;
  a.n = n;
  a.ld = ld;
  a.temperature = temperature > 1e-6f ? temperature : 1e-6f;  // max(T, 1e-6), sampling.py:40
  a.out = out;
  a.ld_out = ld_out;
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kProbsOff);
  const dim3 grid((n + kVocabChunk - 1) / kVocabChunk, rows);
  auto s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_softmax_part, grid, dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL(k_softmax_write, grid, dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_verify_chain_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, int head_rows,
                               int64_t ld_q, const int32_t* d2t_dev, const int32_t* draft_tokens_dev,
                               const int32_t* draft_rows_dev, const wc_uniforms* rng, wc_verdict* verdict_dev,
                               void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(p && verdict_dev && rng && rng->round_dev, "wc_verify_chain_stochastic: NULL buffer");
  WC_REQUIRE(workspace && aligned(workspace, 16), "wc_verify_chain_stochastic: workspace is NULL or misaligned");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "wc_verify_chain_stochastic: rows must be in 1..%d (got %d)",
             WC_MAX_NODES, rows);
  WC_REQUIRE(vocab >= 1 && vocab <= kVocabChunk * kMaxVocabChunks,
             "wc_verify_chain_stochastic: vocab %d out of range", vocab);
  WC_REQUIRE(ld_p >= vocab, "wc_verify_chain_stochastic: p row stride smaller than vocab");
  WC_REQUIRE(rows == 1 || (q && draft_tokens_dev), "wc_verify_chain_stochastic: draft probabilities or tokens NULL");
  WC_REQUIRE(rows == 1 || (head_rows >= 1 && ld_q >= head_rows),
             "wc_verify_chain_stochastic: bad draft distribution width / stride");
  WC_REQUIRE(d2t_dev != nullptr || head_rows <= vocab,
             "wc_verify_chain_stochastic: without d2t the draft distribution must not exceed the vocabulary");
  StochArgs a{};
  a.p = p;
  a.rows = rows;
  a.vocab = vocab;
  a.ld_p = ld_p;
  a.q = q;
  a.head_rows = head_rows;
  a.ld_q = ld_q;
  a.d2t = d2t_dev;
  a.drafts = draft_tokens_dev;
  a.draft_rows = draft_rows_dev;
  a.seed = rng->seed;
  a.round_dev = rng->round_dev;
  a.purpose = rng->purpose;
  a.row_data = reinterpret_cast<double*>(static_cast<char*>(workspace) + kStochRowOff);
  a.chunk_data = reinterpret_cast<double*>(static_cast<char*>(workspace) + kStochChunkOff);
  a.counter = verify_counter(workspace, kCtrStochastic);
  a.verdict = verdict_dev;
  auto s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_stoch_rows, dim3(rows), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL(k_stoch_sample, dim3((vocab + kVocabChunk - 1) / kVocabChunk), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_verify_tree_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, int head_rows,
                              int64_t ld_q, const int32_t* d2t_dev, const int32_t* tree_tokens_dev,
                              const int32_t* tree_parents_dev, const wc_uniforms* rng, wc_verdict* verdict_dev,
                              void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(p && tree_tokens_dev && tree_parents_dev && verdict_dev && rng && rng->round_dev,
             "wc_verify_tree_stochastic: NULL buffer");
  WC_REQUIRE(workspace && aligned(workspace, 16), "wc_verify_tree_stochastic: workspace is NULL or misaligned");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "wc_verify_tree_stochastic: rows must be in 1..%d (got %d)",
             WC_MAX_NODES, rows);
  WC_REQUIRE(vocab >= 1 && vocab <= kVocabChunk * kMaxVocabChunks, "wc_verify_tree_stochastic: vocab %d out of range",
             vocab);
  WC_REQUIRE(ld_p >= vocab, "wc_verify_tree_stochastic: p row stride smaller than vocab");
  WC_REQUIRE(rows == 1 || (q && head_rows >= 1 && ld_q >= head_rows),
             "wc_verify_tree_stochastic: bad draft distribution buffer / width / stride");
  WC_REQUIRE(d2t_dev != nullptr || head_rows <= vocab,
             "wc_verify_tree_stochastic: without d2t the draft distribution must not exceed the vocabulary");
  TreeArgs a{};
  a.p = p;
  a.rows = rows;
  a.vocab = vocab;
  a.ld_p = ld_p;
  a.q = q;
  a.head_rows = rows == 1 ? 0 : head_rows;
  a.ld_q = ld_q;
  a.d2t = d2t_dev;
  a.tokens = tree_tokens_dev;
  a.parents = tree_parents_dev;
  a.seed = rng->seed;
  a.round_dev = rng->round_dev;
  a.purpose = rng->purpose;
  a.st = reinterpret_cast<TreeState*>(static_cast<char*>(workspace) + kTreeStateOff);
  a.chunk_data = reinterpret_cast<double*>(static_cast<char*>(workspace) + kStochChunkOff);
  a.counter = verify_counter(workspace, kCtrTree);
  a.verdict = verdict_dev;
  auto s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_tree_walk, dim3(1), dim3(kTwThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL(k_tree_sample, dim3((vocab + kVocabChunk - 1) / kVocabChunk), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  return WC_OK;
}

}  // extern "C"
