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
//
// wc_verify_chain_stochastic_logits: the same rule on p = softmax(logits / T)
// formed in place -- one launch with mailbox hand-over (k_stoch_fused) for
// K + 1 <= 8 rows, else two launches (k_stoch_stats + k_stoch_sample<true>).
//
// wc_verify_tree_stochastic: the recursive rule down a draft tree (below).
#include <atomic>
#include <cmath>

#include "wc_common.h"

namespace wc {

constexpr int kStThreads = 256;
constexpr int kPerThread = kVocabChunk / kStThreads;  // 16 entries of a chunk per thread

// LDS slot of chunk entry j in the fp64 chunk buffers: entry e of thread t's
// 16 (j = 16 t + e) sits at e * 256 + t, so a wave's reads of one e hit
// consecutive slots instead of one bank every 128 bytes
__device__ __forceinline__ int qslot(int j) { return (j % kPerThread) * kStThreads + j / kPerThread; }

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
  int32_t* chunk_rows; // [kMaxVocabChunks + 1]: first head row of each vocabulary chunk
  unsigned int* counter;
  wc_verdict* verdict;
  // from logits (wc_verify_chain_stochastic_logits): p = softmax(logits / T) computed in place
  const float* logits;
  int64_t ld_l;
  float temperature;
  float inv_t;          // 1 / T when T is a power of two, else 0
  float* part;          // [rows][kMaxVocabChunks][2] softmax partials (max, sum)
  int32_t* dec;         // n, residual, n_uniforms
  float* dec_ms;        // the chosen row's softmax max and sum
  unsigned int* bad_flag;  // invalid d2t / drafts seen by the statistics launch (reset by its last block)
  unsigned int* stats_counter;
  unsigned int spin_limit;  // polls before a waiting block of the one-launch kernel gives up
};

// Block-wide fp64 sum over kStThreads threads (DPP wave sums, then the wave
// totals in order); red holds one slot per wave.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kStThreads / kWave; ++w) t += red[w];
  return t;
}

// Block sums of two doubles at once (one pair of barriers); s_w holds 2 per wave.
__device__ __forceinline__ void block_sum2_f64(double& x, double& y, double* s_w) {
  x = wave_sum_dpp(x);
  y = wave_sum_dpp(y);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) {
    s_w[2 * wave] = x;
    s_w[2 * wave + 1] = y;
  }
  __syncthreads();
  double tx = 0.0, ty = 0.0;
  for (int w = 0; w < kStThreads / kWave; ++w) {
    tx += s_w[2 * w];
    ty += s_w[2 * w + 1];
  }
  x = tx;
  y = ty;
}

// Exclusive prefix sum over the lanes of one wave (lane order); the whole wave
// must be active.
__device__ __forceinline__ double block_wave_excl_scan(double v) {
  return wave_excl_from_incl(wave_incl_scan_dpp(v));
}

// before + the exclusive prefix sum of one value per thread, in thread order:
// a wave-level scan, then the totals of the lower waves.
__device__ __forceinline__ double block_excl_scan(double v, double before, double* s_w) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const double x = wave_incl_scan_dpp(v);
  const double ex = wave_excl_from_incl(x);
  __syncthreads();
  if (lane == kWave - 1) s_w[wave] = x;
  __syncthreads();
  double base = before;
  for (int w = 0; w < wave; ++w) base += s_w[w];
  return lane == 0 ? base : base + ex;
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

// chunk_rows[c] = the first head row whose id is in vocabulary chunk c or later
// (d2t ascending; an invalid d2t yields some table within [0, head_rows], and
// is reported separately).  Head row r writes the entries of the chunks that
// start after row r - 1's chunk, up to and including its own.
__device__ __forceinline__ void chunk_table(const StochArgs& a, int rb, int re) {
  const int nch = (a.vocab + kVocabChunk - 1) / kVocabChunk;
  int32_t* __restrict__ tab = a.chunk_rows;
  if (!a.d2t) {
    if (rb == 0)
      for (int c = threadIdx.x; c <= nch; c += kStThreads) tab[c] = min(c * kVocabChunk, a.head_rows);
    return;
  }
  // batches of 8 rows per thread: every id of a batch is loaded before the
  // first table store, so the loads of a batch are in flight together
  const int32_t* __restrict__ d2t = a.d2t;
  constexpr int kB = 8;
  for (int r0 = rb + threadIdx.x; r0 < re; r0 += kStThreads * kB) {
    int cur[kB], prv[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int r = min(r0 + u * kStThreads, a.head_rows - 1);
      cur[u] = d2t[r];
      prv[u] = d2t[max(r - 1, 0)];
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int r = r0 + u * kStThreads;
      if (r >= re) continue;
      const int ci = min(max(cur[u], 0) / kVocabChunk, nch);
      const int prev = r == 0 ? -1 : min(max(prv[u], 0) / kVocabChunk, nch);
      for (int c = prev + 1; c <= ci; ++c) tab[c] = r;
      if (r == a.head_rows - 1)
        for (int c = ci + 1; c <= nch; ++c) tab[c] = a.head_rows;
    }
  }
}

// 1 when this thread's share of d2t rows [rb, re) is not ascending or leaves
// the vocabulary (branch-free, in batches of 8 rows whose loads are in flight
// together).
__device__ __forceinline__ int d2t_bad(const StochArgs& a, int rb, int re) {
  const int32_t* __restrict__ d2t = a.d2t;
  constexpr int kB = 8;
  int bad = 0;
  for (int j0 = rb + threadIdx.x; j0 < re; j0 += kStThreads * kB) {
    int t[kB], nx[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int j = min(j0 + u * kStThreads, a.head_rows - 1);
      t[u] = d2t[j];
      nx[u] = d2t[min(j + 1, a.head_rows - 1)];
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int j = j0 + u * kStThreads;
      const bool b = t[u] < 0 || t[u] >= a.vocab || (j + 1 < a.head_rows && nx[u] <= t[u]);
      bad |= (j < re && b) ? 1 : 0;
    }
  }
  return bad;
}

// Q_i = sum of draft row i over the head rows in fp64: thread t adds rows
// t, t + 256, ... in order, kB loads in flight per batch; then the block sum.
template <int kB = 16>
__device__ __forceinline__ double draft_mass(const float* qr, int head_rows, double* red) {
  double s = 0.0;
  for (int b0 = threadIdx.x; b0 < head_rows; b0 += kStThreads * kB) {
    float v[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) v[u] = qr[min(b0 + u * kStThreads, head_rows - 1)];
#pragma unroll
    for (int u = 0; u < kB; ++u)
      if (b0 + u * kStThreads < head_rows) s += static_cast<double>(v[u]);
  }
  return block_sum_f64(s, red);
}

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
    if (a.d2t) bad = d2t_bad(a, 0, a.head_rows);
    for (int k = threadIdx.x; k < K; k += kStThreads)
      if (a.drafts[k] < 0 || a.drafts[k] >= a.vocab) bad = 1;
    if (bad) s_bad = 1;
    chunk_table(a, 0, a.head_rows);
    __syncthreads();
    if (threadIdx.x == 0) a.row_data[4 * WC_MAX_NODES - 1] = s_bad ? 1.0 : 0.0;  // flags slot of the last row
    return;
  }
  const float* qr = a.q + static_cast<int64_t>(i) * a.ld_q;
  const double s = draft_mass(qr, a.head_rows, red);
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

// Sequential accept tests (sampling.py:74-80 / 163-170 at width 1) over the
// per-row data rd [K][4] (Q, p(x), q_raw(x)).
__device__ __forceinline__ Decision decide_rows(const double* row_data, int K, unsigned long long seed,
                                                unsigned long long round, int purpose) {
  Decision d{K, 0, 0};
  for (int i = 0; i < K; ++i) {
    const double* rd = row_data + 4 * i;
    const double Q = rd[0];
    const double qx = Q > 0.0 ? rd[2] / Q : 0.0;
    bool accept = false;
    if (qx > 0.0) {
      const double u = philox_uniform(seed, round, purpose, static_cast<unsigned long long>(d.n_uniforms++));
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

// The same over the prologue's results (plain loads: a previous launch).
__device__ __forceinline__ Decision decide(const StochArgs& a, unsigned long long round) {
  return decide_rows(a.row_data, a.rows - 1, a.seed, round, a.purpose);
}

// Raw inputs of chunk c of row n, thread t's 16 consecutive entries: the
// materialised probabilities, or (FL) the logits; issued before anything that
// waits, the softmax (FL) is applied in chunk_values.
template <bool FL>
__device__ __forceinline__ void chunk_raw(const StochArgs& a, int n, int c, float (&raw)[kPerThread]) {
  const int x0 = c * kVocabChunk + threadIdx.x * kPerThread;
  const float* src = FL ? a.logits + static_cast<int64_t>(n) * a.ld_l : a.p + static_cast<int64_t>(n) * a.ld_p;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) raw[e] = src[min(x0 + e, a.vocab - 1)];
}

// Values of chunk c of the row to draw from: residual max(p - q, 0) and p, fp64.
// raw from chunk_raw; q is scattered into LDS from the head rows [r0, r1) whose
// ids fall in the chunk (the chunk table), divided by the draft mass Q.  With FL
// p = exp(logit / T - M) / S exactly as wc_probs_from_logits writes it.
template <bool FL>
__device__ __forceinline__ void chunk_values(const StochArgs& a, const Decision& d, int c, float M, float S,
                                             double Q, int r0, int r1, const float (&raw)[kPerThread],
                                             double* qchunk, double (&rv)[kPerThread], double (&pv)[kPerThread]) {
  // LDS-only barriers: the raw loads stay in flight while q is scattered
  const int x0 = c * kVocabChunk;
  for (int j = threadIdx.x; j < kVocabChunk; j += kStThreads) qchunk[j] = 0.0;
  lds_barrier();
  if (d.residual) {
    const float* qr = a.q + static_cast<int64_t>(d.n) * a.ld_q;
    r0 = min(max(r0, 0), a.head_rows);
    r1 = min(max(r1, r0), a.head_rows);
    for (int r = r0 + threadIdx.x; r < r1; r += kStThreads) {
      const int j = (a.d2t ? a.d2t[r] : r) - x0;
      if (j >= 0 && j < kVocabChunk) qchunk[qslot(j)] = static_cast<double>(qr[r]) / Q;
    }
  }
  lds_barrier();
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int j = threadIdx.x * kPerThread + e, x = x0 + j;
    const float pf = FL ? expf(raw[e] / a.temperature - M) / S : raw[e];
    const double pd = x < a.vocab ? static_cast<double>(pf) : 0.0;
    pv[e] = pd;
    rv[e] = fmax(pd - qchunk[e * kStThreads + threadIdx.x], 0.0);
  }
}

// FL: the decision and the chosen row's softmax (max, sum) come from the
// statistics launch of wc_verify_chain_stochastic_logits.
template <bool FL>
__global__ __launch_bounds__(kStThreads) void k_stoch_sample(StochArgs a) {
  __shared__ double red[kStThreads / kWave];
  __shared__ double qchunk[kVocabChunk];
  __shared__ double s_tsum[kStThreads];
  __shared__ int s_chunk, s_idx;
  __shared__ int s_tab[kMaxVocabChunks + 1];
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  Decision d;
  float M = 0.f, S = 1.f;
  if constexpr (FL) {
    d = Decision{a.dec[0], a.dec[1], a.dec[2]};
    M = a.dec_ms[0];
    S = a.dec_ms[1];
  } else {
    d = decide(a, round);
  }
  const int c = blockIdx.x, nchunks = gridDim.x;

  float raw[kPerThread];
  chunk_raw<FL>(a, d.n, c, raw);
  const int r0 = a.chunk_rows[c], r1 = a.chunk_rows[c + 1];
  const double Q = a.row_data[4 * d.n];
  double rv[kPerThread], pv[kPerThread];
  chunk_values<FL>(a, d, c, M, S, Q, r0, r1, raw, qchunk, rv, pv);
  double sr = 0.0, sp = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    sr += rv[e];
    sp += pv[e];
  }
  block_sum2_f64(sr, sp, s_tsum);
  if (threadIdx.x == 0) {
    unsigned long long* cd = reinterpret_cast<unsigned long long*>(a.chunk_data + 2 * c);
    atomic_store_u64(cd, static_cast<unsigned long long>(__double_as_longlong(sr)));
    atomic_store_u64(cd + 1, static_cast<unsigned long long>(__double_as_longlong(sp)));
  }
  if (!last_block_done(a.counter, nchunks, c)) return;

  // ---- last block: totals, the chunk holding the draw, then the entry.  The
  // chunk table and the drafts are loaded with the chunk masses.
  const bool bad = a.row_data[4 * WC_MAX_NODES - 1] != 0.0;
  for (int k = threadIdx.x; k <= nchunks; k += kStThreads) s_tab[k] = a.chunk_rows[k];
  const int dtok = threadIdx.x < d.n ? a.drafts[threadIdx.x] : 0;
  double cr[2], cp[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int k = threadIdx.x + h * kStThreads;
    const unsigned long long* cd = reinterpret_cast<const unsigned long long*>(a.chunk_data + 2 * min(k, nchunks - 1));
    cr[h] = k < nchunks ? __longlong_as_double(static_cast<long long>(atomic_load_u64(cd))) : 0.0;
    cp[h] = k < nchunks ? __longlong_as_double(static_cast<long long>(atomic_load_u64(cd + 1))) : 0.0;
  }
  double tot_r = cr[0] + cr[1], tot_p = cp[0] + cp[1];
  block_sum2_f64(tot_r, tot_p, s_tsum);
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
  if (nchunks <= kWave) {
    // wave 0, lane k = chunk k: exclusive running sums by lane shifts, the
    // first chunk whose inclusive sum exceeds the target by a ballot
    if (threadIdx.x < kWave) {
      const int k = threadIdx.x;
      const double v = k < nchunks ? qchunk[k] : 0.0;
      const double ex = block_wave_excl_scan(v);
      const unsigned long long hit = __ballot(k < nchunks && ex + v > target);
      const int cs = hit ? __ffsll(static_cast<long long>(hit)) - 1 : nchunks - 1;
      if (k == cs) {
        s_chunk = cs;
        red[0] = hit ? ex : ex + v;  // mass before the chunk (all of it when no chunk is hit, as the walk leaves it)
      }
      if (k == 0) s_idx = kVocabChunk;
    }
  } else if (threadIdx.x == 0) {
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
  chunk_raw<FL>(a, d.n, cs, raw);
  chunk_values<FL>(a, d, cs, M, S, Q, s_tab[cs], s_tab[cs + 1], raw, qchunk, rv, pv);
  double tsum = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) tsum += use_r ? rv[e] : pv[e];
  double run = block_excl_scan(tsum, before, s_tsum);  // running sum before this thread's 16 entries
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
    v->tokens[d.n] = x;
    v->keep[d.n] = d.n;
    v->n_accepted = d.n;
    v->next = x;
    v->n_keep = d.n + 1;
    v->n_uniforms = d.n_uniforms + 1;
    v->status = bad ? WC_E_INVALID : 0;
  }
  if (threadIdx.x < d.n) {
    a.verdict->tokens[threadIdx.x] = dtok;
    a.verdict->keep[threadIdx.x] = threadIdx.x;
  }
}

// ------------------------------------------------------------------ from logits

// Statistics launch of wc_verify_chain_stochastic_logits, grid (chunks, rows + 1):
//   row r < rows, chunk c: the chunk's (max, sum of exp) of logits / T, the
//     arithmetic of the softmax's first launch, handed over device-coherently;
//   row `rows`, block i < K: draft mass Q_i, q_i at the draft's head row and
//     p's logit at the draft (k_stoch_rows' work); block K: d2t / draft
//     validation and the chunk -> head-row table.
// The last block merges each row's partials as the softmax's second launch
// does, forms p_i(d_i), runs the accept tests and leaves the decision and the
// chosen row's (max, sum) for the sampling launch.
__global__ __launch_bounds__(kStThreads) void k_stoch_stats(StochArgs a) {
  __shared__ float s_m[kStThreads / kWave], s_s[kStThreads / kWave];
  __shared__ double red[kStThreads / kWave];
  __shared__ float s_M[WC_MAX_NODES], s_S[WC_MAX_NODES];
  __shared__ double s_rd[4 * WC_MAX_NODES];
  __shared__ int s_bad;
  const int c = blockIdx.x, r = blockIdx.y, K = a.rows - 1, nch = gridDim.x;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();
  if (r < a.rows) {
    const int x0 = c * kVocabChunk;
    const float* lr = a.logits + static_cast<int64_t>(r) * a.ld_l;
    float v[kPerThread];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) v[e] = lr[min(x0 + e * kStThreads + static_cast<int>(threadIdx.x), a.vocab - 1)];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) pin(v[e]);  // every load in flight at once
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int x = x0 + e * kStThreads + threadIdx.x;
      v[e] = x < a.vocab ? v[e] / a.temperature : -INFINITY;
      m = fmaxf(m, v[e]);
    }
    m = wave_max_dpp(m);
    if (lane == 0) s_m[wave] = m;
    __syncthreads();
    float M = s_m[0];
    for (int w = 1; w < kStThreads / kWave; ++w) M = fmaxf(M, s_m[w]);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) sum += v[e] == -INFINITY ? 0.f : expf(v[e] - M);
    sum = wave_sum_dpp(sum);
    if (lane == 0) s_s[wave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int w = 0; w < kStThreads / kWave; ++w) t += s_s[w];
      float* pp = a.part + (static_cast<int64_t>(r) * kMaxVocabChunks + c) * 2;
      publish_f32(pp, M);
      publish_f32(pp + 1, t);
    }
  } else if (c < K) {
    const float* qr = a.q + static_cast<int64_t>(c) * a.ld_q;
    const double sq = draft_mass(qr, a.head_rows, red);
    if (threadIdx.x == 0) {
      const int x = min(max(a.drafts[c], 0), a.vocab - 1);
      int row = -1;
      if (a.draft_rows) {
        row = a.draft_rows[c];
        if (row < 0 || row >= a.head_rows || (a.d2t ? a.d2t[row] : row) != x) row = -1;
      } else if (a.d2t) {
        const int rr = lower_bound_i32(a.d2t, a.head_rows, x);
        row = (rr < a.head_rows && a.d2t[rr] == x) ? rr : -1;
      } else {
        row = x < a.head_rows ? x : -1;
      }
      unsigned long long* rd = reinterpret_cast<unsigned long long*>(a.row_data + 4 * c);
      atomic_store_u64(rd, static_cast<unsigned long long>(__double_as_longlong(sq)));
      atomic_store_u64(rd + 2, static_cast<unsigned long long>(
                                   __double_as_longlong(row >= 0 ? static_cast<double>(qr[row]) : 0.0)));
    }
  } else {
    // blocks K .. gridDim.x - 1 of the extra row: a slice of the head rows each
    // for the d2t check and the chunk table; the first also checks the drafts
    const int ns = nch - K, b = c - K;
    const int rb = static_cast<int>(static_cast<int64_t>(a.head_rows) * b / ns);
    const int re = static_cast<int>(static_cast<int64_t>(a.head_rows) * (b + 1) / ns);
    int bad = 0;
    if (a.d2t) bad = d2t_bad(a, rb, re);
    if (b == 0)
      for (int k = threadIdx.x; k < K; k += kStThreads)
        if (a.drafts[k] < 0 || a.drafts[k] >= a.vocab) bad = 1;
    if (bad) s_bad = 1;
    chunk_table(a, rb, re);
    __syncthreads();
    if (threadIdx.x == 0 && s_bad) atomicOr(a.bad_flag, 1u);
  }
  if (!last_block_done(a.stats_counter, nch * (a.rows + 1), linear_block())) return;

  // ---- last block.  Every load first: the round, the logits at the drafts,
  // the draft rows' data, then each row's partials (a wave per row, two rows
  // per wave in flight, up to kMaxVocabChunks / 64 chunks per lane); the
  // merges then run as the softmax's second launch runs them (same order).
  constexpr int kCpl = kMaxVocabChunks / kWave;
  constexpr int kNw = kStThreads / kWave;
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  float lgx = 0.f;
  if (threadIdx.x < K) {
    const int x = min(max(a.drafts[threadIdx.x], 0), a.vocab - 1);
    lgx = a.logits[static_cast<int64_t>(threadIdx.x) * a.ld_l + x];
  }
  double rdv = 0.0;
  if (threadIdx.x < 4 * K)
    rdv = __longlong_as_double(static_cast<long long>(
        atomic_load_u64(reinterpret_cast<const unsigned long long*>(a.row_data + threadIdx.x))));
  for (int i0 = wave; i0 < a.rows; i0 += 2 * kNw) {
    float mc[2][kCpl], sc[2][kCpl];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float* pp = a.part + static_cast<int64_t>(min(i0 + h * kNw, a.rows - 1)) * kMaxVocabChunks * 2;
#pragma unroll
      for (int u = 0; u < kCpl; ++u) {
        const int cc = min(lane + u * kWave, nch - 1);
        mc[h][u] = fetch_f32(pp + 2 * cc);
        sc[h][u] = fetch_f32(pp + 2 * cc + 1);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = i0 + h * kNw;
      if (i >= a.rows) continue;
      float m = -INFINITY;
#pragma unroll
      for (int u = 0; u < kCpl; ++u)
        if (lane + u * kWave < nch) m = fmaxf(m, mc[h][u]);
      m = wave_max_dpp(m);
      float sum = 0.f;
#pragma unroll
      for (int u = 0; u < kCpl; ++u)
        if (lane + u * kWave < nch) sum += mc[h][u] == -INFINITY ? 0.f : sc[h][u] * expf(mc[h][u] - m);
      sum = wave_sum_dpp(sum);
      if (lane == 0) {
        s_M[i] = m;
        s_S[i] = sum;
      }
    }
  }
  if (threadIdx.x < 4 * K) s_rd[threadIdx.x] = rdv;
  if (threadIdx.x == 0) {  // the flags slot the sampling launch reads; the flag starts at zero for the next call
    const unsigned int bad = __hip_atomic_exchange(a.bad_flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a.row_data[4 * WC_MAX_NODES - 1] = bad ? 1.0 : 0.0;
  }
  __syncthreads();
  if (threadIdx.x < K) {  // p_i(d_i) as the written probabilities would hold it
    const int i = threadIdx.x;
    const float pf = expf(lgx / a.temperature - s_M[i]) / s_S[i];
    s_rd[4 * i + 1] = static_cast<double>(pf);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const Decision d = decide_rows(s_rd, K, a.seed, round, a.purpose);
    a.dec[0] = d.n;
    a.dec[1] = d.residual;
    a.dec[2] = d.n_uniforms;
    a.dec_ms[0] = s_M[d.n];
    a.dec_ms[1] = s_S[d.n];
    // the sampling launch reads Q_n and the flags with plain loads
    a.row_data[4 * d.n] = s_rd[4 * d.n];
  }
}

// ------------------------------------------------------------------ one launch

// wc_verify_chain_stochastic_logits in one launch, when rows <= kFusedRows and
// the chunk blocks (the only ones that wait) fit on the GPU at once (checked on
// the host):
//   statistics blocks (row r, chunk c), rows x nch: the chunk's (max, sum of
//     exp) of logits / T, k_stoch_stats' arithmetic;
//   chunk blocks (chunk c, rows [3 g, 3 g + 3)), ceil(rows / 3) per chunk:
//     this chunk of the block's rows held in registers, a window of head rows
//     holding those whose ids fall in the chunk (one step of a search of the
//     ascending d2t) and, when the window has at most kQPre rows, their ids
//     and the block's draft rows' probabilities staged in LDS;
//   draft-mass blocks i < K: Q_i and q_i at the draft's head row;
//   check blocks: a slice of d2t each (ascending, within the vocabulary), the
//     first also the drafts and the round's uniforms 0..K.
// Hand-over by mailboxes: every result is one 64-bit word, stored once per call
// with an agent-scope atomic store as the bitwise complement of its value, and
// a word reads 0 until it is written.  A chunk block polls (agent-scope atomic
// loads) every word it needs until none is 0 -- the poll's loads are the data
// loads, and no read-modify-write or flag is involved; no acquire / release
// fence at agent scope either, which would write back or invalidate the whole
// L2.  Once every statistics, mass and check word is in, each chunk block
// merges the partials of every row, forms p_i(d_i) and takes the accept tests
// itself -- the same arithmetic on the same data, so the same decision in every
// block; the block of each chunk that holds the chosen row then sums the
// residual / target mass of its chunk into its mailbox, the others end.  Once every chunk's masses are in, each chunk block
// locates the chunk of the draw; that chunk's block finds the entry in the
// values it holds and writes the verdict; the check blocks have cleared the
// other mailbox set for the next call.  Calls alternate between the two sets by
// the parity of the call counter, so a set is always cleared by the call before
// the one that uses it (a zero-initialised workspace starts both clear).  The
// counter moves only once every block of the call has read it: each chunk block
// posts an arrival word derived from the value it read, and the finishing block
// waits for all of them before it advances the counter (the other blocks' words
// are already in by then), so no block of a call can poll the next call's set,
// whatever order the blocks are dispatched in.
// Every wait is bounded (spin_limit polls).  A block that gives up sets the
// sticky failure flag of the control word and WC_E_HIP in the verdict; every
// later call then ends at once with WC_E_HIP, without touching the mailboxes,
// until the host zero-fills the workspace again (wc_workspace_init) -- so words
// a failed call left behind are never read as another call's.
// Every probability, sum and scan is formed as the two-launch path
// (k_stoch_stats + k_stoch_sample<true>) forms it.
struct MailSet {
  // kMailRep copies of every word, each written by the producer; a polling
  // block reads copy (block % kMailRep), which spreads the polls of one word
  // over several lines
  unsigned long long part[kMailRep][kMailRows][kMailChunks];  // row r, chunk c: sum bits << 32 | max bits
  unsigned long long csum[kMailRep][kMailChunks][2];          // chunk c: residual mass, target mass (fp64)
  // [0, 2K): Q_i, q_i at the draft (fp64); [2K, 3K + 1): uniforms 0..K;
  // [3K + 1, 3K + 1 + checks): 1 + (a check block found an invalid input)
  unsigned long long other[kMailRep][kMailOther];
  unsigned long long arrive[kMailArrive];  // chunk block cb: the complement of the call value it read
};
static_assert(sizeof(MailSet) == 8 * kMailSetWords, "mailbox layout");
static_assert(kGridBarOff % 8 == 0, "mailbox alignment");
constexpr unsigned int kSpinLimit = 1u << 22;  // default polls before a wait gives up (WC_E_HIP in the verdict)
static std::atomic<unsigned int> g_spin_limit{kSpinLimit};

// A wait that gave up: the sticky failure flag (high half of the control word)
// and WC_E_HIP in the verdict.  The flag is stored before the status, so a
// verdict that reads WC_E_HIP always leaves a flagged workspace behind.
__device__ __forceinline__ void stoch_give_up(const StochArgs& a, unsigned long long* ctl) {
  if (threadIdx.x == 0) {
    atomic_store_u32(reinterpret_cast<unsigned int*>(ctl) + 1, 1u);
    __builtin_amdgcn_s_waitcnt(0);
    a.verdict->status = WC_E_HIP;
  }
}

// every copy of a word: w points at copy 0, copies lie `stride` words apart
__device__ __forceinline__ void mail_put(unsigned long long* w, size_t stride, unsigned long long v) {
#pragma unroll
  for (int r = 0; r < kMailRep; ++r) atomic_store_u64(w + r * stride, ~v);
}
__device__ __forceinline__ void mail_put_f64(unsigned long long* w, size_t stride, double v) {
  mail_put(w, stride, static_cast<unsigned long long>(__double_as_longlong(v)));
}
constexpr size_t kPartRep = kMailRows * kMailChunks, kCsumRep = 2 * kMailChunks, kOtherRep = kMailOther;
__device__ __forceinline__ double mail_f64(unsigned long long raw) {
  return __longlong_as_double(static_cast<long long>(~raw));
}

constexpr int kFusedRows = kMailRows;           // K + 1 rows whose chunk each chunk block holds
constexpr int kFusedCpl = kMailChunks / kWave;  // chunks per lane in the merge: nch <= 256
constexpr int kQPre = 1024;    // head rows of a chunk staged in LDS before the decision
constexpr int kGroupRows = 3;  // rows of a chunk one chunk block holds: ceil(rows / 3) blocks per chunk
static_assert(kMailArrive >= (kFusedRows + kGroupRows - 1) / kGroupRows * kMailChunks, "arrival words");

// One step of a block-wide search for the first index r in [lo, hi] with
// d2t[r] >= x (d2t ascending).  Width <= 256: thread t probes lo + t; else the
// probes sit `step` apart and the bracket shrinks to step - 1.  Any d2t leaves
// lo <= hi within the starting range, and the width shrinks every step.
struct Probe {
  int lo, hi, step, pos, val;
};
__device__ __forceinline__ void probe_issue(const int32_t* d2t, Probe& p) {
  const int w = p.hi - p.lo;
  p.step = w <= kStThreads ? 1 : (w + kStThreads - 1) / kStThreads;
  p.pos = p.lo + (static_cast<int>(threadIdx.x) + 1) * p.step - 1;
  p.val = w > 0 ? d2t[min(p.pos, p.hi - 1)] : 0;
}
__device__ __forceinline__ void probe_apply(Probe& p, int x, int* s_cnt) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const bool less = p.pos < p.hi && p.val < x;
  const unsigned long long m = __ballot(less);
  if (lane == 0) s_cnt[wave] = __popcll(m);
  lds_barrier();
  int cnt = 0;
#pragma unroll
  for (int w = 0; w < kStThreads / kWave; ++w) cnt += s_cnt[w];
  const int lo = p.lo + cnt * p.step;
  p.hi = min(p.hi, p.lo + (cnt + 1) * p.step - 1);
  p.lo = lo;
}

// logit / T; with P2 (T a power of two) as logit * (1 / T), the same float:
// both round the same exact quotient once.  The product by a power of two is
// exact (normal range), so where the compiler contracts it into a following
// subtraction the fused result equals the two rounded steps.
template <bool P2>
__device__ __forceinline__ float lscale(const StochArgs& a, float x) {
  return P2 ? __fmul_rn(x, a.inv_t) : x / a.temperature;
}

template <bool P2>
__global__ __launch_bounds__(kStThreads) void k_stoch_fused(StochArgs a, int nch, int nchecks, int vec,
                                                           MailSet* sets, unsigned long long* ctl) {
  constexpr int kNw = kStThreads / kWave;
  __shared__ float s_m[kNw], s_s[kNw];
  __shared__ float s_M[kFusedRows], s_S[kFusedRows], s_lgx[kFusedRows];
  __shared__ double s_rd[4 * kFusedRows];  // per draft row: Q, -, q_raw(x), uniform i
  __shared__ double qchunk[kVocabChunk];
  __shared__ double s_tsum[kStThreads];
  __shared__ float s_q[kGroupRows][kQPre];
  __shared__ short s_j[kQPre];
  __shared__ int s_cnt[1][2][kNw];
  __shared__ int s_bad, s_chunk, s_idx;
  __shared__ double s_before;
  const int b = blockIdx.x, K = a.rows - 1, rows = a.rows;
  const int nstat = rows * nch, ngroups = (rows + kGroupRows - 1) / kGroupRows, nchunkb = ngroups * nch;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  // control word: the call counter (moves only at the end of the call, after
  // every block has read it) and the sticky failure flag
  const unsigned long long cw = atomic_load_u64(ctl);
  const unsigned int call = static_cast<unsigned int>(cw);
  if (cw >> 32) {  // an earlier call gave up: the mailboxes may hold its words
    if (b == 0 && threadIdx.x == 0) a.verdict->status = WC_E_HIP;
    return;
  }
  MailSet* mb = sets + (call & 1u);
  const int rep = blockIdx.x % kMailRep;  // the mailbox copy this block polls

  if (b < nstat) {
    // ---- statistics block (row r, chunk c)
    const int r = b / nch, c = b % nch, x0 = c * kVocabChunk;
    const float* lr = a.logits + static_cast<int64_t>(r) * a.ld_l;
    float v[kPerThread];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) v[e] = lr[min(x0 + e * kStThreads + static_cast<int>(threadIdx.x), a.vocab - 1)];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) pin(v[e]);  // every load in flight at once
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int x = x0 + e * kStThreads + threadIdx.x;
      v[e] = x < a.vocab ? lscale<P2>(a, v[e]) : -INFINITY;
      m = fmaxf(m, v[e]);
    }
    m = wave_max_dpp(m);
    if (lane == 0) s_m[wave] = m;
    __syncthreads();
    float M = s_m[0];
    for (int w = 1; w < kNw; ++w) M = fmaxf(M, s_m[w]);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) sum += v[e] == -INFINITY ? 0.f : expf(v[e] - M);
    sum = wave_sum_dpp(sum);
    if (lane == 0) s_s[wave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {  // (max, sum) as one word
      float t = 0.f;
      for (int w = 0; w < kNw; ++w) t += s_s[w];
      mail_put(&mb->part[0][r][c], kPartRep,
               static_cast<unsigned long long>(__float_as_uint(M)) |
                   (static_cast<unsigned long long>(__float_as_uint(t)) << 32));
    }
    return;
  }
  if (b >= nstat + nchunkb) {
    const int e = b - nstat - nchunkb;
    if (e < K) {  // ---- draft mass Q_i; uniform i (and uniform K in the last, on another wave)
      const double sq = draft_mass<64>(a.q + static_cast<int64_t>(e) * a.ld_q, a.head_rows, s_tsum);
      const int u = threadIdx.x == 0 ? e : (threadIdx.x == kWave && e == K - 1 ? K : -1);
      if (u >= 0) {
        const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
        mail_put_f64(&mb->other[0][2 * K + u], kOtherRep, philox_uniform(a.seed, round, a.purpose, u));
      }
      if (threadIdx.x == 0) mail_put_f64(&mb->other[0][2 * e], kOtherRep, sq);
      return;
    }
    // ---- check block bs of ns (ns >= K): a slice of d2t checked; q_bs at
    // draft bs's head row (bs < K); the drafts checked (bs == 0); a slice of
    // the other mailbox set cleared for the next call.  Loads first, then the
    // waits.
    const int ns = nchecks, bs = e - K;
    {
      unsigned long long* nxt = reinterpret_cast<unsigned long long*>(sets + ((call + 1u) & 1u));
      const int w0 = static_cast<int>(kMailSetWords * bs / ns), w1 = static_cast<int>(kMailSetWords * (bs + 1) / ns);
      for (int k = w0 + threadIdx.x; k < w1; k += kStThreads) atomic_store_u64(nxt + k, 0ull);
    }
    const bool lookup = bs < K;
    const int x = lookup ? min(max(a.drafts[bs], 0), a.vocab - 1) : 0;
    int row = lookup && a.draft_rows ? a.draft_rows[bs] : -1;
    if (threadIdx.x == 0) s_bad = 0;
    lds_barrier();
    const int rb = static_cast<int>(static_cast<int64_t>(a.head_rows) * bs / ns);
    const int re = static_cast<int>(static_cast<int64_t>(a.head_rows) * (bs + 1) / ns);
    int bad = a.d2t ? d2t_bad(a, rb, re) : 0;
    if (bs == 0)
      for (int k = threadIdx.x; k < K; k += kStThreads)
        if (a.drafts[k] < 0 || a.drafts[k] >= a.vocab) bad = 1;
    if (lookup) {  // the id at the candidate row and q there load together
      const float* qr = a.q + static_cast<int64_t>(bs) * a.ld_q;
      float qx = 0.f;
      if (a.draft_rows) {  // the given row, if it holds the draft
        const bool in = row >= 0 && row < a.head_rows;
        const int rc = in ? row : 0;
        const int id = a.d2t ? a.d2t[rc] : rc;
        qx = qr[rc];
        row = in && id == x ? row : -1;
      } else if (a.d2t) {  // block-wide search of the ascending d2t
        Probe p{0, a.head_rows, 1, 0, 0};
        for (int it = 0;; ++it) {
          probe_issue(a.d2t, p);
          probe_apply(p, x, s_cnt[0][it & 1]);
          if (p.lo == p.hi) break;
        }
        const int rc = min(p.lo, a.head_rows - 1);
        const int id = a.d2t[rc];
        qx = qr[rc];
        row = p.lo < a.head_rows && id == x ? p.lo : -1;
      } else {
        row = x < a.head_rows ? x : -1;
        qx = qr[max(row, 0)];
      }
      if (threadIdx.x == 0) mail_put_f64(&mb->other[0][2 * bs + 1], kOtherRep, row >= 0 ? static_cast<double>(qx) : 0.0);
    }
    if (K == 0 && bs == 0 && threadIdx.x == 0) {  // no draft-mass block: the one uniform here
      const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
      mail_put_f64(&mb->other[0][0], kOtherRep, philox_uniform(a.seed, round, a.purpose, 0));
    }
    if (bad) s_bad = 1;
    __syncthreads();
    if (threadIdx.x == 0) mail_put(&mb->other[0][3 * K + 1 + bs], kOtherRep, ~(1ull + static_cast<unsigned long long>(s_bad)));
    return;
  }

  // ---- chunk block (chunk c, rows [rlo, rhi)), ceil(rows / 3) blocks per
  // chunk so that no block loads more than three rows.  One step of the d2t
  // search brackets the head rows whose ids fall in the chunk: the window
  // [w0, w1) holds them (ids outside the chunk are dropped by their offset);
  // then the window's ids and the block's draft rows' q, the logits at the
  // drafts and this chunk of the block's rows, all in flight together.
  const int cb = b - nstat, c = cb % nch, rlo = (cb / nch) * kGroupRows, rhi = min(rlo + kGroupRows, rows);
  const int x0 = c * kVocabChunk;
  // arrival: its value depends on the counter value read, so it cannot be
  // posted before that read completed
  if (threadIdx.x == 0) atomic_store_u64(&mb->arrive[cb], ~static_cast<unsigned long long>(call));
  const bool search = K > 0 && a.d2t != nullptr;
  Probe pr[2] = {{0, a.head_rows, 1, 0, 0}, {0, a.head_rows, 1, 0, 0}};
  if (search) {
    probe_issue(a.d2t, pr[0]);
    probe_issue(a.d2t, pr[1]);
  }
  const int dtok = threadIdx.x < K ? a.drafts[threadIdx.x] : 0;
  for (int j = threadIdx.x; j < kVocabChunk; j += kStThreads) qchunk[j] = 0.0;
  int w0 = min(x0, a.head_rows), w1 = min(x0 + kVocabChunk, a.head_rows);
  if (search) {
    probe_apply(pr[0], x0, s_cnt[0][0]);
    probe_apply(pr[1], x0 + kVocabChunk, s_cnt[0][1]);
    w0 = pr[0].lo;           // the chunk's first head row is in [lo, hi] of the first search
    w1 = max(pr[1].hi, w0);  // its end in [lo, hi] of the second
  }
  const int nr = w1 - w0;
  const bool pre = rlo < K && nr <= kQPre;  // the block holds a draft row
  constexpr int kU = kQPre / kStThreads;
  int jv[kU];
  float qv[kU][kGroupRows];
  if (pre) {  // loads at clamped addresses
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int r = min(w0 + static_cast<int>(threadIdx.x) + u * kStThreads, a.head_rows - 1);
      jv[u] = a.d2t ? a.d2t[r] : r;
#pragma unroll
      for (int i = 0; i < kGroupRows; ++i)
        if (rlo + i < K) qv[u][i] = a.q[static_cast<int64_t>(rlo + i) * a.ld_q + r];
    }
  }
  float lgx = 0.f;
  if (threadIdx.x < K) lgx = a.logits[static_cast<int64_t>(threadIdx.x) * a.ld_l + min(max(dtok, 0), a.vocab - 1)];
  // thread t: entries x0 + 16 t .. x0 + 16 t + 15 of each held row (chunk_raw's layout)
  const int xt = x0 + threadIdx.x * kPerThread;
  const bool v4 = vec && xt + kPerThread <= a.vocab;
  float v[kGroupRows][kPerThread];
#pragma unroll
  for (int i = 0; i < kGroupRows; ++i) {
    if (rlo + i < rhi) {
      const float* lr = a.logits + static_cast<int64_t>(rlo + i) * a.ld_l;
      if (v4) {
#pragma unroll
        for (int e4 = 0; e4 < kPerThread / 4; ++e4) {
          const float4 f = reinterpret_cast<const float4*>(lr + xt)[e4];
          v[i][4 * e4] = f.x;
          v[i][4 * e4 + 1] = f.y;
          v[i][4 * e4 + 2] = f.z;
          v[i][4 * e4 + 3] = f.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < kPerThread; ++e) v[i][e] = lr[min(xt + e, a.vocab - 1)];
      }
    }
  }
  if (pre) {  // ids as chunk offsets (-1 outside the window or the chunk) and q into LDS
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      float jf = __int_as_float(jv[u]);
      pin(jf);
      jv[u] = __float_as_int(jf);
#pragma unroll
      for (int i = 0; i < kGroupRows; ++i)
        if (rlo + i < K) pin(qv[u][i]);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = threadIdx.x + u * kStThreads, j = jv[u] - x0;
      s_j[k] = static_cast<short>(k < nr && j >= 0 && j < kVocabChunk ? j : -1);
#pragma unroll
      for (int i = 0; i < kGroupRows; ++i)
        if (rlo + i < K) s_q[i][k] = qv[u][i];
    }
  }
  if (threadIdx.x < K) s_lgx[threadIdx.x] = lgx;
  // ---- wait for every statistics, mass and check word: wave w merges rows w
  // and w + 4, lane l their chunks l, l + 64, ...; thread t < n_other one
  // draft-row / uniform / check word
  const int n_other = 3 * K + 1 + nchecks;
  unsigned long long pw[2][kFusedCpl], ow = 0;
  for (unsigned int it = 0;; ++it) {
    // every word loaded (clamped) before any is tested: one round trip per poll
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < kFusedCpl; ++u)
        pw[h][u] = atomic_load_u64(&mb->part[rep][min(wave + h * kNw, rows - 1)][min(lane + u * kWave, nch - 1)]);
    ow = atomic_load_u64(&mb->other[rep][min(static_cast<int>(threadIdx.x), n_other - 1)]);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < kFusedCpl; ++u) pin(pw[h][u]);
    pin(ow);
    int ok = 1;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int u = 0; u < kFusedCpl; ++u)
        if (wave + h * kNw < rows && lane + u * kWave < nch && pw[h][u] == 0ull) ok = 0;
    if (threadIdx.x < n_other && ow == 0ull) ok = 0;
    if (__syncthreads_and(ok)) break;
    if (it >= a.spin_limit) {
      stoch_give_up(a, ctl);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  // the rows' softmax (max, sum), merged as k_stoch_stats merges them
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = wave + h * kNw;
    if (i >= rows) continue;
    float mc[kFusedCpl], sc[kFusedCpl];
#pragma unroll
    for (int u = 0; u < kFusedCpl; ++u) {
      const unsigned long long w = ~pw[h][u];
      mc[u] = __uint_as_float(static_cast<unsigned int>(w));
      sc[u] = __uint_as_float(static_cast<unsigned int>(w >> 32));
    }
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < kFusedCpl; ++u)
      if (lane + u * kWave < nch) m = fmaxf(m, mc[u]);
    m = wave_max_dpp(m);
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kFusedCpl; ++u)
      if (lane + u * kWave < nch) sum += mc[u] == -INFINITY ? 0.f : sc[u] * expf(mc[u] - m);
    sum = wave_sum_dpp(sum);
    if (lane == 0) {
      s_M[i] = m;
      s_S[i] = sum;
    }
  }
  // s_rd[4 i] = Q_i, s_rd[4 i + 2] = q_i at the draft, s_rd[4 u + 3] = uniform u
  const int t = threadIdx.x;
  if (t < 2 * K) s_rd[4 * (t / 2) + 2 * (t % 2)] = mail_f64(ow);
  else if (t < 3 * K + 1) s_rd[4 * (t - 2 * K) + 3] = mail_f64(ow);
  const bool bad = __syncthreads_or(t >= 3 * K + 1 && t < n_other && ow == 2ull) != 0;
  // The accept tests of decide_rows, every wave at once: lane i < K tests draft
  // i with the uniform it would consume in order (one per earlier draft whose
  // q(x) > 0); the first rejection ends the walk.
  Decision d{K, 0, 0};
  {
    double qx = 0.0;
    bool acc = false;
    if (lane < K) {
      const double Q = s_rd[4 * lane];
      qx = Q > 0.0 ? s_rd[4 * lane + 2] / Q : 0.0;
    }
    const unsigned long long hm = __ballot(lane < K && qx > 0.0);
    if (lane < K && qx > 0.0) {
      const int ui = __popcll(hm & ((1ull << lane) - 1ull));
      const float pf = expf(lscale<P2>(a, s_lgx[lane]) - s_M[lane]) / s_S[lane];
      acc = s_rd[4 * ui + 3] < fmin(1.0, static_cast<double>(pf) / qx);
    }
    const unsigned long long rej = __ballot(lane < K && !acc);
    if (rej) {
      d.n = __ffsll(static_cast<long long>(rej)) - 1;
      d.residual = 1;
      d.n_uniforms = __popcll(hm & ((1ull << d.n) - 1ull)) + static_cast<int>((hm >> d.n) & 1ull);
    } else {
      d.n_uniforms = __popcll(hm);
    }
  }
  if (d.n < rlo || d.n >= rhi) return;  // another block of this chunk holds row n
  const float M = s_M[d.n], S = s_S[d.n];
  const double Q = s_rd[4 * d.n];
  float raw[kPerThread];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) raw[e] = v[0][e];
#pragma unroll
  for (int i = 1; i < kGroupRows; ++i)
    if (rlo + i == d.n)
#pragma unroll
      for (int e = 0; e < kPerThread; ++e) raw[e] = v[i][e];
  // q_n / Q_n scattered over the chunk (chunk_values' arithmetic)
  if (d.residual) {
    if (pre) {
      const float* sq = s_q[d.n - rlo];
      for (int k = threadIdx.x; k < nr; k += kStThreads) {
        const int j = s_j[k];
        if (j >= 0) qchunk[qslot(j)] = static_cast<double>(sq[k]) / Q;
      }
    } else {
      const float* qr = a.q + static_cast<int64_t>(d.n) * a.ld_q;
      for (int r = w0 + threadIdx.x; r < w1; r += kStThreads) {
        const int j = (a.d2t ? a.d2t[r] : r) - x0;
        if (j >= 0 && j < kVocabChunk) qchunk[qslot(j)] = static_cast<double>(qr[r]) / Q;
      }
    }
  }
  lds_barrier();
  double rv[kPerThread], pv[kPerThread];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int j = threadIdx.x * kPerThread + e, x = x0 + j;
    const float pf = expf(lscale<P2>(a, raw[e]) - M) / S;
    const double pd = x < a.vocab ? static_cast<double>(pf) : 0.0;
    pv[e] = pd;
    rv[e] = fmax(pd - qchunk[e * kStThreads + threadIdx.x], 0.0);
  }
  {
    double sr = 0.0, sp = 0.0;
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      sr += rv[e];
      sp += pv[e];
    }
    block_sum2_f64(sr, sp, s_tsum);
    if (threadIdx.x == 0) {
      mail_put_f64(&mb->csum[0][c][0], kCsumRep, sr);
      mail_put_f64(&mb->csum[0][c][1], kCsumRep, sp);
    }
  }

  // ---- every chunk's masses (thread k: chunk k), the totals and the chunk of
  // the draw (k_stoch_sample's arithmetic); the block holding that chunk finishes
  double cr[2] = {0.0, 0.0}, cp[2] = {0.0, 0.0};
  for (unsigned int it = 0;; ++it) {
    const int k = min(static_cast<int>(threadIdx.x), nch - 1);
    unsigned long long wr = atomic_load_u64(&mb->csum[rep][k][0]);
    unsigned long long wp = atomic_load_u64(&mb->csum[rep][k][1]);
    pin(wr);
    pin(wp);
    const int ok = threadIdx.x >= nch || (wr != 0ull && wp != 0ull) ? 1 : 0;
    if (threadIdx.x < nch) {
      cr[0] = mail_f64(wr);
      cp[0] = mail_f64(wp);
    }
    if (__syncthreads_and(ok)) break;
    if (it >= a.spin_limit) {
      stoch_give_up(a, ctl);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  double tot_r = cr[0] + cr[1], tot_p = cp[0] + cp[1];
  block_sum2_f64(tot_r, tot_p, s_tsum);
  const bool use_r = d.residual && tot_r > 1e-12;  // sampling.py:184: residual mass <= 1e-12 -> p
  const double total = use_r ? tot_r : tot_p;
  const double target = s_rd[4 * d.n_uniforms + 3] * total;
  if (nch <= kWave) {
    if (threadIdx.x < kWave) {
      const int k = threadIdx.x;
      const double vk = k < nch ? (use_r ? cr[0] : cp[0]) : 0.0;
      const double ex = block_wave_excl_scan(vk);
      const unsigned long long hit = __ballot(k < nch && ex + vk > target);
      const int cs = hit ? __ffsll(static_cast<long long>(hit)) - 1 : nch - 1;
      if (k == cs) {
        s_chunk = cs;
        s_before = hit ? ex : ex + vk;
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = threadIdx.x + h * kStThreads;
      if (k < nch) qchunk[k] = use_r ? cr[h] : cp[h];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      double run = 0.0;
      int cs = nch - 1;
      for (int k = 0; k < nch; ++k) {
        const double vk = qchunk[k];
        if (run + vk > target) {
          cs = k;
          break;
        }
        run += vk;
      }
      s_chunk = cs;
      s_before = run;
    }
  }
  if (threadIdx.x == 0) s_idx = kVocabChunk;
  __syncthreads();
  if (s_chunk != c) return;
  double tsum = 0.0;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) tsum += use_r ? rv[e] : pv[e];
  double run = block_excl_scan(tsum, s_before, s_tsum);
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
    const int x = min(c * kVocabChunk + s_idx, a.vocab - 1);  // searchsorted clamp (sampling.py:193)
    wc_verdict* vd = a.verdict;
    vd->tokens[d.n] = x;
    vd->keep[d.n] = d.n;
    vd->n_accepted = d.n;
    vd->next = x;
    vd->n_keep = d.n + 1;
    vd->n_uniforms = d.n_uniforms + 1;
    vd->status = bad ? WC_E_INVALID : 0;
  }
  if (threadIdx.x < d.n) {
    a.verdict->tokens[threadIdx.x] = dtok;
    a.verdict->keep[threadIdx.x] = threadIdx.x;
  }
  // the counter moves once every block has read it: the statistics, mass and
  // check blocks' words are in, and every chunk block's arrival
  for (unsigned int it = 0;; ++it) {
    int ok = 1;
    for (int k = threadIdx.x; k < nchunkb; k += kStThreads)
      if (atomic_load_u64(&mb->arrive[k]) == 0ull) ok = 0;
    if (__syncthreads_and(ok)) break;
    if (it >= a.spin_limit) {
      stoch_give_up(a, ctl);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  if (threadIdx.x == 0) atomic_store_u32(reinterpret_cast<unsigned int*>(ctl), call + 1u);
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
  const int32_t* q_rows;    // node v's row of q (NULL: row v), each below q_count
  int q_count;
  const int32_t* count;     // node count on the device (NULL: rows), at most rows
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
  const int t = threadIdx.x;
  const int N = a.count ? *a.count : a.rows;
  const bool n_ok = N >= 1 && N <= a.rows;
  const unsigned long long round = static_cast<unsigned long long>(*a.round_dev);
  if (t == 0) {
    s_bad = n_ok ? 0 : 1;
    s_nu = 0;
  }
  __syncthreads();
  if (n_ok) {  // parents[0] = -1, 0 <= parents[i] < i, tokens inside the vocabulary, d2t ascending
    int bad = 0;
    for (int i = t; i < N; i += kTwThreads) {
      const int par = a.parents[i], tok = a.tokens[i];
      if (i == 0 ? par != -1 : (par < 0 || par >= i)) bad = 1;
      if (tok < 0 || tok >= a.vocab) bad = 1;
      if (a.q_rows && (a.q_rows[i] < 0 || a.q_rows[i] >= a.q_count)) bad = 1;
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
    const float* qr = a.q + static_cast<int64_t>(a.q_rows ? a.q_rows[v] : v) * a.ld_q;
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
  const float* qr = a.q ? a.q + static_cast<int64_t>(a.q_rows ? a.q_rows[v] : v) * a.ld_q : nullptr;
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
    float pxf[kPerThread];  // every load in flight before the first use
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) pxf[e] = pr[min(x0 + t * kPerThread + e, a.vocab - 1)];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) pin(pxf[e]);
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
      const int k = t * kPerThread + e, x = x0 + k;
      double qo;
      val[e] = x < a.vocab ? tree_chain(static_cast<double>(pxf[e]), qchunk[k], x, j, s_x, s_mode, s_div, s_s, qo)
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
  double run = block_excl_scan(tsum, before, s_tsum);
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
  float* part;               // [rows][kMaxVocabChunks][2]
  const uint32_t* kth_key;   // top-k: per row, the order key of the k-th largest scaled logit (NULL: off)
};

__device__ __forceinline__ float scaled(const ProbsArgs& a, float v) { return v / a.temperature; }
// The k-th largest scaled logit's order key of row r, read once per block; 0
// (below every key) when top-k is off.
__device__ __forceinline__ uint32_t kth_order(const ProbsArgs& a, int r) { return a.kth_key ? a.kth_key[r] : 0u; }
// scaled logit x of an entry, or -inf when top-k drops it (x below the k-th largest)
__device__ __forceinline__ float warped(const ProbsArgs& a, uint32_t kth, float raw) {
  const float x = scaled(a, raw);
  return float_order(x) < kth ? -INFINITY : x;
}

// ------------------------------------------------------------------ top-k / top-p warping
//
// Radix select over 32-bit order keys in three digit passes (11, 11, 10 bits),
// one block per row: each pass histograms the digit of the keys that match the
// digits fixed so far, weighted by 1 (top-k) or by the value (top-p, fp64
// sums), and fixes the digit of the bin where the weight of all larger keys
// first reaches the target.  Finds the k-th largest key exactly; for top-p the
// key t of the entry whose inclusive descending-order mass first reaches top_p,
// with the mass G above it and the count of entries equal to it.
constexpr int kRsBins = 2048;
constexpr int kRsPerThread = kRsBins / kStThreads;  // bins per thread

// One pass: digit of the crossing bin; `need` (weight still to cover) and
// `above` (weight of larger keys) are updated.  TOPP: key = bits(p), weight p;
// else key = float_order(logit / T) (the division the softmax kernels use),
// weight 1.  When fp64 rounding leaves the crossing just past the last
// nonempty bin (top-p only), that bin is taken: every remaining entry stays.
// s_w: kStThreads / kWave + 2 doubles.
template <bool TOPP>
__device__ uint32_t rs_pass(const float* row, int n, float temp, int shift, int bits, uint32_t prefix,
                            uint32_t pmask, double& need, double& above, double* s_mass, unsigned* s_cnt,
                            double* s_w, uint32_t* s_digit) {
  const int t = threadIdx.x;
  const uint32_t nb = 1u << bits;
  for (int b = t; b < kRsBins; b += kStThreads) {
    s_mass[b] = 0.0;
    s_cnt[b] = 0u;
  }
  __syncthreads();
  for (int i = t; i < n; i += kStThreads) {
    const float v = row[i];
    const uint32_t key = TOPP ? __float_as_uint(v) : float_order(v / temp);
    if ((key & pmask) == prefix) {
      const uint32_t d = (key >> shift) & (nb - 1);
      if (TOPP) atomicAdd(&s_mass[d], static_cast<double>(v));
      else atomicAdd(&s_cnt[d], 1u);
    }
  }
  __syncthreads();
  // thread t holds bins nb - 1 - (t * per + j), j = 0 .. per - 1 (largest keys first)
  const int per = (static_cast<int>(nb) + kStThreads - 1) / kStThreads;
  double w[kRsPerThread];
  double own = 0.0;
#pragma unroll
  for (int j = 0; j < kRsPerThread; ++j) {
    const int b = static_cast<int>(nb) - 1 - (t * per + j);
    w[j] = (j < per && b >= 0) ? (TOPP ? s_mass[b] : static_cast<double>(s_cnt[b])) : 0.0;
    own += w[j];
  }
  constexpr int kSlot = kStThreads / kWave;
  if (t == 0) s_digit[0] = 0xffffffffu;  // no crossing yet (ordered by the scan's barriers)
  double c = block_excl_scan(own, 0.0, s_w);  // weight of every bin above this thread's
#pragma unroll
  for (int j = 0; j < kRsPerThread; ++j) {
    const int b = static_cast<int>(nb) - 1 - (t * per + j);
    if (j < per && b >= 0 && c < need && c + w[j] >= need) {
      s_digit[0] = static_cast<uint32_t>(b);
      s_w[kSlot] = c;  // weight above the chosen bin
    }
    c += w[j];
  }
  if (t == kStThreads - 1) s_w[kSlot + 1] = c;  // total weight of the pass
  __syncthreads();
  if (s_digit[0] == 0xffffffffu) {  // need beyond the total: the lowest nonempty bin
    __syncthreads();
    if (t == 0) s_digit[1] = 0xffffffffu;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRsPerThread; ++j) {
      const int b = static_cast<int>(nb) - 1 - (t * per + j);
      if (j < per && b >= 0 && w[j] > 0.0) atomicMin(&s_digit[1], static_cast<uint32_t>(b));
    }
    __syncthreads();
    if (t == 0) {
      const uint32_t lo = s_digit[1] == 0xffffffffu ? 0u : s_digit[1];
      s_digit[0] = lo;
      s_w[kSlot] = s_w[kSlot + 1] - (TOPP ? s_mass[lo] : static_cast<double>(s_cnt[lo]));
    }
    __syncthreads();
  }
  const uint32_t d = s_digit[0];
  const double c_above = s_w[kSlot];
  __syncthreads();
  need -= c_above;
  above += c_above;
  return d;
}

// top-k: the order key of the k-th largest logit / T of row blockIdx.x
__global__ __launch_bounds__(kStThreads) void k_topk_key(ProbsArgs a, int k, uint32_t* keys) {
  __shared__ double s_mass[kRsBins];
  __shared__ unsigned s_cnt[kRsBins];
  __shared__ double s_w[kStThreads / kWave + 2];
  __shared__ uint32_t s_digit[2];
  const int r = blockIdx.x;
  const float* row = a.logits + static_cast<int64_t>(r) * a.ld;
  double need = k, above = 0.0;
  uint32_t prefix = 0, pmask = 0;
  const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const uint32_t d = rs_pass<false>(row, a.n, a.temperature, shifts[q], widths[q], prefix, pmask, need, above,
                                      s_mass, s_cnt, s_w, s_digit);
    prefix |= d << shifts[q];
    pmask |= ((1u << widths[q]) - 1u) << shifts[q];
  }
  if (threadIdx.x == 0) keys[r] = prefix;
}

// (max, sum of exp(x - max)) of chunk blockIdx.x of row blockIdx.y
__global__ __launch_bounds__(kStThreads) void k_softmax_part(ProbsArgs a) {
  __shared__ float s_m[kStThreads / kWave], s_s[kStThreads / kWave];
  const int r = blockIdx.y, x0 = blockIdx.x * kVocabChunk;
  const float* lr = a.logits + static_cast<int64_t>(r) * a.ld;
  float v[kPerThread];
  float m = -INFINITY;
  const uint32_t kth = kth_order(a, r);
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) v[e] = lr[min(x0 + e * kStThreads + static_cast<int>(threadIdx.x), a.n - 1)];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) pin(v[e]);  // every load in flight at once
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int x = x0 + e * kStThreads + threadIdx.x;
    v[e] = x < a.n ? warped(a, kth, v[e]) : -INFINITY;
    m = fmaxf(m, v[e]);
  }
  m = wave_max_dpp(m);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  float M = s_m[0];
  for (int w = 1; w < kStThreads / kWave; ++w) M = fmaxf(M, s_m[w]);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) s += v[e] == -INFINITY ? 0.f : expf(v[e] - M);
  s = wave_sum_dpp(s);
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
    m = wave_max_dpp(m);
    float s = 0.f;
    for (int c = threadIdx.x; c < nch; c += kWave) {
      const float mc = pp[2 * c];
      s += mc == -INFINITY ? 0.f : pp[2 * c + 1] * expf(mc - m);
    }
    s = wave_sum_dpp(s);
    if (threadIdx.x == 0) {
      s_M = m;
      s_S = s;
    }
  }
  __syncthreads();
  const float M = s_M, S = s_S;
  const float* lr = a.logits + static_cast<int64_t>(r) * a.ld;
  float* orow = a.out + static_cast<int64_t>(r) * a.ld_out;
  const uint32_t kth = kth_order(a, r);
  float raw[kPerThread];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) raw[e] = lr[min(x0 + e * kStThreads + static_cast<int>(threadIdx.x), a.n - 1)];
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) pin(raw[e]);
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int x = x0 + e * kStThreads + threadIdx.x;
    const float v = warped(a, kth, raw[e]);
    if (x < a.n) orow[x] = v == -INFINITY ? 0.f : expf(v - M) / S;
  }
}

// Rows of at most kSrMax entries (the draft head's 16k trimmed vocabulary): one
// block per row holds the whole row in registers, so the max, the sum of exp
// and the probabilities come from one launch and one read of the logits.
constexpr int kSrThreads = 1024;
constexpr int kSrMax = 16384;
__global__ __launch_bounds__(kSrThreads) void k_softmax_row(ProbsArgs a) {
  constexpr int PER = kSrMax / kSrThreads;
  constexpr int NW = kSrThreads / kWave;
  __shared__ float s_m[NW], s_s[NW];
  const int r = blockIdx.x, t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const float* lr = a.logits + static_cast<int64_t>(r) * a.ld;
  const uint32_t kth = kth_order(a, r);
  float v[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) v[e] = lr[min(e * kSrThreads + t, a.n - 1)];
#pragma unroll
  for (int e = 0; e < PER; ++e) pin(v[e]);  // every load in flight at once
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    v[e] = e * kSrThreads + t < a.n ? warped(a, kth, v[e]) : -INFINITY;
    m = fmaxf(m, v[e]);
  }
  m = wave_max_dpp(m);
  if (lane == 0) s_m[wave] = m;
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w]);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    v[e] = v[e] == -INFINITY ? 0.f : expf(v[e] - M);  // each exp once, kept for the write
    sum += v[e];
  }
  sum = wave_sum_dpp(sum);
  if (lane == 0) s_s[wave] = sum;
  __syncthreads();
  float S = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) S += s_s[w];
  float* orow = a.out + static_cast<int64_t>(r) * a.ld_out;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int x = e * kSrThreads + t;
    if (x < a.n) orow[x] = v[e] / S;
  }
}

// top-p on the written probabilities of row blockIdx.x, in place: keep the
// entries of the descending order (ties: lower index first) whose exclusive
// cumulative mass is below top_p -- every entry above the boundary value t, and
// of the entries equal to t the first ceil((top_p - G) / t) -- then renormalise
// by the kept mass (fp64).
__global__ __launch_bounds__(kStThreads) void k_topp(ProbsArgs a, float top_p) {
  __shared__ double s_mass[kRsBins];
  __shared__ unsigned s_cnt[kRsBins];
  __shared__ double s_w[kStThreads / kWave + 2];
  __shared__ uint32_t s_digit[2];
  const int r = blockIdx.x, t = threadIdx.x, n = a.n;
  float* row = a.out + static_cast<int64_t>(r) * a.ld_out;
  double need = top_p, above = 0.0;
  uint32_t prefix = 0, pmask = 0;
  const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const uint32_t d =
        rs_pass<true>(row, n, 1.f, shifts[q], widths[q], prefix, pmask, need, above, s_mass, s_cnt, s_w, s_digit);
    prefix |= d << shifts[q];
    pmask |= ((1u << widths[q]) - 1u) << shifts[q];
  }
  const uint32_t tk = prefix;  // bits of the boundary value
  const double tv = static_cast<double>(__uint_as_float(tk)), G = above;
  // entries equal to t, each thread over a contiguous index range (index order)
  const int span = (n + kStThreads - 1) / kStThreads;
  const int b0 = min(n, t * span), b1 = min(n, b0 + span);
  double eq = 0.0;
  for (int i = b0; i < b1; ++i) eq += __float_as_uint(row[i]) == tk ? 1.0 : 0.0;
  double rank = block_excl_scan(eq, 0.0, s_w);
  __syncthreads();
  const double keep_eq = tv > 0.0 ? fmax(1.0, ceil((static_cast<double>(top_p) - G) / tv)) : 1.0;
  double kept = 0.0;
  for (int i = b0; i < b1; ++i) {
    const uint32_t k = __float_as_uint(row[i]);
    bool keep = k > tk;
    if (k == tk) {
      keep = rank < keep_eq;
      rank += 1.0;
    }
    if (keep) kept += static_cast<double>(row[i]);
  }
  // kept mass: per-thread sums in index order, then the threads in order
  const double before = block_excl_scan(kept, 0.0, s_w);
  __syncthreads();
  __shared__ double s_tot;
  if (t == kStThreads - 1) s_tot = before + kept;
  __syncthreads();
  const double tot = s_tot;
  rank = block_excl_scan(eq, 0.0, s_w);
  for (int i = b0; i < b1; ++i) {
    const float v = row[i];
    const uint32_t k = __float_as_uint(v);
    bool keep = k > tk;
    if (k == tk) {
      keep = rank < keep_eq;
      rank += 1.0;
    }
    row[i] = keep ? static_cast<float>(static_cast<double>(v) / tot) : 0.f;
  }
}

// Blocks of k_stoch_fused the current device holds at once (occupancy per CU
// times the CUs), queried once per device.
static int fused_capacity(int* hold) {
  static std::atomic<int> cache[64];
  int dev = 0;
  WC_HIP(hipGetDevice(&dev));
  int n = dev >= 0 && dev < 64 ? cache[dev].load(std::memory_order_relaxed) : 0;
  if (n == 0) {
    int cus = 0, per_cu = 0;
    if (device_cus(&cus) != WC_OK) return WC_E_HIP;
    int per_cu2 = 0;
    WC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_stoch_fused<false>, kStThreads, 0));
    WC_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu2, k_stoch_fused<true>, kStThreads, 0));
    per_cu = std::min(per_cu, per_cu2);
    n = cus * per_cu;
    if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  }
  *hold = n;
  return WC_OK;
}

}  // namespace wc

namespace wc {

// Both tree entry points: q_rows / count NULL read node v's q at row v and
// take `rows` nodes.
static int tree_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, const int32_t* q_rows,
                           int q_count, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                           const int32_t* tree_tokens_dev, const int32_t* tree_parents_dev, const int32_t* count_dev,
                           const wc_uniforms* rng, wc_verdict* verdict_dev, void* workspace, wc_stream_t stream,
                           const char* fn) {
  WC_REQUIRE(p && tree_tokens_dev && tree_parents_dev && verdict_dev && rng && rng->round_dev, "%s: NULL buffer", fn);
  WC_REQUIRE(workspace && aligned(workspace, 16), "%s: workspace is NULL or misaligned", fn);
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "%s: rows must be in 1..%d (got %d)", fn, WC_MAX_NODES, rows);
  WC_REQUIRE(vocab >= 1 && vocab <= kVocabChunk * kMaxVocabChunks, "%s: vocab %d out of range", fn, vocab);
  WC_REQUIRE(ld_p >= vocab, "%s: p row stride smaller than vocab", fn);
  const bool any_q = rows > 1 || count_dev != nullptr;
  WC_REQUIRE(!any_q || (q && head_rows >= 1 && ld_q >= head_rows), "%s: bad draft distribution buffer / width / stride",
             fn);
  WC_REQUIRE(d2t_dev != nullptr || head_rows <= vocab,
             "%s: without d2t the draft distribution must not exceed the vocabulary", fn);
  TreeArgs a{};
  a.p = p;
  a.rows = rows;
  a.vocab = vocab;
  a.ld_p = ld_p;
  a.q = q;
  a.head_rows = any_q ? head_rows : 0;
  a.ld_q = ld_q;
  a.q_rows = q_rows;
  a.q_count = q_count;
  a.count = count_dev;
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

}  // namespace wc

extern "C" {

int wc_probs_from_logits(const float* logits, int rows, int n, int64_t ld, float temperature, int top_k, float top_p,
                         float* out, int64_t ld_out, void* workspace, wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(logits && out, "wc_probs_from_logits: NULL buffer");
  WC_REQUIRE(top_k >= 0, "wc_probs_from_logits: top_k must be >= 0 (0 = off), got %d", top_k);
  WC_REQUIRE(top_p > 0.f && top_p <= 1.f, "wc_probs_from_logits: top_p must be in (0, 1] (1 = off), got %g",
             static_cast<double>(top_p));
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
  a.kth_key = nullptr;
  const dim3 grid((n + kVocabChunk - 1) / kVocabChunk, rows);
  auto s = reinterpret_cast<hipStream_t>(stream);
  if (top_k > 0 && top_k < n) {  // sampling.py:41-43: x < the k-th largest x -> -inf
    uint32_t* keys = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kWarpOff);
    hipLaunchKernelGGL(k_topk_key, dim3(rows), dim3(kStThreads), 0, s, a, top_k, keys);
    WC_LAUNCHED();
    a.kth_key = keys;
  }
  if (n <= kSrMax && top_p >= 1.f) {  // the draft head's width: one launch, a block per row
    hipLaunchKernelGGL(k_softmax_row, dim3(rows), dim3(kSrThreads), 0, s, a);
    WC_LAUNCHED();
    return WC_OK;
  }
  hipLaunchKernelGGL(k_softmax_part, grid, dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL(k_softmax_write, grid, dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  if (top_p < 1.f) {  // sampling.py:45-54
    hipLaunchKernelGGL(k_topp, dim3(rows), dim3(kStThreads), 0, s, a, top_p);
    WC_LAUNCHED();
  }
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
  a.chunk_rows = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + kChunkRowsOff);
  a.counter = verify_counter(workspace, kCtrStochastic);
  a.verdict = verdict_dev;
  auto s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_stoch_rows, dim3(rows), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL((k_stoch_sample<false>), dim3((vocab + kVocabChunk - 1) / kVocabChunk), dim3(kStThreads), 0, s,
                     a);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_verify_chain_stochastic_logits(const float* logits, int rows, int vocab, int64_t ld, float temperature,
                                      const float* q, int head_rows, int64_t ld_q, const int32_t* d2t_dev,
                                      const int32_t* draft_tokens_dev, const int32_t* draft_rows_dev,
                                      const wc_uniforms* rng, wc_verdict* verdict_dev, void* workspace,
                                      wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(logits && verdict_dev && rng && rng->round_dev, "wc_verify_chain_stochastic_logits: NULL buffer");
  WC_REQUIRE(workspace && aligned(workspace, 16),
             "wc_verify_chain_stochastic_logits: workspace is NULL or misaligned");
  WC_REQUIRE(rows >= 1 && rows <= WC_MAX_NODES, "wc_verify_chain_stochastic_logits: rows must be in 1..%d (got %d)",
             WC_MAX_NODES, rows);
  WC_REQUIRE(vocab >= 1 && vocab <= kVocabChunk * kMaxVocabChunks,
             "wc_verify_chain_stochastic_logits: vocab %d out of range", vocab);
  WC_REQUIRE(ld >= vocab, "wc_verify_chain_stochastic_logits: logits row stride smaller than vocab");
  WC_REQUIRE(rows == 1 || (q && draft_tokens_dev),
             "wc_verify_chain_stochastic_logits: draft probabilities or tokens NULL");
  WC_REQUIRE(rows == 1 || (head_rows >= 1 && ld_q >= head_rows),
             "wc_verify_chain_stochastic_logits: bad draft distribution width / stride");
  WC_REQUIRE(d2t_dev != nullptr || head_rows <= vocab,
             "wc_verify_chain_stochastic_logits: without d2t the draft distribution must not exceed the vocabulary");
  StochArgs a{};
  a.rows = rows;
  a.vocab = vocab;
  a.q = q;
  a.head_rows = head_rows;
  a.ld_q = ld_q;
  a.d2t = d2t_dev;
  a.drafts = draft_tokens_dev;
  a.draft_rows = draft_rows_dev;
  a.seed = rng->seed;
  a.round_dev = rng->round_dev;
  a.purpose = rng->purpose;
  char* ws = static_cast<char*>(workspace);
  a.row_data = reinterpret_cast<double*>(ws + kStochRowOff);
  a.chunk_data = reinterpret_cast<double*>(ws + kStochChunkOff);
  a.chunk_rows = reinterpret_cast<int32_t*>(ws + kChunkRowsOff);
  a.counter = verify_counter(workspace, kCtrStochastic);
  a.stats_counter = verify_counter(workspace, kCtrStochStats);
  a.verdict = verdict_dev;
  a.logits = logits;
  a.ld_l = ld;
  a.temperature = temperature > 1e-6f ? temperature : 1e-6f;  // max(T, 1e-6), sampling.py:40
  a.part = reinterpret_cast<float*>(ws + kProbsOff);
  a.dec = reinterpret_cast<int32_t*>(ws + kStochDecOff);
  a.dec_ms = reinterpret_cast<float*>(ws + kStochDecOff + 16);
  a.bad_flag = reinterpret_cast<unsigned int*>(ws + kStochDecOff + 32);
  const int nch = (vocab + kVocabChunk - 1) / kVocabChunk;
  auto s = reinterpret_cast<hipStream_t>(stream);
  // check blocks: a d2t slice each, and one per draft for its head-row lookup
  const int ncheck = std::max(rows - 1, d2t_dev ? std::min(32, std::max(1, (head_rows + 1023) / 1024)) : 1);
  const int groups = (rows + kGroupRows - 1) / kGroupRows;
  const int grid = rows * nch + groups * nch + (rows - 1) + ncheck;
  int hold = 0;
  if (fused_capacity(&hold) != WC_OK) return WC_E_HIP;
  // only the chunk blocks wait for other blocks: they must fit at once; the
  // other blocks never wait, so they run whenever a slot frees
  if (rows <= kFusedRows && nch <= kMailChunks && groups * nch < hold) {
    MailSet* sets = reinterpret_cast<MailSet*>(ws + kGridBarOff);
    auto* ctl = reinterpret_cast<unsigned long long*>(ws + kGridBarOff + 2 * sizeof(MailSet));
    a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
    const int vec = aligned(logits, 16) && ld % 4 == 0;
    int e2 = 0;
    const bool p2 = std::frexp(a.temperature, &e2) == 0.5f;  // T = 2^(e2 - 1)
    if (p2) {
      a.inv_t = std::ldexp(1.0f, 1 - e2);
      hipLaunchKernelGGL(k_stoch_fused<true>, dim3(grid), dim3(kStThreads), 0, s, a, nch, ncheck, vec, sets, ctl);
    } else {
      hipLaunchKernelGGL(k_stoch_fused<false>, dim3(grid), dim3(kStThreads), 0, s, a, nch, ncheck, vec, sets, ctl);
    }
    WC_LAUNCHED();
    return WC_OK;
  }
  // two launches; the extra row needs K draft-mass blocks plus at least one check block
  hipLaunchKernelGGL(k_stoch_stats, dim3(std::max(nch, rows), rows + 1), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  hipLaunchKernelGGL((k_stoch_sample<true>), dim3(nch), dim3(kStThreads), 0, s, a);
  WC_LAUNCHED();
  return WC_OK;
}

int wc_set_spin_limit(int polls) {
  wc::g_spin_limit.store(polls < 0 ? wc::kSpinLimit : static_cast<unsigned int>(polls), std::memory_order_relaxed);
  return WC_OK;
}

int wc_verify_tree_stochastic(const float* p, int rows, int vocab, int64_t ld_p, const float* q, int head_rows,
                              int64_t ld_q, const int32_t* d2t_dev, const int32_t* tree_tokens_dev,
                              const int32_t* tree_parents_dev, const wc_uniforms* rng, wc_verdict* verdict_dev,
                              void* workspace, wc_stream_t stream) {
  return wc::tree_stochastic(p, rows, vocab, ld_p, q, nullptr, 0, head_rows, ld_q, d2t_dev, tree_tokens_dev,
                             tree_parents_dev, nullptr, rng, verdict_dev, workspace, stream, "wc_verify_tree_stochastic");
}

int wc_verify_tree_stochastic_indexed(const float* p, int rows, int vocab, int64_t ld_p, const float* q,
                                      int q_count, const int32_t* q_rows_dev, int head_rows, int64_t ld_q,
                                      const int32_t* d2t_dev, const int32_t* tree_tokens_dev,
                                      const int32_t* tree_parents_dev, const int32_t* count_dev,
                                      const wc_uniforms* rng, wc_verdict* verdict_dev, void* workspace,
                                      wc_stream_t stream) {
  using namespace wc;
  WC_REQUIRE(q && q_rows_dev && count_dev, "wc_verify_tree_stochastic_indexed: NULL buffer");
  WC_REQUIRE(q_count >= 1, "wc_verify_tree_stochastic_indexed: q_count must be positive");
  return tree_stochastic(p, rows, vocab, ld_p, q, q_rows_dev, q_count, head_rows, ld_q, d2t_dev, tree_tokens_dev,
                         tree_parents_dev, count_dev, rng, verdict_dev, workspace, stream,
                         "wc_verify_tree_stochastic_indexed");
}

}  // extern "C"
