// gemv.h -- batch-M streaming bf16 GEMV for gfx950 (M <= 16 input rows).
//
//   y[m][n] = sum_s sum_k W_s[n][k] * xhat_s[m][k]        for m < M, n < N
//   xhat_s[m] = RMSNorm(x_s[m]) * gain_s   (or x_s[m] when the segment has no gain)
//
// Design (HBM-streaming, one pass over W):
//   - a 256-thread block = 4 waves; each wave owns R consecutive output rows
//     (x2 physical rows for the gate/up pair epilogue); every lane reads 8
//     consecutive bf16 weights (one 128-bit load) per 512-wide K step, so each
//     load instruction of a wave covers 1 KB of one weight row, fully coalesced;
//   - the (normalised) fp32 inputs of all M rows are staged in LDS once per
//     block and K chunk; the RMSNorm sum of squares is a block reduction over
//     the same rows (fp32), applied as x * inv * gain like the reference
//     (src/backends/cpu_ops.cpp:50-59);
//   - U K-steps of every row are loaded before the first FMA so each lane
//     keeps R*U 128-bit loads in flight;
//   - fp32 accumulation, wave reduction with cross-lane shuffles.
// Epilogues: plain store, residual add, SiLU(gate)*up of paired rows
// (cpu_ops.cpp:79-84), and argmax over the rows (packed-key device atomics)
// with a last-block finalisation that maps the winning row through d2t.
#pragma once

#include "wc_common.h"

namespace wc {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kMaxM = 16;
constexpr int kMaxIn = 3;
constexpr int kMaxSeg = 3;
constexpr int kGemvLdsBytes = 48 * 1024;

struct InSeg {
  const void* x;           // [rows][ld] fp32 or bf16
  int64_t ld;              // row stride in elements
  int dtype;               // WC_F32 / WC_BF16
  const int32_t* row_idx;  // optional: input row m reads x row row_idx[m] + row_add
  int row_add;
  const uint16_t* gain;    // RMSNorm gain [K] (bf16) or NULL: no norm
  int K;                   // multiple of 8
  int max_row;             // > 0: gathered rows are clamped to [0, max_row)
};

enum Epi { kEpiStore = 0, kEpiResidual = 1, kEpiSiluPair = 2, kEpiArgmax = 3 };

struct Gumbel {
  unsigned long long seed;
  const int32_t* round_dev;  // round index read on device
  int purpose;
  float inv_temperature;
};

struct GemvArgs {
  InSeg in[kMaxIn];
  int n_in;
  int64_t ldw[kMaxIn];                     // weight row stride per input segment
  const uint16_t* w[kMaxSeg][kMaxIn];      // per row-segment, per input segment: row 0 of the segment
  int seg_start[kMaxSeg + 1];              // logical-row segment boundaries (seg_start[n_seg] = N)
  int n_seg;
  int N;                                   // logical output rows
  int M;                                   // input rows handled by this launch (<= kMaxM)
  const int32_t* m_dev;                    // optional device row count (<= M)
  float eps;
  int epi;
  float* y;                                // [M][ldy] (store / residual / pair; optional for argmax)
  int64_t ldy;
  const float* res;                        // residual [M][ldres]
  int64_t ldres;
  const int32_t* res_row_idx;              // optional: residual row m is res_row_idx[m] + res_row_add
  int res_row_add;
  // argmax epilogue
  unsigned long long* slots;               // [M] packed keys, zero on entry, zeroed on exit
  unsigned int* counter;                   // zero on entry, zeroed on exit
  const int32_t* d2t;                      // head row -> token id (NULL = identity)
  int32_t* tok_out;                        // [M] token ids
  int32_t* row_out;                        // [M] winning rows (optional)
  int use_gumbel;
  Gumbel gumbel;
  // last-block epilogue: final RMSNorm of y rows into fin_out, and an offset advance
  const uint16_t* fin_gain;
  float* fin_out;
  int64_t ld_fin;
  unsigned int* fin_counter;
  const int32_t* adv_src;                  // *adv_dst = *adv_src + adv_add + (m rows) when adv_dst != NULL
  int adv_add;
  int32_t* adv_dst;
};

__device__ __forceinline__ float dot8(const uint4 w, const float4 a, const float4 b) {
  float s = bf16_lo(w.x) * a.x;
  s = fmaf(bf16_hi(w.x), a.y, s);
  s = fmaf(bf16_lo(w.y), a.z, s);
  s = fmaf(bf16_hi(w.y), a.w, s);
  s = fmaf(bf16_lo(w.z), b.x, s);
  s = fmaf(bf16_hi(w.z), b.y, s);
  s = fmaf(bf16_lo(w.w), b.z, s);
  s = fmaf(bf16_hi(w.w), b.w, s);
  return s;
}

__device__ __forceinline__ float load_in(const InSeg& s, int64_t row, int k) {
  const int64_t i = row * s.ld + k;
  return s.dtype == WC_BF16 ? bf16_to_float(static_cast<const uint16_t*>(s.x)[i]) : static_cast<const float*>(s.x)[i];
}

__device__ __forceinline__ int in_row(const InSeg& s, int m) {
  int r = (s.row_idx ? s.row_idx[m] : m) + s.row_add;
  if (s.max_row > 0) r = min(max(r, 0), s.max_row - 1);
  return r;
}

// Philox4x64-10 (Salmon et al., SC'11): same stream as the host oracle.
__device__ __forceinline__ void philox4x64(unsigned long long c[4], unsigned long long k0, unsigned long long k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B97F4A7C15ull;
      k1 += 0xBB67AE8584CAA73Bull;
    }
    const unsigned long long lo0 = 0xD2E7470EE14C6C93ull * c[0], hi0 = __umul64hi(0xD2E7470EE14C6C93ull, c[0]);
    const unsigned long long lo1 = 0xCA5A826395121157ull * c[2], hi1 = __umul64hi(0xCA5A826395121157ull, c[2]);
    const unsigned long long n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

// uniform i of (seed, round, purpose): counter (i/4, round, purpose, 0), key (seed, 0), word i%4
__device__ __forceinline__ double philox_uniform(unsigned long long seed, unsigned long long round, int purpose,
                                                 unsigned long long i) {
  unsigned long long c[4] = {i >> 2, round, static_cast<unsigned long long>(purpose), 0ull};
  philox4x64(c, seed, 0ull);
  return static_cast<double>(c[i & 3] >> 11) * (1.0 / 9007199254740992.0);
}

// Stage rows [0, m) x chunk [c0, c0+kc) of input segment s into LDS as x*inv*gain.
__device__ __forceinline__ void stage_chunk(const InSeg& s, int m, int c0, int kc, int ldk, const float* inv,
                                            float* xs) {
  for (int mi = 0; mi < m; ++mi) {
    const int64_t row = in_row(s, mi);
    for (int k = threadIdx.x; k < kc; k += kGemvThreads) {
      float v = load_in(s, row, c0 + k);
      if (s.gain) v = v * inv[mi] * bf16_to_float(s.gain[c0 + k]);
      xs[mi * ldk + k] = v;
    }
  }
}

// inv[mi] = 1 / sqrt(mean(x^2) + eps) for rows [0, m) of segment s (block reduction).
__device__ __forceinline__ void row_inv_norms(const InSeg& s, int m, float eps, float* inv, float* red) {
  for (int mi = 0; mi < m; ++mi) {
    const int64_t row = in_row(s, mi);
    float ss = 0.f;
    for (int k = threadIdx.x; k < s.K; k += kGemvThreads) {
      const float v = load_in(s, row, k);
      ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x % kWave) == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int w = 0; w < kGemvWaves; ++w) t += red[w];
      inv[mi] = 1.f / sqrtf(t / static_cast<float>(s.K) + eps);
    }
    __syncthreads();
  }
}

template <int R, int MM, bool PAIR, int U>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(GemvArgs a) {
  constexpr int P = PAIR ? 2 : 1;
  extern __shared__ float smem[];
  __shared__ float s_inv[kMaxIn][kMaxM];
  __shared__ float s_red[kGemvWaves];
  __shared__ unsigned long long s_key[kGemvWaves][MM];

  int m = a.M;
  if (a.m_dev) m = min(max(*a.m_dev, 0), a.M);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;

  // per-segment RMS norms of every input row
  for (int s = 0; s < a.n_in; ++s)
    if (a.in[s].gain) row_inv_norms(a.in[s], m, a.eps, s_inv[s], s_red);

  // (segment, offset) of this wave's rows; physical row p of a PAIR row n is row n of segment p
  int rseg[R][P], roff[R][P];
  bool valid[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = row0 + r;
    valid[r] = n < a.N;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      int seg = p, off = n;
      if (!PAIR) {
        seg = 0;
        for (int j = 1; j < a.n_seg; ++j)
          if (n >= a.seg_start[j]) seg = j;
        off = n - a.seg_start[seg];
      }
      rseg[r][p] = seg;
      roff[r][p] = off;
    }
  }

  float acc[R][P][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = 0.f;

  const int lds_floats = kGemvLdsBytes / 4;
  for (int s = 0; s < a.n_in; ++s) {
    const InSeg seg = a.in[s];
    const uint16_t* wrow[R][P];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p)
        wrow[r][p] = valid[r] ? a.w[rseg[r][p]][s] + static_cast<int64_t>(roff[r][p]) * a.ldw[s] : nullptr;
    int kcap = lds_floats / (m > 0 ? m : 1);
    kcap = kcap / 512 * 512;
    if (kcap < 512) kcap = 512;
    for (int c0 = 0; c0 < seg.K; c0 += kcap) {
      const int kc = min(kcap, seg.K - c0);
      __syncthreads();  // previous chunk fully consumed
      stage_chunk(seg, m, c0, kc, kc, s_inv[s], smem);
      __syncthreads();
      for (int k = lane * 8; k < kc; k += kWave * 8 * U) {
        uint4 w[R][P][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int kk = k + u * kWave * 8;
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int p = 0; p < P; ++p)
              w[r][p][u] = (valid[r] && kk < kc) ? *reinterpret_cast<const uint4*>(wrow[r][p] + c0 + kk)
                                                 : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int kk = k + u * kWave * 8;
          if (kk < kc) {
#pragma unroll
            for (int mi = 0; mi < MM; ++mi) {
              if (mi < m) {
                const float4 x0 = *reinterpret_cast<const float4*>(smem + mi * kc + kk);
                const float4 x1 = *reinterpret_cast<const float4*>(smem + mi * kc + kk + 4);
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                  for (int p = 0; p < P; ++p) acc[r][p][mi] += dot8(w[r][p][u], x0, x1);
              }
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = wave_sum(acc[r][p][mi]);

  if (a.epi != kEpiArgmax) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (!valid[r]) continue;
        const int n = row0 + r;
#pragma unroll
        for (int mi = 0; mi < MM; ++mi) {
          if (mi >= m) continue;
          float v = acc[r][0][mi];
          if (PAIR) {
            const float g = acc[r][0][mi], u = acc[r][P - 1][mi];
            v = g / (1.f + expf(-g)) * u;
          } else if (a.epi == kEpiResidual) {
            const int64_t rr = (a.res_row_idx ? a.res_row_idx[mi] : mi) + a.res_row_add;
            v = a.res[rr * a.ldres + n] + v;
          }
          a.y[mi * a.ldy + n] = v;
        }
      }
    }
    // optional last-block epilogue: final RMSNorm of the produced rows, offset advance
    if (a.fin_counter) {
      if (!last_block_done(a.fin_counter, gridDim.x)) return;
      if (a.fin_gain) {
        for (int mi = 0; mi < m; ++mi) {
          float ss = 0.f;
          for (int k = threadIdx.x; k < a.N; k += kGemvThreads) {
            const float v = a.y[mi * a.ldy + k];
            ss = fmaf(v, v, ss);
          }
          ss = wave_sum(ss);
          if (lane == 0) s_red[wave] = ss;
          __syncthreads();
          float t = 0.f;
          for (int w = 0; w < kGemvWaves; ++w) t += s_red[w];
          const float inv = 1.f / sqrtf(t / static_cast<float>(a.N) + a.eps);
          for (int k = threadIdx.x; k < a.N; k += kGemvThreads)
            a.fin_out[mi * a.ld_fin + k] = a.y[mi * a.ldy + k] * inv * bf16_to_float(a.fin_gain[k]);
          __syncthreads();
        }
      }
      if (threadIdx.x == 0) {
        if (a.adv_dst) *a.adv_dst = *a.adv_src + a.adv_add + m;
        atomic_store_u32(a.fin_counter, 0u);
      }
    }
    return;
  }

  // ---- argmax epilogue (draft head): per-wave keys -> per-block -> device atomics
  if (lane == 0) {
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      unsigned long long best = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (!valid[r] || mi >= m) continue;
        const int n = row0 + r;
        float z = acc[r][0][mi];
        if (a.y) a.y[mi * a.ldy + n] = z;
        if (a.use_gumbel) {
          // Gumbel-max draw: argmax z/T - log(-log u) == a draw from softmax(z/T)
          // (python/woodcock/sampling.py:196-203 with one uniform per head row)
          const double u = philox_uniform(a.gumbel.seed, static_cast<unsigned long long>(*a.gumbel.round_dev),
                                          a.gumbel.purpose + mi, static_cast<unsigned long long>(n));
          z = static_cast<float>(static_cast<double>(z) * a.gumbel.inv_temperature - log(-log(u)));
        }
        const unsigned long long key = argmax_key(z, n);
        best = key > best ? key : best;
      }
      s_key[wave][mi] = best;
    }
  }
  __syncthreads();
  if (threadIdx.x < MM && static_cast<int>(threadIdx.x) < m) {
    unsigned long long best = 0;
    for (int w = 0; w < kGemvWaves; ++w) best = s_key[w][threadIdx.x] > best ? s_key[w][threadIdx.x] : best;
    atomic_max_u64(&a.slots[threadIdx.x], best);
  }
  if (!last_block_done(a.counter, gridDim.x)) return;
  if (threadIdx.x < MM && static_cast<int>(threadIdx.x) < m) {
    const unsigned long long k = atomic_load_u64(&a.slots[threadIdx.x]);
    atomic_store_u64(&a.slots[threadIdx.x], 0ull);
    const int row = argmax_key_index(k);
    a.tok_out[threadIdx.x] = a.d2t ? a.d2t[row] : row;
    if (a.row_out) a.row_out[threadIdx.x] = row;
  }
  if (threadIdx.x == 0) atomic_store_u32(a.counter, 0u);
}

}  // namespace wc
