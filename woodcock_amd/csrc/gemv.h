// gemv.h -- batch-M streaming bf16 GEMV for gfx950 (M <= 16 input rows).
//
//   y[m][n] = sum_s sum_k W_s[n][k] * xhat_s[m][k]        for m < M, n < N
//   xhat_s[m] = RMSNorm(x_s[m]) * gain_s   (or x_s[m] when the segment has no gain)
//
// The weights are read exactly once, with 128-bit loads: a 256-thread block is
// 4 waves, each wave owns R consecutive output rows (x2 physical rows for the
// gate/up pair epilogue), and lane j reads bf16 k = 8j..8j+7 of every 512-wide
// step, so one load instruction of a wave covers 1 KB of one weight row.
//
// M = 1 (the draft step): k_gemv1 keeps everything in registers.  Every weight
// load of every input segment is issued first; the lane then loads its own x
// slices (the same k positions as its weights), and the RMSNorm sum of squares
// is a wave reduction -- a wave's lanes tile the whole row -- so there is no
// LDS and no barrier between the first weight byte requested and the FMAs.
// The norm scale is applied after the dot product (sum W (x g) * inv).
//
// M > 1 (the update over a+1 accepted tokens): k_gemvm stages x * gain of all
// rows in LDS per K chunk with 128-bit accesses, accumulating the sums of
// squares in the same pass, requests the first weight group before staging,
// and applies each row's 1/rms to the partial dot products at the end.
//
// Epilogues: plain store, residual add, SiLU(gate)*up of paired rows
// (cpu_ops.cpp:79-84), argmax over rows (packed (value, lowest index) keys,
// device-scope atomicMax spread over kSlots addresses, last block maps the winner
// through d2t), and a last-block final RMSNorm of the produced rows.
#pragma once

#include "wc_common.h"

namespace wc {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kMaxM = 16;
constexpr int kMaxIn = 3;
constexpr int kMaxSeg = 3;
constexpr int kGemvLdsBytes = 48 * 1024;
constexpr int kMaxSteps1 = 24;   // M=1 kernel: up to 24 x 512 = 12288 inputs per segment

struct InSeg {
  const void* x;           // [rows][ld] fp32 or bf16
  int64_t ld;              // row stride in elements
  int dtype;               // WC_F32 / WC_BF16
  const int32_t* row_idx;  // optional: input row m reads x row row_idx[m] + row_add
  int row_add;
  const uint16_t* gain;    // RMSNorm gain [K] (bf16) or NULL: no norm
  int K;                   // multiple of 8
  int max_row;             // > 0: gathered rows are clamped to [0, max_row)
  // optional (one input row): the row is the token of a pending draft-head
  // argmax -- the largest of the kSlots keys at pend_slots (stride
  // kSlotStride), its head row mapped through pend_d2t (NULL = identity)
  const unsigned long long* pend_slots;
  const int32_t* pend_d2t;
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
  int lds_floats;                          // dynamic LDS of the M>1 kernel
  float* y;                                // [M][ldy] (store / residual / pair; optional for argmax)
  int64_t ldy;
  const float* res;                        // residual [M][ldres]
  int64_t ldres;
  const int32_t* res_row_idx;              // optional: residual row m is res_row_idx[m] + res_row_add
  int res_row_add;
  // argmax epilogue
  unsigned long long* slots;               // [M][kSlots] keys (stride kSlotStride), zero on entry and exit
  unsigned int* counter;                   // tree counter (kTreeCounterBytes), zero on entry and exit
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
  // staged few-row kernel split over k: per (tile, piece) partials and per-tile
  // counters (zero on entry and exit); NULL = no split
  float* gs_part;
  unsigned int* gs_ctr;
  // one-row kernel: the normalised input segment 0 (x * gain / rms) written to
  // xn_out at the input's row index by block 0 (the drafter output `out`)
  float* xn_out;
  int64_t ld_xn;
  // w[][] hold fragment-major matrices (wc_weights_frag): only the few-row MFMA
  // kernel reads that layout
  int wfrag;
  // a segment with pend_slots: block 0 also writes the resolved token and head
  // row (one-row kernel only)
  int32_t* pend_tok_out;
  int32_t* pend_row_out;
  // 2..8 input rows on the few-row MFMA kernel rather than the vector-ALU one
  // (wide matrices: a draft head storing its logits)
  int few_mfma;
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

// acc + w . (a, b) as one running fma chain
__device__ __forceinline__ float dot8_acc(const uint4 w, const float4 a, const float4 b, float s) {
  s = fmaf(bf16_lo(w.x), a.x, s);
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

// Head row of the pending argmax: the largest key over the slots (each a
// device-scope maximum of block keys written by the head launch before this
// one), read with one wave-wide load (lane j: slot j) and reduced across the
// wave.  Every lane of the wave must call it.
__device__ __forceinline__ unsigned long long pend_key(const unsigned long long* slots) {
  return slots[min(static_cast<int>(threadIdx.x % kWave), kSlots - 1) * kSlotStride];
}
__device__ __forceinline__ int pend_reduce(unsigned long long best) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const unsigned long long v = __shfl_xor(best, o);
    best = v > best ? v : best;
  }
  return __builtin_amdgcn_readfirstlane(argmax_key_index(best));
}
__device__ __forceinline__ int pend_head_row(const unsigned long long* slots) { return pend_reduce(pend_key(slots)); }
__device__ __forceinline__ int pend_token(const InSeg& s, int head_row) {
  int r = s.pend_d2t ? s.pend_d2t[head_row] : head_row;
  if (s.max_row > 0) r = min(max(r, 0), s.max_row - 1);
  return r;
}

// Input row m of segment s (every lane of the wave calls it).
__device__ __forceinline__ int in_row(const InSeg& s, int m) {
  if (s.pend_slots) return pend_token(s, pend_head_row(s.pend_slots));
  int r = (s.row_idx ? s.row_idx[m] : m) + s.row_add;
  if (s.max_row > 0) r = min(max(r, 0), s.max_row - 1);
  return r;
}

// (segment, offset) of logical row n; PAIR rows live in segments 0 and 1 at offset n
template <bool PAIR>
__device__ __forceinline__ void row_segment(const GemvArgs& a, int n, int p, int& seg, int& off) {
  if (PAIR) {
    seg = p;
    off = n;
    return;
  }
  seg = 0;
  for (int j = 1; j < a.n_seg; ++j)
    if (n >= a.seg_start[j]) seg = j;
  off = n - a.seg_start[seg];
}

// Weight row pointer of logical row n (pair member p) for input segment s,
// resolved with constant indices only so that a wave-uniform n keeps the whole
// lookup in scalar registers.
template <bool PAIR>
__device__ __forceinline__ const uint16_t* row_ptr(const GemvArgs& a, int n, int p, int s) {
  if (PAIR) return (p ? a.w[1][s] : a.w[0][s]) + static_cast<int64_t>(n) * a.ldw[s];
  const uint16_t* base = a.w[0][s];
  int start = 0;
#pragma unroll
  for (int j = 1; j < kMaxSeg; ++j)
    if (j < a.n_seg && n >= a.seg_start[j]) {
      base = a.w[j][s];
      start = a.seg_start[j];
    }
  return base + static_cast<int64_t>(n - start) * a.ldw[s];
}

// ------------------------------------------------------------------ shared epilogues

// Residual input of output (mi, n), in two steps so that kernels can request
// every row index first and every value later, none waiting on another:
// res_row() the residual row of input row mi, res_at() the value (0 when the
// epilogue has no residual).  Addresses are wave-uniform: every lane reads.
__device__ __forceinline__ int res_row(const GemvArgs& a, int mi) {
  return (a.epi == kEpiResidual && a.res_row_idx ? a.res_row_idx[mi] : mi) + a.res_row_add;
}
__device__ __forceinline__ float res_at(const GemvArgs& a, int row, int n) {
  return a.epi == kEpiResidual ? a.res[static_cast<int64_t>(row) * a.ldres + n] : 0.f;
}
__device__ __forceinline__ float res_value(const GemvArgs& a, int mi, int n) { return res_at(a, res_row(a, mi), n); }

// Store / residual / pair epilogue for one output value (res from res_value);
// published (device coherent) when a last-block epilogue will read it back.
template <bool PAIR>
__device__ __forceinline__ void store_out(const GemvArgs& a, int mi, int n, float g, float u, float res) {
  float v = g;
  if (PAIR)
    v = g / (1.f + expf(-g)) * u;
  else if (a.epi == kEpiResidual)
    v = res + v;
  float* dst = a.y + mi * a.ldy + n;
  if (a.fin_counter)
    publish_f32(dst, v);
  else
    *dst = v;
}

// Last block: final RMSNorm of the m produced rows (read back coherently) and the offset advance.
__device__ __forceinline__ void fin_epilogue(const GemvArgs& a, int m, float* s_red) {
  if (!last_block_done(a.fin_counter, gridDim.x)) return;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int adv = (threadIdx.x == 0 && a.adv_dst) ? *a.adv_src : 0;  // issued early, used last
  if (a.fin_gain) {
    constexpr int kPer = 16;  // rows up to 16 * 256 = 4096 wide are held in registers
    for (int mi = 0; mi < m; ++mi) {
      const float* yr = a.y + mi * a.ldy;
      float ss = 0.f;
      float v[kPer];
      const bool small = a.N <= kPer * kGemvThreads;
      uint32_t gw[kPer];
      if (small) {
        // all loads issued back to back from clamped addresses (the gains with
        // them, pinned so that none waits inside the store branch), masked after
#pragma unroll
        for (int j = 0; j < kPer; ++j) v[j] = fetch_f32(yr + min(static_cast<int>(threadIdx.x) + j * kGemvThreads, a.N - 1));
#pragma unroll
        for (int j = 0; j < kPer; ++j) gw[j] = a.fin_gain[min(static_cast<int>(threadIdx.x) + j * kGemvThreads, a.N - 1)];
#pragma unroll
        for (int j = 0; j < kPer; ++j) pin(gw[j]);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          if (static_cast<int>(threadIdx.x) + j * kGemvThreads >= a.N) v[j] = 0.f;
          ss = fmaf(v[j], v[j], ss);
        }
      } else {
        for (int k = threadIdx.x; k < a.N; k += kGemvThreads) {
          const float x = fetch_f32(yr + k);
          ss = fmaf(x, x, ss);
        }
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) s_red[wave] = ss;
      __syncthreads();
      float t = 0.f;
      for (int w = 0; w < kGemvWaves; ++w) t += s_red[w];
      const float inv = 1.f / sqrtf(t / static_cast<float>(a.N) + a.eps);
      if (small) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int k = threadIdx.x + j * kGemvThreads;
          if (k < a.N) a.fin_out[mi * a.ld_fin + k] = v[j] * inv * bf16_to_float(static_cast<uint16_t>(gw[j]));
        }
      } else {
        for (int k = threadIdx.x; k < a.N; k += kGemvThreads)
          a.fin_out[mi * a.ld_fin + k] = fetch_f32(yr + k) * inv * bf16_to_float(a.fin_gain[k]);
      }
      __syncthreads();
    }
  }
  if (threadIdx.x == 0 && a.adv_dst) *a.adv_dst = adv + a.adv_add + m;
}

// Draft-head value of row n for input row mi (optional logits store, Gumbel noise).
__device__ __forceinline__ unsigned long long head_key(const GemvArgs& a, int mi, int n, float z) {
  if (a.y) a.y[mi * a.ldy + n] = z;
  if (a.use_gumbel) {
    // Gumbel-max draw: argmax z/T - log(-log u) is a draw from softmax(z/T)
    // (python/woodcock/sampling.py:196-203 with one uniform per head row)
    const double u = philox_uniform(a.gumbel.seed, static_cast<unsigned long long>(*a.gumbel.round_dev),
                                    a.gumbel.purpose + mi, static_cast<unsigned long long>(n));
    z = static_cast<float>(static_cast<double>(z) * a.gumbel.inv_temperature - log(-log(u)));
  }
  return argmax_key(z, n);
}

// Block keys -> spread device atomics -> last block: winner row -> d2t token.
template <int MM>
__device__ __forceinline__ void argmax_epilogue(const GemvArgs& a, int m, unsigned long long (*s_key)[MM]) {
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < m) {
    unsigned long long best = 0;
    for (int w = 0; w < kGemvWaves; ++w) best = s_key[w][threadIdx.x] > best ? s_key[w][threadIdx.x] : best;
    if (best) atomic_max_u64(&a.slots[(threadIdx.x * kSlots + blockIdx.x % kSlots) * kSlotStride], best);
  }
  if (!a.counter) return;  // pending: the next launch resolves the slots
  if (!last_block_done(a.counter, gridDim.x)) return;
  // thread (row, slot): every slot read in parallel, then a max over the 32
  // lanes of the row's slots (kSlots == 32 lanes, half a wave)
  static_assert(kSlots == 32, "one half-wave per row");
  const int j = threadIdx.x % kSlots;
  for (int mi = threadIdx.x / kSlots; mi < m; mi += static_cast<int>(blockDim.x) / kSlots) {
    unsigned long long* sl = &a.slots[(mi * kSlots + j) * kSlotStride];
    unsigned long long best = atomic_load_u64(sl);
    atomic_store_u64(sl, 0ull);
#pragma unroll
    for (int o = kSlots / 2; o > 0; o >>= 1) {
      const unsigned long long other = __shfl_xor(best, o);
      best = other > best ? other : best;
    }
    if (j == 0) {
      const int row = argmax_key_index(best);
      a.tok_out[mi] = a.d2t ? a.d2t[row] : row;
      if (a.row_out) a.row_out[mi] = row;
    }
  }
}

// ------------------------------------------------------------------ M = 1

// Fast path for one input row when every segment's K is a multiple of 512.
// With norm gains (GB != 0): load order is x slices, then gains, then
// weights, so the norm (which needs only the L2-resident x) waits for nothing
// the weight stream is carrying, and the dot products retire the weight loads
// in the order they were issued; the norm scale is applied after the dot
// product (sum W (x g) * inv).  Without gains (GB == 0: o_proj, down): the
// weights are requested first, then the x slices are loaded and consumed step
// by step, so nothing but the weights stays live across the steps, which
// keeps the register count (and the number of waves streaming per SIMD) high.
// XB: bit s set = input segment s is bf16; GB: bit s set = segment s has a
// norm gain (RMSNorm applied).  S: max 512-wide steps per segment.
template <int R, bool PAIR, int NIN, int S, int XB, int GB>
__global__ __launch_bounds__(kGemvThreads) void k_gemv1(GemvArgs a) {
  constexpr int P = PAIR ? 2 : 1;
  __shared__ float s_red[kGemvWaves];
  __shared__ unsigned long long s_key[kGemvWaves][1];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int m = a.m_dev ? min(max(*a.m_dev, 0), 1) : 1;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
  const int rrow = res_row(a, 0);

  float acc[R][P];
  float resv[R];
  if constexpr (GB != 0) {
    // Every load below is unconditional (addresses clamped into the operands), so
    // the compiler issues them back to back with no branch or merge between them;
    // out-of-range steps are zeroed in the x slices, and out-of-range rows are
    // never stored.
    // 1. x slices, kept raw until the weights are in flight; a segment whose row
    // is a pending head argmax is resolved now and loaded after the weights, so
    // its chain (keys -> d2t -> row) holds back no weight load
    uint4 xq[NIN][S][2];
    int steps[NIN];
    int64_t xrow[NIN];
    auto load_x = [&](int s) {
      const InSeg& seg = a.in[s];
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int k = min(u, steps[s] - 1) * kWave * 8 + lane * 8;
        if (XB & (1 << s)) {
          xq[s][u][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(seg.x) + xrow[s] * seg.ld + k);
        } else {
          const float* xp = static_cast<const float*>(seg.x) + xrow[s] * seg.ld + k;
          xq[s][u][0] = *reinterpret_cast<const uint4*>(xp);
          xq[s][u][1] = *reinterpret_cast<const uint4*>(xp + 4);
        }
      }
    };
    // the pending keys first (one wave-wide load), reduced after the weights are requested
    unsigned long long pkey = 0;
#pragma unroll
    for (int s = 0; s < NIN; ++s)
      if (a.in[s].pend_slots) pkey = pend_key(a.in[s].pend_slots);
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      steps[s] = a.in[s].K / (kWave * 8);
      if (!a.in[s].pend_slots) {
        xrow[s] = m > 0 ? in_row(a.in[s], 0) : 0;
        load_x(s);
      }
    }
    // 2. gains
    uint4 gr[NIN][S];
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      if (!((GB >> s) & 1)) continue;
      const uint16_t* gp = a.in[s].gain;
#pragma unroll
      for (int u = 0; u < S; ++u)
        gr[s][u] = *reinterpret_cast<const uint4*>(gp + min(u, steps[s] - 1) * kWave * 8 + lane * 8);
    }
    // 3. weights of this wave's rows
    uint4 w[NIN][R][P][S];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(row0 + r, a.N - 1);
#pragma unroll
      for (int p = 0; p < P; ++p) {
#pragma unroll
        for (int s = 0; s < NIN; ++s) {
          const uint16_t* wr = row_ptr<PAIR>(a, n, p, s) + lane * 8;
#pragma unroll
          for (int u = 0; u < S; ++u)
            w[s][r][p][u] = *reinterpret_cast<const uint4*>(wr + min(u, steps[s] - 1) * kWave * 8);
        }
      }
    }
    int pend_hr = 0;  // head row of the pending segment
#pragma unroll
    for (int s = 0; s < NIN; ++s)
      if (a.in[s].pend_slots) {
        pend_hr = pend_reduce(pkey);
        xrow[s] = m > 0 ? pend_token(a.in[s], pend_hr) : 0;
        load_x(s);
      }
#pragma unroll
    for (int r = 0; r < R; ++r) resv[r] = res_at(a, rrow, min(row0 + r, a.N - 1));
    if (a.pend_tok_out && blockIdx.x == 0 && threadIdx.x == 0) {
#pragma unroll
      for (int s = 0; s < NIN; ++s) {
        if (!a.in[s].pend_slots) continue;
        a.pend_tok_out[0] = a.in[s].pend_d2t ? a.in[s].pend_d2t[pend_hr] : pend_hr;
        if (a.pend_row_out) a.pend_row_out[0] = pend_hr;
      }
    }
    // 4. per-segment 1/rms and x * gain (waits only for x and gain)
    float4 xr[NIN][S][2];
    float inv[NIN];
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      const bool gain = (GB >> s) & 1;
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        float4 x0, x1;
        if (XB & (1 << s)) {
          const uint4 h = xq[s][u][0];
          x0 = make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
          x1 = make_float4(bf16_lo(h.z), bf16_hi(h.z), bf16_lo(h.w), bf16_hi(h.w));
        } else {
          x0 = make_float4(__uint_as_float(xq[s][u][0].x), __uint_as_float(xq[s][u][0].y),
                           __uint_as_float(xq[s][u][0].z), __uint_as_float(xq[s][u][0].w));
          x1 = make_float4(__uint_as_float(xq[s][u][1].x), __uint_as_float(xq[s][u][1].y),
                           __uint_as_float(xq[s][u][1].z), __uint_as_float(xq[s][u][1].w));
        }
        if (u >= steps[s]) x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);
        ss = fmaf(x0.x, x0.x, ss); ss = fmaf(x0.y, x0.y, ss); ss = fmaf(x0.z, x0.z, ss); ss = fmaf(x0.w, x0.w, ss);
        ss = fmaf(x1.x, x1.x, ss); ss = fmaf(x1.y, x1.y, ss); ss = fmaf(x1.z, x1.z, ss); ss = fmaf(x1.w, x1.w, ss);
        if (gain) {
          const uint4 g = gr[s][u];
          x0 = make_float4(x0.x * bf16_lo(g.x), x0.y * bf16_hi(g.x), x0.z * bf16_lo(g.y), x0.w * bf16_hi(g.y));
          x1 = make_float4(x1.x * bf16_lo(g.z), x1.y * bf16_hi(g.z), x1.z * bf16_lo(g.w), x1.w * bf16_hi(g.w));
        }
        xr[s][u][0] = x0;
        xr[s][u][1] = x1;
      }
      inv[s] = gain ? 1.f / sqrtf(wave_sum_dpp(ss) / static_cast<float>(a.in[s].K) + a.eps) : 1.f;
    }
    if (a.xn_out && blockIdx.x == 0 && wave == 0 && m > 0) {
      float* xo = a.xn_out + static_cast<int64_t>(in_row(a.in[0], 0)) * a.ld_xn + lane * 8;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        if (u >= steps[0]) continue;
        const float4 x0 = xr[0][u][0], x1 = xr[0][u][1];
        *reinterpret_cast<float4*>(xo + u * kWave * 8) =
            make_float4(x0.x * inv[0], x0.y * inv[0], x0.z * inv[0], x0.w * inv[0]);
        *reinterpret_cast<float4*>(xo + u * kWave * 8 + 4) =
            make_float4(x1.x * inv[0], x1.y * inv[0], x1.z * inv[0], x1.w * inv[0]);
      }
    }
    // 5. dot products in weight-issue order
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float t = 0.f;
#pragma unroll
        for (int s = 0; s < NIN; ++s) {
          float part = 0.f;
#pragma unroll
          for (int u = 0; u < S; ++u) part += dot8(w[s][r][p][u], xr[s][u][0], xr[s][u][1]);
          t = fmaf(part, inv[s], t);
        }
        acc[r][p] = wave_sum_dpp(t);
      }

  } else {
    // Every load below is unconditional (addresses clamped into the operands), so
    // the compiler issues them with no branch or merge between them; out-of-range
    // steps are zeroed in the x slices, and out-of-range rows are never stored.
    int steps[NIN];
    int64_t xrow[NIN];
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      steps[s] = a.in[s].K / (kWave * 8);
      xrow[s] = m > 0 ? in_row(a.in[s], 0) : 0;
    }
    // 1. weights of this wave's rows
    uint4 w[NIN][R][P][S];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(row0 + r, a.N - 1);
#pragma unroll
      for (int p = 0; p < P; ++p) {
#pragma unroll
        for (int s = 0; s < NIN; ++s) {
          const uint16_t* wr = row_ptr<PAIR>(a, n, p, s) + lane * 8;
#pragma unroll
          for (int u = 0; u < S; ++u)
            w[s][r][p][u] = *reinterpret_cast<const uint4*>(wr + min(u, steps[s] - 1) * kWave * 8);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) resv[r] = res_at(a, rrow, min(row0 + r, a.N - 1));

    // 2. per step: x slice and gains -> sum of squares, x * gain -> dot products
    float part[NIN][R][P], ssq[NIN];
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      const InSeg& seg = a.in[s];
      const bool gain = (GB >> s) & 1;
      float ss = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) part[s][r][p] = 0.f;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        const int k = min(u, steps[s] - 1) * kWave * 8 + lane * 8;
        float4 x0, x1;
        if (XB & (1 << s)) {
          const uint4 h = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(seg.x) + xrow[s] * seg.ld + k);
          x0 = make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
          x1 = make_float4(bf16_lo(h.z), bf16_hi(h.z), bf16_lo(h.w), bf16_hi(h.w));
        } else {
          const float* xp = static_cast<const float*>(seg.x) + xrow[s] * seg.ld + k;
          x0 = *reinterpret_cast<const float4*>(xp);
          x1 = *reinterpret_cast<const float4*>(xp + 4);
        }
        const bool live = u < steps[s];  // selects, not a branch: the loads stay schedulable
        x0 = make_float4(live ? x0.x : 0.f, live ? x0.y : 0.f, live ? x0.z : 0.f, live ? x0.w : 0.f);
        x1 = make_float4(live ? x1.x : 0.f, live ? x1.y : 0.f, live ? x1.z : 0.f, live ? x1.w : 0.f);
        ss = fmaf(x0.x, x0.x, ss); ss = fmaf(x0.y, x0.y, ss); ss = fmaf(x0.z, x0.z, ss); ss = fmaf(x0.w, x0.w, ss);
        ss = fmaf(x1.x, x1.x, ss); ss = fmaf(x1.y, x1.y, ss); ss = fmaf(x1.z, x1.z, ss); ss = fmaf(x1.w, x1.w, ss);
        if (gain) {
          const uint4 g = *reinterpret_cast<const uint4*>(seg.gain + k);
          x0 = make_float4(x0.x * bf16_lo(g.x), x0.y * bf16_hi(g.x), x0.z * bf16_lo(g.y), x0.w * bf16_hi(g.y));
          x1 = make_float4(x1.x * bf16_lo(g.z), x1.y * bf16_hi(g.z), x1.z * bf16_lo(g.w), x1.w * bf16_hi(g.w));
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int p = 0; p < P; ++p) part[s][r][p] = dot8_acc(w[s][r][p][u], x0, x1, part[s][r][p]);
      }
      ssq[s] = ss;
    }
    // 3. per-segment 1/rms, then the row sums
    float inv[NIN];
#pragma unroll
    for (int s = 0; s < NIN; ++s)
      inv[s] = ((GB >> s) & 1) ? 1.f / sqrtf(wave_sum_dpp(ssq[s]) / static_cast<float>(a.in[s].K) + a.eps) : 1.f;
    if (a.xn_out && blockIdx.x == 0 && wave == 0 && m > 0) {
      // the normalised input row (segment 0) for the caller: x * gain * inv
      const InSeg& seg = a.in[0];
      float* xo = a.xn_out + static_cast<int64_t>(xrow[0]) * a.ld_xn + lane * 8;
#pragma unroll
      for (int u = 0; u < S; ++u) {
        if (u >= steps[0]) continue;
        const int k = u * kWave * 8 + lane * 8;
        float4 x0, x1;
        if (XB & 1) {
          const uint4 h = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(seg.x) + xrow[0] * seg.ld + k);
          x0 = make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
          x1 = make_float4(bf16_lo(h.z), bf16_hi(h.z), bf16_lo(h.w), bf16_hi(h.w));
        } else {
          const float* xp = static_cast<const float*>(seg.x) + xrow[0] * seg.ld + k;
          x0 = *reinterpret_cast<const float4*>(xp);
          x1 = *reinterpret_cast<const float4*>(xp + 4);
        }
        if (GB & 1) {
          const uint4 g = *reinterpret_cast<const uint4*>(seg.gain + k);
          x0 = make_float4(x0.x * bf16_lo(g.x), x0.y * bf16_hi(g.x), x0.z * bf16_lo(g.y), x0.w * bf16_hi(g.y));
          x1 = make_float4(x1.x * bf16_lo(g.z), x1.y * bf16_hi(g.z), x1.z * bf16_lo(g.w), x1.w * bf16_hi(g.w));
        }
        *reinterpret_cast<float4*>(xo + u * kWave * 8) =
            make_float4(x0.x * inv[0], x0.y * inv[0], x0.z * inv[0], x0.w * inv[0]);
        *reinterpret_cast<float4*>(xo + u * kWave * 8 + 4) =
            make_float4(x1.x * inv[0], x1.y * inv[0], x1.z * inv[0], x1.w * inv[0]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        float t = 0.f;
#pragma unroll
        for (int s = 0; s < NIN; ++s) t = fmaf(part[s][r][p], inv[s], t);
        acc[r][p] = wave_sum_dpp(t);
      }

  }
  // 6. epilogues
  if (a.epi != kEpiArgmax) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < a.N && m > 0) store_out<PAIR>(a, 0, row0 + r, acc[r][0], acc[r][P - 1], resv[r]);
    }
    if (a.fin_counter) fin_epilogue(a, m, s_red);
    return;
  }
  if (lane == 0) {
    unsigned long long best = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r >= a.N || m == 0) continue;
      const unsigned long long key = head_key(a, 0, row0 + r, acc[r][0]);
      best = key > best ? key : best;
    }
    s_key[wave][0] = best;
  }
  argmax_epilogue<1>(a, m, s_key);
}

// ------------------------------------------------------------------ 2..MM rows, x staged in LDS

// Few input rows (M <= MM) with every segment's K a multiple of 512.
//   1. the wave's weight rows are requested first (all of them);
//   2. fp32 x rows are copied HBM/L2 -> LDS by direct-to-LDS loads, bf16 rows
//      (the embedding gather) and the gains go to registers;
//   3. after the barrier (weights and copies in), the block writes x * gain
//      as fp32 into LDS once and reduces the per-row sums of squares;
//   4. each wave runs its weights against x from LDS, widening each weight
//      vector from bf16 once for all rows.
// Row addressing uses the host row count M, so nothing waits on the device
// count m before the loads are issued; m only masks compute and stores.
// LDS: fp32 [NIN][M][S * 512] (x * gain).
template <int R, bool PAIR, int NIN, int S, int XB, int MM>
__global__ __launch_bounds__(kGemvThreads) void k_gemvx(GemvArgs a) {
  constexpr int P = PAIR ? 2 : 1;
  constexpr int C = S / 4;  // 2048-element chunks of a row: thread t owns elements c*2048 + t*8 .. +8
  static_assert(S % 4 == 0, "steps in multiples of 4");
  extern __shared__ __attribute__((aligned(16))) float smem[];  // 16-byte aligned: b128 LDS accesses and LDS DMA
  __shared__ float s_red[kGemvWaves];
  __shared__ float s_ss[kGemvWaves][NIN * MM];
  __shared__ unsigned long long s_key[kGemvWaves][MM];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int m = a.m_dev ? min(max(*a.m_dev, 0), a.M) : a.M;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
  const int row_len = S * 512;  // LDS row stride (floats)

  int steps[NIN];
#pragma unroll
  for (int s = 0; s < NIN; ++s) steps[s] = a.in[s].K / (kWave * 8);

  // 0. gathered row indices (before anything that would wait on them one by one)
  int xrow_idx[NIN][MM];
#pragma unroll
  for (int s = 0; s < NIN; ++s)
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) xrow_idx[s][mi] = in_row(a.in[s], min(mi, a.M - 1));
  int rrow[MM];
#pragma unroll
  for (int mi = 0; mi < MM; ++mi) rrow[mi] = res_row(a, min(mi, a.M - 1));

  // 1. the wave's weight rows first: the stream starts at once
  uint4 w[NIN][R][P][S];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(row0 + r, a.N - 1);
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int s = 0; s < NIN; ++s) {
        const uint16_t* wr = row_ptr<PAIR>(a, n, p, s) + lane * 8;
#pragma unroll
        for (int u = 0; u < S; ++u)
          w[s][r][p][u] = *reinterpret_cast<const uint4*>(wr + min(u, steps[s] - 1) * kWave * 8);
      }
  }

  // 2a. fp32 rows -> LDS in 1 KB pieces (one wave-wide 16-byte load each); wave w
  //     issues pieces w, w+4, ... of every row.  Branch-free: every one of the
  //     M rows is copied (rows past the device row count are never used).
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    if ((XB >> s) & 1) continue;
    const InSeg& seg = a.in[s];
    constexpr int kPieces = S * 512 * 4 / 1024;
    static_assert(kPieces % kGemvWaves == 0, "pieces per row split evenly over the waves");
    const int row_bytes = seg.K * 4;
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      if (mi >= a.M) continue;
      const int slot = mi;
      const char* xrow = static_cast<const char*>(seg.x) + static_cast<int64_t>(xrow_idx[s][mi]) * seg.ld * 4;
#pragma unroll
      for (int k = 0; k < kPieces / kGemvWaves; ++k) {
        const int pc = k * kGemvWaves + wave;
        const int gb = min(pc * 1024, row_bytes - 1024) + lane * 16;  // clamped into the row
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(xrow + gb),
                                         smem + (s * a.M + slot) * row_len + pc * 256, 16, 0, 0);
      }
    }
  }
  // 2b. bf16 rows -> registers (8 elements per thread and chunk), gains of the
  //     thread's elements
  uint4 xb[NIN][MM][C];
  uint4 gq[NIN][C];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    const InSeg& seg = a.in[s];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int e = min(c * 2048 + static_cast<int>(threadIdx.x) * 8, seg.K - 8);
      const uint16_t* gp = seg.gain ? seg.gain : a.w[0][s];
      gq[s][c] = *reinterpret_cast<const uint4*>(gp + e);
      if ((XB >> s) & 1) {
#pragma unroll
        for (int mi = 0; mi < MM; ++mi)
          xb[s][mi][c] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(seg.x) +
                                                         static_cast<int64_t>(xrow_idx[s][mi]) * seg.ld + e);
      }
    }
  }
  float resv[R][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) resv[r][mi] = res_at(a, rrow[mi], min(row0 + r, a.N - 1));

  // the copies land before the barrier (the compiler waits for every load here,
  // the weights included: they were requested first and arrive with the copies)
  __syncthreads();

  // 3. x * gain into LDS (fp32, in place for fp32 rows) and per-row sums of squares
  float ss[NIN][MM];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    const bool bf = (XB >> s) & 1;
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      ss[s][mi] = 0.f;
      if (mi >= m) continue;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int e = c * 2048 + static_cast<int>(threadIdx.x) * 8;
        if (e >= a.in[s].K) continue;
        float* xp = smem + (s * a.M + mi) * row_len + e;
        float x[8];
        if (bf) {
          const uint4 h = xb[s][mi][c];
          x[0] = bf16_lo(h.x); x[1] = bf16_hi(h.x); x[2] = bf16_lo(h.y); x[3] = bf16_hi(h.y);
          x[4] = bf16_lo(h.z); x[5] = bf16_hi(h.z); x[6] = bf16_lo(h.w); x[7] = bf16_hi(h.w);
        } else {
          const float4 v0 = *reinterpret_cast<const float4*>(xp), v1 = *reinterpret_cast<const float4*>(xp + 4);
          x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w; x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
        }
        float t = ss[s][mi];
#pragma unroll
        for (int j = 0; j < 8; ++j) t = fmaf(x[j], x[j], t);
        ss[s][mi] = t;
        if (a.in[s].gain) {
          const uint4 g = gq[s][c];
          x[0] *= bf16_lo(g.x); x[1] *= bf16_hi(g.x); x[2] *= bf16_lo(g.y); x[3] *= bf16_hi(g.y);
          x[4] *= bf16_lo(g.z); x[5] *= bf16_hi(g.z); x[6] *= bf16_lo(g.w); x[7] *= bf16_hi(g.w);
        }
        *reinterpret_cast<float4*>(xp) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(xp + 4) = make_float4(x[4], x[5], x[6], x[7]);
      }
    }
  }
#pragma unroll
  for (int s = 0; s < NIN; ++s)
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      const float t = wave_sum_dpp(ss[s][mi]);
      if (lane == 0) s_ss[wave][s * MM + mi] = t;
    }
  lds_barrier();
  float inv[NIN][MM];
#pragma unroll
  for (int s = 0; s < NIN; ++s)
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < kGemvWaves; ++q) t += s_ss[q][s * MM + mi];
      inv[s][mi] = a.in[s].gain ? 1.f / sqrtf(t / static_cast<float>(a.in[s].K) + a.eps) : 1.f;
    }

  // 4. dot products: each weight vector widened once, then used for every row
  float acc[R][P][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = 0.f;
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    float part[R][P][MM];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int mi = 0; mi < MM; ++mi) part[r][p][mi] = 0.f;
#pragma unroll
    for (int u = 0; u < S; ++u) {
      if (u >= steps[s]) continue;
      float wf[R][P][8];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const uint4 q = w[s][r][p][u];
          wf[r][p][0] = bf16_lo(q.x); wf[r][p][1] = bf16_hi(q.x); wf[r][p][2] = bf16_lo(q.y);
          wf[r][p][3] = bf16_hi(q.y); wf[r][p][4] = bf16_lo(q.z); wf[r][p][5] = bf16_hi(q.z);
          wf[r][p][6] = bf16_lo(q.w); wf[r][p][7] = bf16_hi(q.w);
        }
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) {
        if (mi >= m) continue;
        const float* xp = smem + (s * a.M + mi) * row_len + u * 512 + lane * 8;
        const float4 x0 = *reinterpret_cast<const float4*>(xp), x1 = *reinterpret_cast<const float4*>(xp + 4);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int p = 0; p < P; ++p) {
            float t = part[r][p][mi];
            t = fmaf(wf[r][p][0], x0.x, t); t = fmaf(wf[r][p][1], x0.y, t);
            t = fmaf(wf[r][p][2], x0.z, t); t = fmaf(wf[r][p][3], x0.w, t);
            t = fmaf(wf[r][p][4], x1.x, t); t = fmaf(wf[r][p][5], x1.y, t);
            t = fmaf(wf[r][p][6], x1.z, t); t = fmaf(wf[r][p][7], x1.w, t);
            part[r][p][mi] = t;
          }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = fmaf(part[r][p][mi], inv[s][mi], acc[r][p][mi]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = wave_sum_dpp(acc[r][p][mi]);

  // 5. epilogues
  if (a.epi != kEpiArgmax) {
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (row0 + r >= a.N) continue;
#pragma unroll
        for (int mi = 0; mi < MM; ++mi)
          if (mi < m) store_out<PAIR>(a, mi, row0 + r, acc[r][0][mi], acc[r][P - 1][mi], resv[r][mi]);
      }
    }
    if (a.fin_counter) fin_epilogue(a, m, s_red);
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      unsigned long long best = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (row0 + r >= a.N || mi >= m) continue;
        const unsigned long long key = head_key(a, mi, row0 + r, acc[r][0][mi]);
        best = key > best ? key : best;
      }
      s_key[wave][mi] = best;
    }
  }
  argmax_epilogue<MM>(a, m, s_key);
}

// ------------------------------------------------------------------ M > 1

// Four consecutive inputs of segment s, row `row`, from k (k % 4 == 0).
__device__ __forceinline__ float4 load4(const InSeg& s, int64_t row, int k) {
  if (s.dtype == WC_BF16) {
    const uint2 h = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(s.x) + row * s.ld + k);
    return make_float4(bf16_lo(h.x), bf16_hi(h.x), bf16_lo(h.y), bf16_hi(h.y));
  }
  return *reinterpret_cast<const float4*>(static_cast<const float*>(s.x) + row * s.ld + k);
}

template <int R, int MM, bool PAIR, int U>
__global__ __launch_bounds__(kGemvThreads) void k_gemvm(GemvArgs a) {
  constexpr int P = PAIR ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) float smem[];  // 16-byte aligned: b128 LDS accesses and LDS DMA
  __shared__ float s_red[kGemvWaves];
  __shared__ float s_ss[kGemvWaves][MM];
  __shared__ unsigned long long s_key[kGemvWaves][MM];

  int m = a.M;
  if (a.m_dev) m = min(max(*a.m_dev, 0), a.M);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;

  int rseg[R][P], roff[R][P];
  bool valid[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    valid[r] = row0 + r < a.N;
#pragma unroll
    for (int p = 0; p < P; ++p) row_segment<PAIR>(a, row0 + r, p, rseg[r][p], roff[r][p]);
  }

  int kcap = a.lds_floats / (m > 0 ? m : 1);
  kcap = kcap / 512 * 512;
  if (kcap < 512) kcap = 512;

  // the first weight group of segment 0 is requested before any staging
  uint4 w[R][P][U];
  {
    const int kc0 = min(kcap, a.in[0].K);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = lane * 8 + u * kWave * 8;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p)
          w[r][p][u] = (valid[r] && kk < kc0)
                           ? *reinterpret_cast<const uint4*>(a.w[rseg[r][p]][0] +
                                                             static_cast<int64_t>(roff[r][p]) * a.ldw[0] + kk)
                           : make_uint4(0, 0, 0, 0);
    }
  }

  float acc[R][P][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) acc[r][p][mi] = 0.f;

  bool prefetched = true;
  for (int s = 0; s < a.n_in; ++s) {
    const InSeg seg = a.in[s];
    const uint16_t* wrow[R][P];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p)
        wrow[r][p] = valid[r] ? a.w[rseg[r][p]][s] + static_cast<int64_t>(roff[r][p]) * a.ldw[s] : nullptr;
    float part[R][P][MM], ssp[MM];
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      ssp[mi] = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) part[r][p][mi] = 0.f;
    }
    for (int c0 = 0; c0 < seg.K; c0 += kcap) {
      const int kc = min(kcap, seg.K - c0);
      __syncthreads();  // previous chunk fully consumed
      // stage x * gain (the norm scale is applied after the dot product) and
      // accumulate the sums of squares in the same pass
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) {
        if (mi < m) {
          const int64_t row = in_row(seg, mi);
          for (int k = threadIdx.x * 4; k < kc; k += kGemvThreads * 4) {
            float4 v = load4(seg, row, c0 + k);
            if (seg.gain) {
              ssp[mi] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ssp[mi]))));
              const uint2 g = *reinterpret_cast<const uint2*>(seg.gain + c0 + k);
              v.x *= bf16_lo(g.x);
              v.y *= bf16_hi(g.x);
              v.z *= bf16_lo(g.y);
              v.w *= bf16_hi(g.y);
            }
            *reinterpret_cast<float4*>(smem + mi * kc + k) = v;
          }
        }
      }
      __syncthreads();
      for (int k = lane * 8; k < kc; k += kWave * 8 * U) {
        if (!prefetched) {
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
        }
        prefetched = false;
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
                  for (int p = 0; p < P; ++p) part[r][p][mi] += dot8(w[r][p][u], x0, x1);
              }
            }
          }
        }
      }
    }
    // per-row 1/rms of this segment (block reduction), applied to the partial sums
    if (seg.gain) {
#pragma unroll
      for (int mi = 0; mi < MM; ++mi) {
        const float t = wave_sum(ssp[mi]);
        if (lane == 0) s_ss[wave][mi] = t;
      }
      __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      float inv = 1.f;
      if (seg.gain) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < kGemvWaves; ++q) t += s_ss[q][mi];
        inv = 1.f / sqrtf(t / static_cast<float>(seg.K) + a.eps);
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) acc[r][p][mi] = fmaf(part[r][p][mi], inv, acc[r][p][mi]);
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
#pragma unroll
        for (int mi = 0; mi < MM; ++mi)
          if (mi < m) store_out<PAIR>(a, mi, row0 + r, acc[r][0][mi], acc[r][P - 1][mi], res_value(a, mi, row0 + r));
      }
    }
    if (a.fin_counter) fin_epilogue(a, m, s_red);
    return;
  }
  if (lane == 0) {
#pragma unroll
    for (int mi = 0; mi < MM; ++mi) {
      unsigned long long best = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (!valid[r] || mi >= m) continue;
        const unsigned long long key = head_key(a, mi, row0 + r, acc[r][0][mi]);
        best = key > best ? key : best;
      }
      s_key[wave][mi] = best;
    }
  }
  argmax_epilogue<MM>(a, m, s_key);
}

}  // namespace wc
