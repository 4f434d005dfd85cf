// gemv1s.h -- one-row streaming GEMV with the input row staged once per block.
//
// The same computation and epilogues as k_gemv1 (gemv.h), with one change in
// where each wave gets x * gain: k_gemv1 has every wave load the x slices and
// gains it needs from L2 (for a K-wide row that is 4K bytes of x and 2K of
// gain per wave, 1.5 to 3 times the wave's own weight bytes), while here the
// block's threads load x and the gains once -- 8 elements per thread per 2048,
// issued before any weight so that waiting for them waits for nothing the
// weight stream carries -- and write x * gain to LDS with the row's sum of
// squares; after an LDS-only barrier each wave reads its 8 elements per step
// from LDS.  The L2-to-CU traffic per block drops from 4 x (x + gain) to
// 1 x (x + gain), and the wave keeps no x registers across the weight wait.
// It pays where x dominates a wave's loads: a gain-free 6144-wide row (the
// down projection, 24 KB of fp32 x against 12 KB of weights per wave), and
// where the per-wave registers cap the resident waves: normed rows wider than
// 2048 (at 2560 one segment keeps 73-82 VGPRs against 116, the dual-stream
// QKV 146 against 210, so its 6144-row launch is resident at once) and the
// 2048-wide draft head (73 against 94, six waves per SIMD instead of five).
// With several segments, a segment whose row is a pending head argmax has its
// keys loaded first and its row staged only after the weights are requested.
// Other 2048-wide rows keep the per-wave loads of k_gemv1 (measured as fast).
#pragma once
#include "gemv.h"

namespace wc {

template <int R, bool PAIR, int NIN, int S, int XB, int GB>
__global__ __launch_bounds__(kGemvThreads) void k_gemv1s(GemvArgs a) {
  constexpr int P = PAIR ? 2 : 1;
  constexpr int C = (S * kWave * 8 + kGemvThreads * 8 - 1) / (kGemvThreads * 8);  // staged chunks per thread
  extern __shared__ __attribute__((aligned(16))) float g_xs[];  // [segment][K_s] x * gain
  __shared__ float s_ss[NIN][kGemvWaves];
  __shared__ float s_red[kGemvWaves];
  __shared__ unsigned long long s_key[kGemvWaves][1];
  const int t = threadIdx.x, lane = t % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int m = a.m_dev ? min(max(*a.m_dev, 0), 1) : 1;
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
  const int rrow = res_row(a, 0);

  // 0. with several input segments (the dual-stream QKV), the keys of a
  // pending head argmax (one wave-wide load) first of all: they are reduced
  // only after the weights are requested, so the chain keys -> d2t -> row holds
  // back no weight load (one segment: in_row resolves it up front)
  constexpr bool kPend = NIN > 1;
  unsigned long long pkey = 0;
  if constexpr (kPend) {
#pragma unroll
    for (int s = 0; s < NIN; ++s)
      if (a.in[s].pend_slots) pkey = pend_key(a.in[s].pend_slots);
  }
  int steps[NIN], soff[NIN];
  int64_t xrow[NIN];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    steps[s] = a.in[s].K / (kWave * 8);
    soff[s] = s == 0 ? 0 : soff[s - 1] + a.in[s - 1].K;
    xrow[s] = m > 0 && !(kPend && a.in[s].pend_slots) ? in_row(a.in[s], 0) : 0;
  }

  // 1. the block's share of x and the gains (clamped addresses, unconditional);
  // a pending segment's row after the weights
  uint4 sx[NIN][C][2], sg[NIN][C];
  auto stage_x = [&](int s, int c, int k) {
    const InSeg& seg = a.in[s];
    if ((XB >> s) & 1) {
      sx[s][c][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(seg.x) + xrow[s] * seg.ld + k);
    } else {
      const float* xp = static_cast<const float*>(seg.x) + xrow[s] * seg.ld + k;
      sx[s][c][0] = *reinterpret_cast<const uint4*>(xp);
      sx[s][c][1] = *reinterpret_cast<const uint4*>(xp + 4);
    }
  };
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    const InSeg& seg = a.in[s];
    const bool defer = kPend && seg.pend_slots;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int k = min(c * kGemvThreads * 8 + t * 8, seg.K - 8);
      if (!defer) stage_x(s, c, k);
      if ((GB >> s) & 1) sg[s][c] = *reinterpret_cast<const uint4*>(seg.gain + k);
    }
  }
  // 2. weights of this wave's rows, then its residual values
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
  float resv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) resv[r] = res_at(a, rrow, min(row0 + r, a.N - 1));
  // 2b. the pending segment's row: its token from the keys, then the row's share
  if constexpr (kPend) {
#pragma unroll
    for (int s = 0; s < NIN; ++s) {
      if (!a.in[s].pend_slots) continue;
      const int hr = pend_reduce(pkey);
      xrow[s] = m > 0 ? pend_token(a.in[s], hr) : 0;
#pragma unroll
      for (int c = 0; c < C; ++c) stage_x(s, c, min(c * kGemvThreads * 8 + t * 8, a.in[s].K - 8));
      if (a.pend_tok_out && blockIdx.x == 0 && t == 0) {
        a.pend_tok_out[0] = a.in[s].pend_d2t ? a.in[s].pend_d2t[hr] : hr;
        if (a.pend_row_out) a.pend_row_out[0] = hr;
      }
    }
  }

  // 3. x * gain -> LDS, sums of squares -> LDS (waits only for the staging loads)
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
    const InSeg& seg = a.in[s];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int k = c * kGemvThreads * 8 + t * 8;
      float x[8];
      if ((XB >> s) & 1) {
        const uint4 h = sx[s][c][0];
        x[0] = bf16_lo(h.x); x[1] = bf16_hi(h.x); x[2] = bf16_lo(h.y); x[3] = bf16_hi(h.y);
        x[4] = bf16_lo(h.z); x[5] = bf16_hi(h.z); x[6] = bf16_lo(h.w); x[7] = bf16_hi(h.w);
      } else {
        x[0] = __uint_as_float(sx[s][c][0].x); x[1] = __uint_as_float(sx[s][c][0].y);
        x[2] = __uint_as_float(sx[s][c][0].z); x[3] = __uint_as_float(sx[s][c][0].w);
        x[4] = __uint_as_float(sx[s][c][1].x); x[5] = __uint_as_float(sx[s][c][1].y);
        x[6] = __uint_as_float(sx[s][c][1].z); x[7] = __uint_as_float(sx[s][c][1].w);
      }
      if (k < seg.K) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
        if ((GB >> s) & 1) {
          const uint4 g = sg[s][c];
          x[0] *= bf16_lo(g.x); x[1] *= bf16_hi(g.x); x[2] *= bf16_lo(g.y); x[3] *= bf16_hi(g.y);
          x[4] *= bf16_lo(g.z); x[5] *= bf16_hi(g.z); x[6] *= bf16_lo(g.w); x[7] *= bf16_hi(g.w);
        }
        float* dst = g_xs + soff[s] + k;
        *reinterpret_cast<float4*>(dst) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(x[4], x[5], x[6], x[7]);
      }
    }
    if ((GB >> s) & 1) {
      ss = wave_sum_dpp(ss);
      if (lane == 0) s_ss[s][wave] = ss;
    }
  }
  lds_barrier();
  float inv[NIN];
#pragma unroll
  for (int s = 0; s < NIN; ++s)
    inv[s] = ((GB >> s) & 1)
                 ? 1.f / sqrtf(((s_ss[s][0] + s_ss[s][1]) + (s_ss[s][2] + s_ss[s][3])) / static_cast<float>(a.in[s].K) +
                               a.eps)
                 : 1.f;

  // 4. dot products in weight-issue order, x * gain read from LDS per step
  float acc[R][P];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p) acc[r][p] = 0.f;
  float part[NIN][R][P];
#pragma unroll
  for (int s = 0; s < NIN; ++s) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) part[s][r][p] = 0.f;
#pragma unroll
    for (int u = 0; u < S; ++u) {
      if (u >= steps[s]) continue;  // wave-uniform: the weights are already in registers
      const float* xp = g_xs + soff[s] + u * kWave * 8 + lane * 8;
      const float4 x0 = *reinterpret_cast<const float4*>(xp), x1 = *reinterpret_cast<const float4*>(xp + 4);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) part[s][r][p] = dot8_acc(w[s][r][p][u], x0, x1, part[s][r][p]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p) {
      float tt = 0.f;
#pragma unroll
      for (int s = 0; s < NIN; ++s) tt = fmaf(part[s][r][p], inv[s], tt);
      acc[r][p] = wave_sum_dpp(tt);
    }
  if (a.xn_out && blockIdx.x == 0 && wave == 0 && m > 0) {
    // the normalised input row (segment 0) for the caller: x * gain * inv
    float* xo = a.xn_out + static_cast<int64_t>(xrow[0]) * a.ld_xn;
    for (int k = lane * 4; k < a.in[0].K; k += kWave * 4) {
      const float4 v = *reinterpret_cast<const float4*>(g_xs + k);
      *reinterpret_cast<float4*>(xo + k) = make_float4(v.x * inv[0], v.y * inv[0], v.z * inv[0], v.w * inv[0]);
    }
  }

  // 5. epilogues (as k_gemv1)
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

}  // namespace wc
